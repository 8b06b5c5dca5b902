"""The BASELINE configurations at full size on the GPU.

At full size the CPU oracle runs per (batch, head) slice: the forward is
independent per (batch, head), so the HIP output restricted to a few
(batch, head) pairs is compared with the oracle and the fp32 gold on those
pairs alone.  Size-independent properties cover the rest: determinism, the
resume invariant (split at a chunk boundary, bit-exact), finiteness.
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import kda_bt16_fwd
from kda_oracle import chunked_reference, make_inputs, recurrent_gold
from kda_testlib import assert_close_rel, maxdiff

pytestmark = pytest.mark.gpu

CONFIGS = {
    "c0_B2_T1024_H4": dict(B=2, T=1024, H=4),
    "c1_B2_T4096_H8": dict(B=2, T=4096, H=8, h0_std=0.05),
    "c2_B1_T8192_H32": dict(B=1, T=8192, H=32),
    "c3_B1_T8192_H96": dict(B=1, T=8192, H=96),
    "c4_B16_T2048_H32": dict(B=16, T=2048, H=32, h0_std=0.05, g_std=2.0),
}
LB = -5.0
SCALE = 128 ** -0.5


def _inputs(name):
    cfg = dict(CONFIGS[name])
    B, T, H = cfg.pop("B"), cfg.pop("T"), cfg.pop("H")
    return make_inputs(B, T, H, seed=42, **cfg)


def _fwd(c, dev, sl=slice(None), h0=None):
    args = [c[x][:, sl].contiguous().to(dev) for x in ("q", "k", "v", "g", "beta")]
    return kda_bt16_fwd(
        *args, scale=SCALE, initial_state=h0, output_final_state=True,
        use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True,
        lower_bound=LB, A_log=c["A_log"].to(dev), dt_bias=c["dt_bias"].to(dev),
    )


def _pair(c, b, h):
    """Inputs restricted to batch b, head h (as B=1, H=1)."""
    out = {x: c[x][b:b + 1, :, h:h + 1].contiguous() for x in ("q", "k", "v", "g", "beta")}
    out["A_log"] = c["A_log"][h:h + 1]
    out["dt_bias"] = c["dt_bias"][h * 128:(h + 1) * 128]
    out["h0"] = None if c["h0"] is None else c["h0"][b:b + 1, h:h + 1]
    return out


@pytest.mark.parametrize("name", list(CONFIGS))
def test_config_parity_and_properties(name, gpu_device):
    print(f"config {name}", flush=True)
    c = _inputs(name)
    B, T, H = c["q"].shape[:3]
    h0 = None if c["h0"] is None else c["h0"].to(gpu_device)
    o, ht = _fwd(c, gpu_device, h0=h0)
    o2, ht2 = _fwd(c, gpu_device, h0=h0)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all() and torch.isfinite(ht).all()
    assert torch.equal(o, o2) and torch.equal(ht, ht2), "repeat run differs"

    # resume invariant: split at a chunk boundary, bit-exact
    T1 = (T // 2) // 16 * 16
    oa, hta = _fwd(c, gpu_device, slice(0, T1), h0=h0)
    ob, htb = _fwd(c, gpu_device, slice(T1, T), h0=hta)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([oa, ob], dim=1), o), "resume: o differs"
    assert torch.equal(htb, ht), "resume: ht differs"

    # oracle and gold on (batch, head) slices
    o_c, ht_c = o.float().cpu(), ht.cpu()
    for b, h in sorted({(0, 0), (B - 1, H - 1), (B // 2, H // 2)}):
        p = _pair(c, b, h)
        kw = dict(A_log=p["A_log"], dt_bias=p["dt_bias"], lower_bound=LB, initial_state=p["h0"])
        o_r, ht_r, _ = chunked_reference(p["q"], p["k"], p["v"], p["g"].float(), p["beta"].float(),
                                         SCALE, **kw)
        o_g, ht_g = recurrent_gold(p["q"], p["k"], p["v"], p["g"].float(), p["beta"].float(),
                                   SCALE, dtype=torch.float32, **kw)
        got_o = o_c[b:b + 1, :, h:h + 1]
        got_h = ht_c[b:b + 1, h:h + 1]
        assert_close_rel(f"{name} b{b} h{h} o vs oracle", o_r.float(), got_o, 0.006)
        assert_close_rel(f"{name} b{b} h{h} ht vs oracle", ht_r, got_h, 0.006)
        bar_o = 1.5 * maxdiff(o_r.float(), o_g) + 1e-5
        bar_h = 1.5 * maxdiff(ht_r, ht_g) + 1e-5
        do, dh = maxdiff(got_o, o_g), maxdiff(got_h, ht_g)
        print(f"  b{b} h{h}: o {do:.3e} (bar {bar_o:.3e}) ht {dh:.3e} (bar {bar_h:.3e})", flush=True)
        assert do <= bar_o and dh <= bar_h

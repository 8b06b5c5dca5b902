"""The HIP path on the inputs of the fixtures the reference's own kernels
wrote (tests/golden/make_ref_fixtures.py; only the .npz is read here).

Two comparisons per case, through kda_bt16_debug -> C ABI -> gfx950 kernels:

* against the oracle on the same inputs, rounding to nearest as the GPU
  does (the oracle's rounding points are pinned to these fixtures on the
  CPU, tests/test_oracle_ref.py): stage-1 intermediates within 3 bf16 ulps
  of the largest element, g within 1e-4, o and ht within the reference
  tests' relative-RMS tolerance 0.006 (/root/reference/tests/
  test_kda_bt16.py:78-79) and 1e-2 max-abs;
* against the reference's outputs themselves.  They come from Triton's CPU
  interpreter, which rounds fp32 -> bf16 by truncation where the GPU rounds
  to nearest; truncation shrinks every rounded value, so the
  round-to-nearest oracle itself sits up to 2.2% (o) and 1.35% (ht)
  relative RMS and 4.5 bf16 ulps (w) from them.  The bar is that distance,
  measured in the test on the same case: the HIP result may be at most 1.5x
  as far (+1e-3) in relative RMS, and 2 ulps further for the intermediates.
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import kda_bt16_debug
from kda_oracle import chunked_reference
from kda_testlib import assert_close_rel, load_ref_fixture, maxdiff, ref_fixture_cases

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ref_fixture_cases())
def test_hip_vs_reference_fixtures(name, gpu_device):
    c = load_ref_fixture(name)
    dev = gpu_device
    print(f"[ref fixture] {name} T={c['q'].shape[1]}", flush=True)
    kw = dict(scale=c["scale"], initial_state=None if c["h0"] is None else c["h0"].to(dev),
              output_final_state=True, use_qk_l2norm_in_kernel=c["use_l2norm"],
              use_gate_in_kernel=c["use_gate"], use_beta_sigmoid_in_kernel=c["use_beta_sigmoid"],
              lower_bound=c["lower_bound"], A_log=c["A_log"].to(dev),
              dt_bias=c["dt_bias"].to(dev), state_v_first=c["state_v_first"])
    o, ht, dbg = kda_bt16_debug(*(c[x].to(dev) for x in ("q", "k", "v", "g", "beta")), **kw)
    torch.cuda.synchronize()
    o, ht = o.float().cpu(), ht.cpu()
    dbg = {key: t.float().cpu() for key, t in dbg.items()}
    assert torch.isfinite(o).all() and torch.isfinite(ht).all(), name

    o_or, ht_or, inter = chunked_reference(
        c["q"], c["k"], c["v"], c["g"], c["beta"], c["scale"], A_log=c["A_log"],
        dt_bias=c["dt_bias"], lower_bound=c["lower_bound"], initial_state=c["h0"],
        state_v_first=c["state_v_first"], use_gate=c["use_gate"], use_l2norm=c["use_l2norm"],
        use_beta_sigmoid=c["use_beta_sigmoid"])
    assert maxdiff(dbg["g"], inter["g"]) < 1e-4, name
    for key in ("Aqk", "A_inv", "w", "u"):
        want = inter[key].float()
        tol = 3 * 2.0 ** -8 * want.abs().max().item()
        assert maxdiff(dbg[key], want) <= tol, f"{name} {key} vs oracle: {maxdiff(dbg[key], want):.3e}"
    assert_close_rel(f"{name} o vs oracle", o_or.float(), o, 0.006)
    assert_close_rel(f"{name} ht vs oracle", ht_or, ht, 0.006)
    assert maxdiff(o, o_or.float()) < 1e-2 and maxdiff(ht, ht_or) < 1e-2, name

    ref = c["ref"]
    assert maxdiff(dbg["g"], ref["g"]) < 1e-4, name
    for key in ("Aqk", "A_inv", "w", "u"):
        want = ref[key].float()
        ulp = 2.0 ** -8 * want.abs().max().item()
        tol = maxdiff(inter[key].float(), want) + 2 * ulp
        assert maxdiff(dbg[key], want) <= tol, f"{name} {key} vs reference: {maxdiff(dbg[key], want):.3e}"
    for key, got, near in (("o", o, o_or.float()), ("ht", ht, ht_or)):
        want = ref[key].float()
        bar = 1.5 * _rel_rms(near, want) + 1e-3
        err = _rel_rms(got, want)
        print(f"  {key} vs reference: {err:.4f} (bar {bar:.4f})", flush=True)
        assert err <= bar, f"{name} {key} vs reference: rel RMS {err:.4f} > {bar:.4f}"


def _rel_rms(a: torch.Tensor, ref: torch.Tensor) -> float:
    a, ref = a.double(), ref.double()
    return ((a - ref).pow(2).mean().sqrt() / ref.pow(2).mean().sqrt()).item()

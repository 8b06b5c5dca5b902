"""The BASELINE configurations, and the bench's varlen workload, at full
size on the GPU.

Every output element is checked, at every config:

* against the CPU oracle (``chunked_reference``, the reference's chunked
  path with its bf16 rounding points), run one batch row at a time to bound
  host memory: per (batch, head), the relative RMS error of o and of ht is
  at most 0.006 (the reference tests' tolerance for the chunked path
  against its gold, tests/test_kda_bt16.py:78-79) and the largest absolute
  error at most 1e-2, so a fault confined to one head or one batch row
  cannot hide in an average;
* against the token recurrence in fp32 on the GPU (``kda_recurrent_fwd``):
  the largest absolute error of o and ht over the whole tensor is at most
  1.5x the oracle's own error against that recurrence (BASELINE's
  tolerance); the recurrence itself is pinned against the CPU fp32 gold
  (``recurrent_gold``) on three (batch, head) slices;

plus size-independent properties: determinism, and the resume invariant
(split at a chunk boundary, bit-exact).
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import kda_bt16_fwd, kda_recurrent_fwd
from kda_oracle import chunked_reference, make_inputs, per_sequence, recurrent_gold
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
REL_RMS = 0.006
MAX_ABS = 1e-2


def _inputs(name):
    cfg = dict(CONFIGS[name])
    B, T, H = cfg.pop("B"), cfg.pop("T"), cfg.pop("H")
    return make_inputs(B, T, H, seed=42, **cfg)


def _gate_kw(c, dev):
    return dict(scale=SCALE, output_final_state=True, use_qk_l2norm_in_kernel=True,
                use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, lower_bound=LB,
                A_log=c["A_log"].to(dev), dt_bias=c["dt_bias"].to(dev))


def _fwd(c, dev, sl=slice(None), h0=None):
    args = [c[x][:, sl].contiguous().to(dev) for x in ("q", "k", "v", "g", "beta")]
    return kda_bt16_fwd(*args, initial_state=h0, **_gate_kw(c, dev))


def _per_head_close(what, o_ref, o_got, ht_ref, ht_got):
    """o [B, T, H, V] and ht [B, H, V, K] (CPU, fp32): relative RMS and
    largest absolute error per (batch, head)."""
    def check(name, ref, got, red):
        d = (got.double() - ref.double())
        assert torch.isfinite(got).all(), f"{what} {name}: non-finite values"
        rel = d.pow(2).mean(dim=red).sqrt() / ref.double().pow(2).mean(dim=red).sqrt().clamp_min(1e-30)
        mx = d.abs().amax(dim=red)
        b, h = divmod(int(rel.argmax()), rel.shape[1])
        print(f"  {name}: worst rel-RMS {rel.max():.3e} (b{b} h{h}), worst max-abs {mx.max():.3e}",
              flush=True)
        assert (rel <= REL_RMS).all(), f"{what} {name}: rel-RMS {rel.max():.3e} at b{b} h{h}"
        assert (mx <= MAX_ABS).all(), f"{what} {name}: max-abs {mx.max():.3e}"
    check("o", o_ref, o_got, (1, 3))
    check("ht", ht_ref, ht_got, (2, 3))


def _oracle_rows(c):
    """The CPU oracle over the whole batch, one batch row at a time."""
    B = c["q"].shape[0]
    o_rows, ht_rows = [], []
    for b in range(B):
        row = {x: c[x][b:b + 1] for x in ("q", "k", "v", "g", "beta")}
        o_r, ht_r, _ = chunked_reference(
            row["q"], row["k"], row["v"], row["g"].float(), row["beta"].float(), SCALE,
            A_log=c["A_log"], dt_bias=c["dt_bias"], lower_bound=LB,
            initial_state=None if c["h0"] is None else c["h0"][b:b + 1])
        o_rows.append(o_r.float())
        ht_rows.append(ht_r)
    return torch.cat(o_rows), torch.cat(ht_rows)


def _pin_gold_slices(name, c, o_gold, ht_gold, pairs):
    """The GPU fp32 recurrence against the CPU fp32 gold on (batch, head)
    slices."""
    for b, h in pairs:
        hs = slice(h, h + 1)
        o_c, ht_c = recurrent_gold(
            c["q"][b:b + 1, :, hs], c["k"][b:b + 1, :, hs], c["v"][b:b + 1, :, hs],
            c["g"][b:b + 1, :, hs].float(), c["beta"][b:b + 1, :, hs].float(), SCALE,
            A_log=c["A_log"][hs], dt_bias=c["dt_bias"][h * 128:(h + 1) * 128], lower_bound=LB,
            initial_state=None if c["h0"] is None else c["h0"][b:b + 1, hs])
        assert_close_rel(f"{name} gold b{b} h{h} o", o_c, o_gold[b:b + 1, :, hs], 1e-5)
        assert_close_rel(f"{name} gold b{b} h{h} ht", ht_c, ht_gold[b:b + 1, hs], 1e-5)


def _against_gpu_gold(name, o_ref, ht_ref, o_got, ht_got, o_gold, ht_gold):
    bar_o = 1.5 * maxdiff(o_ref, o_gold) + 1e-5
    bar_h = 1.5 * maxdiff(ht_ref, ht_gold) + 1e-5
    do, dh = maxdiff(o_got, o_gold), maxdiff(ht_got, ht_gold)
    print(f"  vs fp32 recurrence: o {do:.3e} (bar {bar_o:.3e}) ht {dh:.3e} (bar {bar_h:.3e})",
          flush=True)
    assert do <= bar_o, f"{name}: o {do:.3e} > {bar_o:.3e}"
    assert dh <= bar_h, f"{name}: ht {dh:.3e} > {bar_h:.3e}"


@pytest.mark.parametrize("name", list(CONFIGS))
def test_config_parity_and_properties(name, gpu_device):
    print(f"config {name}", flush=True)
    dev = gpu_device
    c = _inputs(name)
    B, T, H = c["q"].shape[:3]
    h0 = None if c["h0"] is None else c["h0"].to(dev)
    o, ht = _fwd(c, dev, h0=h0)
    o2, ht2 = _fwd(c, dev, h0=h0)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all() and torch.isfinite(ht).all()
    assert torch.equal(o, o2) and torch.equal(ht, ht2), "repeat run differs"
    del o2, ht2

    # resume invariant: split at a chunk boundary, bit-exact
    T1 = (T // 2) // 16 * 16
    oa, hta = _fwd(c, dev, slice(0, T1), h0=h0)
    ob, htb = _fwd(c, dev, slice(T1, T), h0=hta)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([oa, ob], dim=1), o), "resume: o differs"
    assert torch.equal(htb, ht), "resume: ht differs"
    del oa, hta, ob, htb

    # the GPU fp32 recurrence on the same inputs
    x = [c[n].to(dev) for n in ("q", "k", "v", "g", "beta")]
    o_gold, ht_gold = kda_recurrent_fwd(*x, initial_state=h0, output_dtype=torch.float32,
                                        **_gate_kw(c, dev))
    torch.cuda.synchronize()
    del x
    o_gold, ht_gold = o_gold.cpu(), ht_gold.cpu()
    o_c, ht_c = o.float().cpu(), ht.cpu()
    del o, ht

    # every (batch, head) against the CPU oracle
    o_ref, ht_ref = _oracle_rows(c)
    _per_head_close(name, o_ref, o_c, ht_ref, ht_c)
    # the whole tensor against the fp32 recurrence, and that recurrence's pin
    _against_gpu_gold(name, o_ref, ht_ref, o_c, ht_c, o_gold, ht_gold)
    _pin_gold_slices(name, c, o_gold, ht_gold,
                     sorted({(0, 0), (B - 1, H - 1), (B // 2, H // 2)}))


def test_varlen_workload_full_size(gpu_device):
    """bench.py's varlen workload: the headline's 8192 tokens and 32 heads as
    16 packed sequences of uneven lengths (cu_seqlens), every (sequence,
    head) against the oracle run per sequence, and the whole tensor against
    the fp32 recurrence over the same cu_seqlens."""
    import bench

    dev = gpu_device
    cu_list = bench.varlen_offsets(seed=7)
    c = make_inputs(1, cu_list[-1], 32, seed=42)
    print(f"varlen: {len(cu_list) - 1} sequences, lengths "
          f"{[b - a for a, b in zip(cu_list, cu_list[1:])]}", flush=True)
    cu = torch.tensor(cu_list, dtype=torch.int32, device=dev)
    x = [c[n].to(dev) for n in ("q", "k", "v", "g", "beta")]
    o, ht = kda_bt16_fwd(*x, cu_seqlens=cu, **_gate_kw(c, dev))
    o_gold, ht_gold = kda_recurrent_fwd(*x, cu_seqlens=cu, output_dtype=torch.float32,
                                        **_gate_kw(c, dev))
    torch.cuda.synchronize()
    o_c, ht_c = o.float().cpu(), ht.cpu()
    o_gold, ht_gold = o_gold.cpu(), ht_gold.cpu()
    o_ref, ht_ref = per_sequence(
        chunked_reference, c["q"], c["k"], c["v"], c["g"].float(), c["beta"].float(), cu_list,
        SCALE, A_log=c["A_log"], dt_bias=c["dt_bias"], lower_bound=LB)
    o_ref = o_ref.float()
    # per (sequence, head): view the packed tokens of each sequence as a row
    for n, (a, b) in enumerate(zip(cu_list, cu_list[1:])):
        _per_head_close(f"varlen sequence {n}", o_ref[:, a:b], o_c[:, a:b], ht_ref[n:n + 1],
                        ht_c[n:n + 1])
    _against_gpu_gold("varlen", o_ref, ht_ref, o_c, ht_c, o_gold, ht_gold)
    # the recurrence's pin: the CPU gold on the first and last sequences, one head each
    for n, h in ((0, 0), (len(cu_list) - 2, 31)):
        a, b = cu_list[n], cu_list[n + 1]
        hs = slice(h, h + 1)
        o_c1, ht_c1 = recurrent_gold(
            c["q"][:, a:b, hs], c["k"][:, a:b, hs], c["v"][:, a:b, hs], c["g"][:, a:b, hs].float(),
            c["beta"][:, a:b, hs].float(), SCALE, A_log=c["A_log"][hs],
            dt_bias=c["dt_bias"][h * 128:(h + 1) * 128], lower_bound=LB)
        assert_close_rel(f"varlen gold n{n} h{h} o", o_c1, o_gold[:, a:b, hs], 1e-5)
        assert_close_rel(f"varlen gold n{n} h{h} ht", ht_c1, ht_gold[n:n + 1, hs], 1e-5)

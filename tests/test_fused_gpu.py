"""The fused forward (csrc/kda_fused.hip) against the two-stage forward
(csrc/kda_k1.hip, then csrc/kda_k2.hip or csrc/kda_k2w.hip), bit for bit:
the fused kernel runs stage 1's per-chunk code and the wide stage 2's step
(kernels.py:53-302) on records kept in LDS instead of HBM, so only where the
record lives differs.

``forward_choice(fused=...)`` (the ``KDA_BT16_TWO_STAGE`` /
``KDA_BT16_FUSED_KERNEL`` flags of the C ABI) forces the choice over the
launch heuristic, which fuses when the (sequence, head) pairs are more than
half the CUs (with cu_seqlens: at least as many as the CUs).  The cases
cover what the record ring has edges at: fewer chunks than ring slots,
counts that are and are not multiples of the ring and of the producer count,
partial last chunks, empty sequences in a varlen batch, grouped value heads,
both state layouts, fp32 and bf16 gates, and the precomputed-gate mode.
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import forward_choice, kda_bt16_fwd, workspace

pytestmark = pytest.mark.gpu

# 0: the two stages, 1: the fused kernel, None: the library's choice
_CHOICE = {0: False, 1: True, None: None}

# name, B, T, H, HV, cu_seqlens, state_v_first, h0, g dtype, in-kernel gate
CASES = [
    ("one_token", 1, 1, 1, 1, None, True, True, "bf16", True),
    ("one_chunk", 1, 16, 1, 2, None, True, True, "bf16", True),
    ("five_chunks", 2, 80, 1, 1, None, True, False, "bf16", True),
    ("six_chunks", 1, 96, 2, 2, None, False, True, "bf16", True),
    ("seven_chunks_partial", 1, 100, 1, 1, None, True, True, "fp32", True),
    ("partial_T300", 1, 300, 2, 2, None, True, False, "bf16", True),
    ("gva_kfirst_T1037", 2, 1037, 2, 4, None, False, True, "bf16", True),
    ("long_T2500_fp32g", 1, 2500, 1, 1, None, True, True, "fp32", True),
    ("precomputed_gate", 2, 333, 2, 2, None, True, True, "fp32", False),
    ("varlen_empty", 1, 400, 2, 2, [0, 0, 37, 53, 53, 120, 400], True, True, "bf16", True),
    ("varlen_kfirst", 1, 700, 1, 2, [0, 17, 300, 301, 700], False, True, "bf16", True),
    ("batch16_H32", 16, 160, 32, 32, None, True, True, "bf16", True),
]


def _inputs(B, T, H, HV, S, seed, gdt, in_kernel_gate):
    gen = torch.Generator().manual_seed(seed)
    if in_kernel_gate:
        g = torch.randn(B, T, HV, 128, generator=gen)
    else:
        # chunk-local log2 cumsum of a decay in (-1, 0) per token
        g = -torch.rand(B, T, HV, 128, generator=gen)
        pos = torch.arange(T) % 16
        g = torch.stack([g[:, t - int(pos[t]):t + 1].sum(1) for t in range(T)], 1)
    return dict(
        q=torch.randn(B, T, H, 128, generator=gen).bfloat16(),
        k=torch.randn(B, T, H, 128, generator=gen).bfloat16(),
        v=torch.randn(B, T, HV, 128, generator=gen).bfloat16(),
        g=g.bfloat16() if gdt == "bf16" else g.float(),
        beta=torch.randn(B, T, HV, generator=gen).bfloat16(),
        A_log=torch.log(torch.rand(HV, generator=gen) * 15 + 1),
        dt_bias=torch.randn(HV * 128, generator=gen) * 0.1,
        h0=torch.randn(S, HV, 128, 128, generator=gen) * 0.05,
    )


def _run(c, dev, cu, svf, h0, gate, fused):
    with forward_choice(fused=_CHOICE[fused]):
        init = None
        if h0:
            init = c["h0"] if svf else c["h0"].transpose(-1, -2).contiguous()
            init = init.to(dev)
        o, ht = kda_bt16_fwd(
            *(c[x].to(dev) for x in ("q", "k", "v", "g", "beta")), scale=0.1,
            initial_state=init, output_final_state=True, use_qk_l2norm_in_kernel=True,
            use_gate_in_kernel=gate, use_beta_sigmoid_in_kernel=True, lower_bound=-5.0,
            A_log=c["A_log"].to(dev) if gate else None,
            dt_bias=c["dt_bias"].to(dev) if gate else None, state_v_first=svf,
            cu_seqlens=None if cu is None else torch.tensor(cu, dtype=torch.int32, device=dev))
        torch.cuda.synchronize()
        return o, ht


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fused_forward_equals_two_stage(case, gpu_device):
    name, B, T, H, HV, cu, svf, h0, gdt, gate = case
    S = B if cu is None else len(cu) - 1
    c = _inputs(B, T, H, HV, S, seed=sum(map(ord, name)), gdt=gdt, in_kernel_gate=gate)
    print(f"[fused] {name}", flush=True)
    o2, ht2 = _run(c, gpu_device, cu, svf, h0, gate, 0)
    assert torch.isfinite(o2.float()).all() and torch.isfinite(ht2).all()
    o1, ht1 = _run(c, gpu_device, cu, svf, h0, gate, 1)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), f"{name}: o"
    assert torch.equal(ht1.view(torch.int32), ht2.view(torch.int32)), f"{name}: ht"
    # a second call on the same inputs gives the same bits (no state kept
    # between calls in the LDS ring or its flags)
    o3, ht3 = _run(c, gpu_device, cu, svf, h0, gate, 1)
    assert torch.equal(o3.view(torch.int16), o1.view(torch.int16)), f"{name}: o, second call"
    assert torch.equal(ht3.view(torch.int32), ht1.view(torch.int32)), f"{name}: ht, second call"


def test_heuristic_fuses_when_pairs_fill_the_cus(gpu_device):
    """B=16 T=64 H=32 (512 (sequence, head) pairs) runs fused by default and
    gives the two-stage result."""
    c = _inputs(16, 64, 32, 32, 16, seed=5, gdt="bf16", in_kernel_gate=True)
    o2, ht2 = _run(c, gpu_device, None, True, True, True, 0)
    o, ht = _run(c, gpu_device, None, True, True, True, None)
    assert torch.equal(o, o2) and torch.equal(ht, ht2)


@pytest.mark.parametrize("B,T,H,h0", [(1, 8192, 32, False), (16, 2048, 32, True)],
                         ids=["configs2_B1_T8192_H32", "configs4_B16_T2048_H32"])
def test_fused_equals_two_stage_at_baseline_sizes(B, T, H, h0, gpu_device):
    """BASELINE configs[2] and configs[4] at full size: the fused kernel
    (forced at configs[2], where the forward picks the two stages; picked by
    itself at configs[4]) against the two stages, bit for bit."""
    c = _inputs(B, T, H, H, B, seed=42 + B, gdt="bf16", in_kernel_gate=True)
    print(f"[fused] full size B={B} T={T} H={H}", flush=True)
    o2, ht2 = _run(c, gpu_device, None, True, h0, True, 0)
    o1, ht1 = _run(c, gpu_device, None, True, h0, True, 1)
    assert torch.isfinite(o2.float()).all() and torch.isfinite(ht2).all()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(ht1.view(torch.int32), ht2.view(torch.int32))


@pytest.mark.parametrize("lower_bound", [-8.0, -10.0])
def test_fused_saturated_gate(lower_bound, gpu_device):
    """The reference's saturated-gate case (tests/test_kda_bt16.py:128-171:
    A_log = 0, no dt_bias, g = 20, lower_bound -8 and -10) through the fused
    kernel: finite, and the two-stage bits."""
    B, T, H = 2, 200, 2
    c = _inputs(B, T, H, H, B, seed=11, gdt="bf16", in_kernel_gate=True)
    c["g"] = torch.full((B, T, H, 128), 20.0).bfloat16()
    c["A_log"] = torch.zeros(H)
    outs = []
    for fused in (0, 1):
        with forward_choice(fused=_CHOICE[fused]):
            o, ht = kda_bt16_fwd(
                *(c[x].to(gpu_device) for x in ("q", "k", "v", "g", "beta")), scale=0.1,
                initial_state=c["h0"].to(gpu_device), output_final_state=True,
                use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                use_beta_sigmoid_in_kernel=True, lower_bound=lower_bound,
                A_log=c["A_log"].to(gpu_device), dt_bias=None)
            torch.cuda.synchronize()
        assert torch.isfinite(o.float()).all() and torch.isfinite(ht).all()
        outs.append((o, ht))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def test_fused_repeated_calls_are_bit_identical(gpu_device):
    """Twenty back-to-back fused forwards at B=16 T=512 H=32 on one stream:
    every call gives the first call's bits (the LDS flags and ring start
    clean each launch, and no wait of the producer/consumer protocol runs
    out)."""
    c = _inputs(16, 512, 32, 32, 16, seed=13, gdt="bf16", in_kernel_gate=True)
    dev = gpu_device
    args = [c[x].to(dev) for x in ("q", "k", "v", "g", "beta")]
    kw = dict(scale=0.1, initial_state=c["h0"].to(dev), output_final_state=True,
              use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              use_beta_sigmoid_in_kernel=True, lower_bound=-5.0, A_log=c["A_log"].to(dev),
              dt_bias=c["dt_bias"].to(dev))
    with forward_choice(fused=True):
        runs = [kda_bt16_fwd(*args, **kw) for _ in range(20)]
        torch.cuda.synchronize()
    o0, h0 = runs[0]
    assert torch.isfinite(o0.float()).all()
    for i, (o, ht) in enumerate(runs[1:], 1):
        assert torch.equal(o.view(torch.int16), o0.view(torch.int16)), f"call {i}: o"
        assert torch.equal(ht.view(torch.int32), h0.view(torch.int32)), f"call {i}: ht"


def test_fused_forward_leases_no_workspace(gpu_device):
    """A fused forward keeps its records in LDS: it leases nothing from the
    workspace pool (B=16 T=512 H=32 would otherwise pin 272 MiB), while a
    two-stage forward of the same inputs does."""
    c = _inputs(16, 512, 32, 32, 16, seed=17, gdt="bf16", in_kernel_gate=True)
    workspace.clear()
    o1, ht1 = _run(c, gpu_device, None, True, True, True, None)
    assert workspace.pooled_bytes() == 0
    o2, ht2 = _run(c, gpu_device, None, True, True, True, 0)
    assert workspace.pooled_bytes() >= 16 * 32 * 32 * 17408
    workspace.clear()
    assert torch.equal(o1, o2) and torch.equal(ht1, ht2)


def test_varlen_max_seqlen_hint_keeps_the_results(gpu_device):
    """With cu_seqlens, max_seqlen only steers the choice of kernels: one
    long sequence among short ones (256 pairs) takes the two stages with the
    hint and the fused kernel without it, and both give the same bits."""
    lens = [2048] + [128] * 7
    cu_list = [0]
    for n in lens:
        cu_list.append(cu_list[-1] + n)
    T, HV = cu_list[-1], 32
    dev = gpu_device
    if len(lens) * HV < torch.cuda.get_device_properties(dev).multi_processor_count:
        pytest.skip("the case needs at least as many (sequence, head) pairs as CUs")
    c = _inputs(1, T, HV, HV, len(lens), seed=19, gdt="bf16", in_kernel_gate=True)
    cu = torch.tensor(cu_list, dtype=torch.int32, device=dev)
    kw = dict(scale=0.1, initial_state=c["h0"].to(dev), output_final_state=True,
              use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              use_beta_sigmoid_in_kernel=True, lower_bound=-5.0, A_log=c["A_log"].to(dev),
              dt_bias=c["dt_bias"].to(dev), cu_seqlens=cu)
    args = [c[x].to(dev) for x in ("q", "k", "v", "g", "beta")]
    workspace.clear()
    o1, ht1 = kda_bt16_fwd(*args, **kw)  # 256 pairs: fused
    torch.cuda.synchronize()
    assert workspace.pooled_bytes() == 0
    o2, ht2 = kda_bt16_fwd(*args, max_seqlen=max(lens), **kw)  # skewed: two stages
    torch.cuda.synchronize()
    assert workspace.pooled_bytes() > 0
    workspace.clear()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(ht1.view(torch.int32), ht2.view(torch.int32))

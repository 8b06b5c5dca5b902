"""The token recurrence on the GPU (kda_recurrent_fwd / kda_decode_step ->
kda_recurrent_fwd_hip -> gfx950 kernel) against the oracle's fp32
recurrent gold, and the chunked path against it at the headline size.

Bars (written in each test):
* fp32 output vs the oracle's fp32 recurrence: relative RMS <= 1e-5 and
  max-abs <= 1e-4 relative to the output's scale (both fp32; they differ
  only in summation order);
* bf16 output = the fp32 output rounded to nearest even, bit for bit;
* T decode steps with the state updated in place = one call over T tokens,
  bit for bit (the steps run the kernel's one-token variant, the single
  call its general one);
* chunked path at B=1 T=8192 H=32 vs this gold: max-abs error of o and ht
  no worse than 1.5x the reference chunked path's own error (the oracle in
  kernel mode) on the same inputs, plus 1e-5.
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import kda_bt16_fwd, kda_decode_step, kda_recurrent_fwd
from kda_oracle import chunked_reference, make_inputs, recurrent_gold
from kda_testlib import assert_close_rel, maxdiff

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, HV, seed, *, h0_std=0.05, gate_dtype=torch.float32, small=False):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(B, T, H, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(B, T, HV, 128, generator=gen).to(torch.bfloat16)
    g = torch.randn(B, T, HV, 128, generator=gen)
    beta = torch.randn(B, T, HV, generator=gen)
    A_log = torch.log(torch.rand(HV, generator=gen) * 15.0 + 1.0)
    dt_bias = torch.randn(HV * 128, generator=gen) * 0.1
    h0 = torch.randn(B, HV, 128, 128, generator=gen) * h0_std if h0_std > 0 else None
    if small:  # no l2norm: keep |k|^2 * beta below 1 so the recurrence stays bounded
        q, k = ((x.float() * 0.08).to(torch.bfloat16) for x in (q, k))
    return dict(q=q, k=k, v=v, g=g.to(gate_dtype), beta=beta.to(gate_dtype), A_log=A_log,
                dt_bias=dt_bias, h0=h0)


CASES = {
    # name: (B, T, H, HV, flags, state_v_first, gate_dtype)
    "all_flags_h0": (2, 37, 2, 2, dict(gate=True, l2=True, sig=True), True, torch.float32),
    "kfirst_state": (1, 33, 2, 2, dict(gate=True, l2=True, sig=True), False, torch.float32),
    "gva_x2": (2, 24, 2, 4, dict(gate=True, l2=True, sig=True), True, torch.float32),
    "decode_T1": (3, 1, 4, 4, dict(gate=True, l2=True, sig=True), True, torch.float32),
    "bf16_gates": (1, 29, 2, 2, dict(gate=True, l2=True, sig=True), True, torch.bfloat16),
    "log_decay_raw": (2, 21, 2, 2, dict(gate=False, l2=False, sig=False), True, torch.float32),
}


def _run(c, dev, flags, state_v_first, output_dtype=torch.float32, **over):
    h0 = c["h0"]
    if h0 is not None and not state_v_first:
        h0 = h0.transpose(-1, -2).contiguous()
    g = c["g"] if flags["gate"] else (-torch.rand_like(c["g"].float()) * 0.3).to(c["g"].dtype)
    kw = dict(
        scale=0.1, initial_state=None if h0 is None else h0.to(dev), output_final_state=True,
        use_qk_l2norm_in_kernel=flags["l2"], use_gate_in_kernel=flags["gate"],
        use_beta_sigmoid_in_kernel=flags["sig"], lower_bound=-5.0,
        A_log=c["A_log"].to(dev), dt_bias=c["dt_bias"].to(dev), state_v_first=state_v_first,
        output_dtype=output_dtype,
    )
    kw.update(over)
    o, ht = kda_recurrent_fwd(c["q"].to(dev), c["k"].to(dev), c["v"].to(dev), g.to(dev),
                              c["beta"].to(dev), **kw)
    gold = recurrent_gold(
        c["q"], c["k"], c["v"], g.float(), c["beta"].float(), 0.1, A_log=c["A_log"],
        dt_bias=c["dt_bias"], lower_bound=-5.0, initial_state=h0, state_v_first=state_v_first,
        use_gate=flags["gate"], use_l2norm=flags["l2"], use_beta_sigmoid=flags["sig"],
        gate_log=not flags["gate"], dtype=torch.float32,
    )
    return o, ht, gold


@pytest.mark.parametrize("name", list(CASES))
def test_recurrent_matches_fp32_gold(name, gpu_device):
    B, T, H, HV, flags, vfirst, gdt = CASES[name]
    c = _inputs(B, T, H, HV, seed=7, gate_dtype=gdt, small=not flags["l2"])
    o, ht, (o_g, ht_g) = _run(c, gpu_device, flags, vfirst)
    o, ht = o.cpu(), ht.cpu()
    assert torch.isfinite(o).all() and torch.isfinite(ht).all()
    # both fp32; they differ only in summation order
    assert_close_rel(f"{name} o", o_g, o, 1e-5)
    assert_close_rel(f"{name} ht", ht_g, ht, 1e-5)
    assert maxdiff(o, o_g) <= 1e-4 * max(o_g.abs().max().item(), 1e-3), name
    assert maxdiff(ht, ht_g) <= 1e-4 * max(ht_g.abs().max().item(), 1e-3), name


def test_bf16_output_is_rounded_fp32(gpu_device):
    B, T, H, HV, flags, vfirst, gdt = CASES["all_flags_h0"]
    c = _inputs(B, T, H, HV, seed=11)
    o32, ht32, _ = _run(c, gpu_device, flags, vfirst, torch.float32)
    o16, ht16, _ = _run(c, gpu_device, flags, vfirst, torch.bfloat16)
    assert o16.dtype == torch.bfloat16
    assert torch.equal(o16, o32.to(torch.bfloat16))
    assert torch.equal(ht16, ht32)


@pytest.mark.parametrize("vfirst", [True, False])
def test_decode_steps_equal_one_call(vfirst, gpu_device):
    dev = gpu_device
    B, T, H, HV = 2, 9, 2, 4
    c = _inputs(B, T, H, HV, seed=3)
    h0 = c["h0"] if vfirst else c["h0"].transpose(-1, -2).contiguous()
    kw = dict(scale=0.1, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              use_beta_sigmoid_in_kernel=True, lower_bound=-5.0, A_log=c["A_log"].to(dev),
              dt_bias=c["dt_bias"].to(dev), state_v_first=vfirst)
    x = {n: c[n].to(dev) for n in ("q", "k", "v", "g", "beta")}
    o_all, ht_all = kda_recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"],
                                      initial_state=h0.to(dev), output_final_state=True, **kw)
    state = h0.to(dev).clone()
    outs = []
    for t in range(T):
        step = {n: x[n][:, t:t + 1].contiguous() for n in x}
        outs.append(kda_decode_step(step["q"], step["k"], step["v"], step["g"], step["beta"],
                                    state, **kw))
    assert torch.equal(torch.cat(outs, dim=1), o_all)
    assert torch.equal(state, ht_all)


def test_chunked_path_vs_gpu_gold_headline(gpu_device):
    """BASELINE configs[2] (B=1 T=8192 H=32, bf16 storage) against the GPU
    recurrence in fp32, pinned itself against the CPU gold on two heads."""
    dev = gpu_device
    c = make_inputs(1, 8192, 32)
    x = {n: c[n].to(dev) for n in ("q", "k", "v", "g", "beta")}
    kw = dict(scale=128 ** -0.5, output_final_state=True, use_qk_l2norm_in_kernel=True,
              use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, lower_bound=-5.0,
              A_log=c["A_log"].to(dev), dt_bias=c["dt_bias"].to(dev))
    o_gold, ht_gold = kda_recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"],
                                        output_dtype=torch.float32, **kw)
    o_hip, ht_hip = kda_bt16_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], **kw)
    torch.cuda.synchronize()
    o_gold, ht_gold, o_hip, ht_hip = (t.float().cpu() for t in (o_gold, ht_gold, o_hip, ht_hip))

    # the GPU gold against the CPU gold on heads 0 and 17
    for h in (0, 17):
        sl = slice(h, h + 1)
        o_c, ht_c = recurrent_gold(
            c["q"][:, :, sl], c["k"][:, :, sl], c["v"][:, :, sl], c["g"][:, :, sl].float(),
            c["beta"][:, :, sl].float(), 128 ** -0.5, A_log=c["A_log"][sl],
            dt_bias=c["dt_bias"][h * 128:(h + 1) * 128], lower_bound=-5.0)
        assert_close_rel(f"gold head {h} o", o_c, o_gold[:, :, sl], 1e-5)
        assert_close_rel(f"gold head {h} ht", ht_c, ht_gold[:, sl], 1e-5)

    # the reference chunked path's own error on the same inputs
    o_ref, ht_ref, _ = chunked_reference(
        c["q"], c["k"], c["v"], c["g"].float(), c["beta"].float(), 128 ** -0.5,
        A_log=c["A_log"], dt_bias=c["dt_bias"], lower_bound=-5.0, mode="kernel")
    bar_o = 1.5 * maxdiff(o_ref.float(), o_gold) + 1e-5
    bar_h = 1.5 * maxdiff(ht_ref, ht_gold) + 1e-5
    do, dh = maxdiff(o_hip, o_gold), maxdiff(ht_hip, ht_gold)
    print(f"headline: o {do:.3e} (bar {bar_o:.3e})  ht {dh:.3e} (bar {bar_h:.3e})", flush=True)
    assert do <= bar_o and dh <= bar_h

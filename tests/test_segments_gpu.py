"""The two-stage forward in chunk ranges against one pass, bit for bit.

A fixed-length forward whose stage-1 records would outgrow the GPU's
last-level cache runs stage 1 then stage 2 on each of 2 or more consecutive
chunk ranges, stage 2 carrying the state from one range to the next
(``kda_bt16_fwd_segments``).  Stage 2 resuming from a state gives the bits of
the uninterrupted recurrence (kernels.py:225-302 run over the chunks in
order either way), so ``kda_bt16_fwd`` must equal the stage-level entry
points run once over all chunks (``kda_bt16_stage_launchers``, one pass):
batch rows (the row stride of a range), a partial last chunk, grouped value
heads, both state layouts, with and without an initial and a final state,
stage 2 at one, two and four value tiles per work-group, and 2 to 16
ranges.
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import forward_choice, kda_bt16_fwd, kda_bt16_stage_launchers

pytestmark = pytest.mark.gpu

# name, B, T, H, HV, initial state, final state, state_v_first, ranges
CASES = [
    ("one_row", 1, 8192, 32, 32, False, True, True, 2),
    ("two_rows_kfirst", 2, 8192, 16, 16, True, True, False, 2),
    ("partial_last_chunk", 1, 8192 + 37, 32, 32, True, False, True, 2),
    ("grouped_heads", 1, 8192, 16, 32, True, True, True, 2),
    ("four_ranges", 1, 16384, 32, 32, False, True, True, 4),
    ("two_tiles", 1, 4096, 64, 64, True, True, True, 2),
    ("four_tiles", 1, 4096, 96, 96, True, True, True, 3),
    ("c3_four_tiles", 1, 8192, 96, 96, False, True, True, 6),
    ("sixteen_ranges_kfirst", 1, 16384, 128, 128, True, True, False, 16),
]


def _inputs(B, T, H, HV, seed, dev):
    gen = torch.Generator(device=dev).manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen, device=dev)
    return dict(
        q=r(B, T, H, 128).bfloat16(), k=r(B, T, H, 128).bfloat16(),
        v=r(B, T, HV, 128).bfloat16(), g=r(B, T, HV, 128).bfloat16(),
        beta=r(B, T, HV).bfloat16(),
        A_log=torch.log(torch.rand(HV, generator=gen, device=dev) * 15 + 1),
        dt_bias=r(HV * 128) * 0.1,
        h0=r(B, HV, 128, 128) * 0.05,
    )


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_ranges_equal_one_pass(case, gpu_device):
    name, B, T, H, HV, with_h0, with_ht, svf, ranges = case
    print(f"[segments] {name}: B={B} T={T} H={H} HV={HV}", flush=True)
    x = _inputs(B, T, H, HV, seed=len(name), dev=gpu_device)
    h0 = None
    if with_h0:
        h0 = x["h0"] if svf else x["h0"].transpose(-1, -2).contiguous()
    kw = dict(scale=0.1, initial_state=h0, output_final_state=with_ht, use_qk_l2norm_in_kernel=True,
              use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, lower_bound=-5.0,
              A_log=x["A_log"], dt_bias=x["dt_bias"], state_v_first=svf)
    ins = [x[n] for n in ("q", "k", "v", "g", "beta")]
    k1, k2, o1, ht1 = kda_bt16_stage_launchers(*ins, **kw)
    assert k1.forward_plan == "two-stage" and k1.forward_segments == ranges, name
    k1()
    k2()
    with forward_choice(fused=False):
        o, ht = kda_bt16_fwd(*ins, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all(), name
    assert torch.equal(o.view(torch.int16), o1.view(torch.int16)), f"{name}: o"
    if with_ht:
        assert torch.equal(ht.view(torch.int32), ht1.view(torch.int32)), f"{name}: ht"
    else:
        assert ht is None and ht1 is None


def test_ranges_graph_replays_equal_eager(gpu_device):
    """The forward in chunk ranges captured into a HIP graph
    (torch.cuda.CUDAGraph): four launches, the state between ranges carried
    in the captured workspace.  Each replay, on new inputs copied into the
    captured buffers with eager work and a synchronisation between replays,
    equals the eager call bit for bit."""
    B, T, H, reps = 1, 8192, 32, 2
    print(f"[segments] graph capture: B={B} T={T} H={H}", flush=True)
    cases = [_inputs(B, T, H, H, seed=100 + i, dev=gpu_device) for i in range(reps)]
    names = ("q", "k", "v", "g", "beta", "h0")
    kw = dict(scale=0.1, output_final_state=True, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              use_beta_sigmoid_in_kernel=True, lower_bound=-5.0,
              A_log=cases[0]["A_log"], dt_bias=cases[0]["dt_bias"])
    k1, *_ = kda_bt16_stage_launchers(*(cases[0][n] for n in names[:5]), **kw)
    assert k1.forward_plan == "two-stage" and k1.forward_segments == 2
    eager = []
    for x in cases:
        o, ht = kda_bt16_fwd(*(x[n] for n in names[:5]), initial_state=x["h0"], **kw)
        eager.append((o.clone(), ht.clone()))
    torch.cuda.synchronize()

    static = [cases[0][n].clone() for n in names]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_static, ht_static = kda_bt16_fwd(*static[:5], initial_state=static[5], **kw)
    for i, x in enumerate(cases):
        for dst, n in zip(static, names):
            dst.copy_(x[n])
        graph.replay()
        torch.cuda.synchronize()
        float(torch.randn(4096, device=gpu_device).square().sum())  # unrelated eager work
        assert torch.equal(o_static.view(torch.int16), eager[i][0].view(torch.int16)), f"replay {i}: o"
        assert torch.equal(ht_static.view(torch.int32), eager[i][1].view(torch.int32)), f"replay {i}: ht"


@pytest.mark.parametrize("B,T,H,HV,ranges", [(1, 8192, 32, 32, 2), (1, 4096, 48, 96, 3)],
                         ids=["c2_two_ranges", "gva_three_ranges"])
def test_training_forward_in_ranges(B, T, H, HV, ranges, gpu_device):
    """The training forward that keeps its state (autograd's default,
    kda_bt16_fwd_save_hip) runs in the same chunk ranges, its saved state in
    the whole forward's record slots: o and ht equal the inference
    forward's, and the gradients from that state equal the recompute
    path's, which rebuilds the state in one pass, bit for bit."""
    from kda_bt16 import set_backward_recompute

    print(f"[segments] training forward: B={B} T={T} H={H} HV={HV}", flush=True)
    x = _inputs(B, T, H, HV, seed=7, dev=gpu_device)
    names = ("q", "k", "v", "g", "beta", "A_log", "dt_bias", "h0")
    kw = dict(scale=0.1, output_final_state=True, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              use_beta_sigmoid_in_kernel=True, lower_bound=-5.0)
    k1, *_ = kda_bt16_stage_launchers(*(x[n] for n in names[:5]), initial_state=x["h0"],
                                      A_log=x["A_log"], dt_bias=x["dt_bias"], **kw)
    assert k1.forward_plan == "two-stage" and k1.forward_segments == ranges
    gen = torch.Generator(device=gpu_device).manual_seed(3)
    do = torch.randn(B, T, HV, 128, generator=gen, device=gpu_device).bfloat16()
    dht = torch.randn(B, HV, 128, 128, generator=gen, device=gpu_device) * 0.1

    def run(recompute):
        set_backward_recompute(recompute)
        lv = {n: x[n].detach().clone().requires_grad_(True) for n in names}
        o, ht = kda_bt16_fwd(*(lv[n] for n in names[:5]), initial_state=lv["h0"],
                             A_log=lv["A_log"], dt_bias=lv["dt_bias"], **kw)
        loss = (o.float() * do.float()).sum() + (ht * dht).sum()
        return o.detach(), ht.detach(), torch.autograd.grad(loss, [lv[n] for n in names])

    try:
        o_s, ht_s, g_s = run(False)
        _, _, g_r = run(True)
    finally:
        set_backward_recompute(False)
    with torch.no_grad():
        o_i, ht_i = kda_bt16_fwd(*(x[n] for n in names[:5]), initial_state=x["h0"],
                                 A_log=x["A_log"], dt_bias=x["dt_bias"], **kw)
    torch.cuda.synchronize()
    assert torch.equal(o_s.view(torch.int16), o_i.view(torch.int16)), "o"
    assert torch.equal(ht_s.view(torch.int32), ht_i.view(torch.int32)), "ht"
    for n, a, b in zip(names, g_s, g_r):
        assert torch.isfinite(a.float()).all(), n
        assert torch.equal(a, b), f"d{n}"


def _random_range_cases(n=8, seed=2024):
    """Seeded shapes whose records exceed 200 MB: batch rows 1-3, value
    heads 16-64 in groups of 1, 2 or 4, ragged token counts."""
    import random

    rng = random.Random(seed)
    cases = []
    while len(cases) < n:
        B = rng.choice([1, 1, 2, 3])
        group = rng.choice([1, 1, 2, 4])
        HV = rng.choice([16, 24, 32, 48, 64])
        if HV % group:
            continue
        T = rng.randrange(2048, 12000)
        if B * HV * ((T + 15) // 16) * 17408 <= 210e6:
            continue
        cases.append((B, T, HV // group, HV, rng.random() < 0.7, rng.random() < 0.7, rng.random() < 0.5))
    return cases


RANDOM_CASES = _random_range_cases()


@pytest.mark.parametrize("case", RANDOM_CASES, ids=[f"B{c[0]}_T{c[1]}_H{c[2]}_HV{c[3]}" for c in RANDOM_CASES])
def test_ranges_random_shapes(case, gpu_device):
    """Seeded shapes above 200 MB of records: the forward in chunk ranges
    equals one pass bit for bit."""
    B, T, H, HV, with_h0, with_ht, svf = case
    print(f"[segments] random: B={B} T={T} H={H} HV={HV} h0={with_h0} ht={with_ht} v_first={svf}", flush=True)
    x = _inputs(B, T, H, HV, seed=T, dev=gpu_device)
    h0 = None
    if with_h0:
        h0 = x["h0"] if svf else x["h0"].transpose(-1, -2).contiguous()
    kw = dict(scale=0.1, initial_state=h0, output_final_state=with_ht, use_qk_l2norm_in_kernel=True,
              use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, lower_bound=-5.0,
              A_log=x["A_log"], dt_bias=x["dt_bias"], state_v_first=svf)
    ins = [x[n] for n in ("q", "k", "v", "g", "beta")]
    with forward_choice(fused=False):
        k1, k2, o1, ht1 = kda_bt16_stage_launchers(*ins, **kw)
        assert k1.forward_segments >= 2
        k1()
        k2()
        o, ht = kda_bt16_fwd(*ins, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()
    assert torch.equal(o.view(torch.int16), o1.view(torch.int16)), "o"
    if with_ht:
        assert torch.equal(ht.view(torch.int32), ht1.view(torch.int32)), "ht"


@pytest.mark.parametrize("mode", ["fp32_gate_beta", "precomputed_gate"])
def test_ranges_gate_forms(mode, gpu_device):
    """The range offsets of g and beta follow their element type (fp32 g and
    beta here), and a precomputed gate (no in-kernel gate, kernels.py:116-124
    with USE_GATE off) runs in ranges too: bit for bit against one pass."""
    B, T, H = 1, 8192 + 5, 32
    print(f"[segments] {mode}: B={B} T={T} H={H}", flush=True)
    x = _inputs(B, T, H, H, seed=11, dev=gpu_device)
    if mode == "fp32_gate_beta":
        g, beta = x["g"].float(), x["beta"].float()
        kw = dict(use_gate_in_kernel=True, lower_bound=-5.0, A_log=x["A_log"], dt_bias=x["dt_bias"])
    else:
        # a precomputed gate: small non-positive values, no in-kernel gate
        g = (-torch.nn.functional.softplus(x["g"].float()) * 0.1).bfloat16()
        beta = x["beta"]
        kw = dict(use_gate_in_kernel=False)
    kw.update(scale=0.1, initial_state=x["h0"], output_final_state=True, use_qk_l2norm_in_kernel=True,
              use_beta_sigmoid_in_kernel=True)
    ins = [x["q"], x["k"], x["v"], g, beta]
    k1, k2, o1, ht1 = kda_bt16_stage_launchers(*ins, **kw)
    assert k1.forward_plan == "two-stage" and k1.forward_segments == 2
    k1()
    k2()
    o, ht = kda_bt16_fwd(*ins, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()
    assert torch.equal(o.view(torch.int16), o1.view(torch.int16)), "o"
    assert torch.equal(ht.view(torch.int32), ht1.view(torch.int32)), "ht"

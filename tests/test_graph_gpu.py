"""HIP graph capture (torch.cuda.CUDAGraph) of the decode step and of the
forward, two-stage and fused.  The C-ABI entry points launch on torch's
current stream, record no memset and allocate nothing themselves, so a
serving loop can capture a step once and replay it without the Python
wrapper's cost.

Each test captures once, then replays with new inputs copied into the
captured buffers, with eager work and a synchronisation between replays,
and requires every replay to equal the eager call on the same inputs bit
for bit.  An eager call comes first, so the library and its code objects
are loaded before the capture.
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import kda_bt16_fwd, kda_decode_step

pytestmark = pytest.mark.gpu

D = 128


def _step_inputs(B, T, H, dev, gen):
    q, k, v = (torch.randn(B, T, H, D, device=dev, generator=gen).bfloat16() for _ in range(3))
    g = torch.randn(B, T, H, D, device=dev, generator=gen)
    beta = torch.randn(B, T, H, device=dev, generator=gen)
    return [q, k, v, g, beta]


def _gate_kw(H, dev, gen):
    return dict(scale=D ** -0.5, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                use_beta_sigmoid_in_kernel=True, lower_bound=-5.0,
                A_log=torch.log(torch.rand(H, device=dev, generator=gen) * 15.0 + 1.0),
                dt_bias=torch.randn(H * D, device=dev, generator=gen) * 0.1)


def _eager_noise(dev):
    # unrelated eager work between replays
    x = torch.randn(4096, device=dev)
    return float((x * x).sum())


def test_decode_step_graph_replays_equal_eager(gpu_device):
    dev = gpu_device
    B, H, steps = 4, 8, 6
    gen = torch.Generator(device=dev).manual_seed(5)
    kw = _gate_kw(H, dev, gen)
    state0 = torch.randn(B, H, D, D, device=dev, generator=gen) * 0.05
    inputs = [_step_inputs(B, 1, H, dev, gen) for _ in range(steps)]
    print(f"[graph] decode B={B} H={H} steps={steps}", flush=True)

    state_e = state0.clone()
    outs_e = [kda_decode_step(*x, state_e, **kw).clone() for x in inputs]
    torch.cuda.synchronize()

    static = [t.clone() for t in inputs[0]]
    state_g = state0.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_static = kda_decode_step(*static, state_g, **kw)
    # capture runs nothing: the state is untouched until the first replay
    assert torch.equal(state_g, state0)
    for i, x in enumerate(inputs):
        for dst, src in zip(static, x):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        _eager_noise(dev)
        assert torch.equal(o_static, outs_e[i]), f"replay {i}: o differs"
    assert torch.equal(state_g, state_e), "state after the replays differs"


@pytest.mark.parametrize("fused", [False, True], ids=["two_stage", "fused"])
def test_forward_graph_replays_equal_eager(fused, gpu_device):
    dev = gpu_device
    B, T, H, reps = 2, 80, 4, 3
    gen = torch.Generator(device=dev).manual_seed(9)
    kw = _gate_kw(H, dev, gen)
    kw.update(output_final_state=True, use_fused_kernel=fused)
    cases = []
    for _ in range(reps):
        x = _step_inputs(B, T, H, dev, gen)
        x[3] = x[3].bfloat16()
        x[4] = x[4].bfloat16()
        cases.append(x + [torch.randn(B, H, D, D, device=dev, generator=gen) * 0.05])
    print(f"[graph] forward B={B} T={T} H={H} fused={fused}", flush=True)

    eager = []
    for *x, h0 in cases:
        o, ht = kda_bt16_fwd(*x, initial_state=h0, **kw)
        eager.append((o.clone(), ht.clone()))
    torch.cuda.synchronize()

    static = [t.clone() for t in cases[0]]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_static, ht_static = kda_bt16_fwd(*static[:5], initial_state=static[5], **kw)
    for i, case in enumerate(cases):
        for dst, src in zip(static, case):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        _eager_noise(dev)
        assert torch.equal(o_static, eager[i][0]), f"replay {i}: o differs"
        assert torch.equal(ht_static, eager[i][1]), f"replay {i}: ht differs"

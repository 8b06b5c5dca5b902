"""Pins for the backward oracle (oracle/kda_oracle_bwd.py) before it is
trusted as the checker of the HIP backward.  Everything here runs on the CPU.

* autograd through the token recurrence against central finite differences
  (torch.autograd.gradcheck) on tiny shapes: the gold gradient is the
  gradient of the op's definition;
* the hand-written chunked backward (the algorithm the HIP kernels run) in
  fp64 against that gold, on partial chunks, non-zero states and their
  gradients, both layouts, grouped value heads and every gate mode: the two
  agree only if every term (solve, grams, recentring, gates, beta, l2norm,
  the reverse state chain) is right;
* a planted mistake in the restatement (a dropped term) fails the check.
"""

from __future__ import annotations

import pytest
import torch

import kda_oracle_bwd
from kda_oracle import k1_reference, make_inputs, recurrent_gold
from kda_oracle_bwd import autograd_grads, chunked_backward


def _rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).pow(2).mean().sqrt() / b.pow(2).mean().sqrt().clamp_min(1e-300)).item()


def _case(B, T, H, HV, *, seed=5, gate_log=False, precomputed=False, svf=True):
    c = make_inputs(B, T, HV, seed=seed, h0_std=0.1)
    q = c["q"][:, :, :H].contiguous()
    k = c["k"][:, :, :H].contiguous()
    g = c["g"].float()
    if gate_log:
        g = -torch.rand(B, T, HV, 128, generator=torch.Generator().manual_seed(seed)) * 0.5
    if precomputed:
        st = k1_reference(q, k, c["v"], g, c["beta"].float(), 0.1, A_log=c["A_log"],
                          dt_bias=c["dt_bias"], mode="exact")
        NT = -(-T // 16)
        g = st["G"].reshape(B, HV, NT * 16, 128)[:, :, :T].movedim(1, 2).contiguous().float()
    gen = torch.Generator().manual_seed(seed + 1)
    do = torch.randn(B, T, HV, 128, generator=gen)
    dht = torch.randn(B, HV, 128, 128, generator=gen) * 0.1
    h0 = c["h0"] if svf else c["h0"].transpose(-1, -2).contiguous()
    return (q, k, c["v"], g, c["beta"].float(), do), dict(
        A_log=c["A_log"], dt_bias=c["dt_bias"], initial_state=h0, dht=dht, state_v_first=svf,
        use_gate=not (gate_log or precomputed), gate_log=gate_log)


@pytest.mark.parametrize("B,T,H,HV,kw", [
    (1, 16, 1, 1, {}),
    (2, 37, 2, 2, {}),
    (1, 33, 2, 4, {}),                       # grouped value heads
    (1, 17, 1, 1, {"svf": False}),           # K-first state
    (1, 20, 1, 1, {"gate_log": True}),       # FLA's per-token log decay
    (1, 40, 2, 2, {"precomputed": True}),    # the reference's precomputed cumsum
    (1, 1, 1, 1, {}),                        # one token
])
def test_chunked_backward_equals_autograd(B, T, H, HV, kw):
    args, fkw = _case(B, T, H, HV, **kw)
    ga = autograd_grads(*args, 0.1, **fkw)
    gc = chunked_backward(*args, 0.1, **fkw)
    names = [n for n in ga if n.startswith("d")]
    assert set(names) <= set(gc)
    for n in names:
        # RCP_LN2 = 1.4426950216 vs 1/ln 2 (1.3e-8 relative) is the only
        # non-roundoff difference between the formulations
        assert _rel(gc[n], ga[n]) < 1e-6, n


def test_no_l2norm_no_sigmoid():
    c = make_inputs(1, 40, 2, seed=8, h0_std=0.1)
    do = torch.randn(1, 40, 2, 128, generator=torch.Generator().manual_seed(2))
    kw = dict(A_log=c["A_log"], dt_bias=c["dt_bias"], initial_state=c["h0"],
              use_l2norm=False, use_beta_sigmoid=False)
    ga = autograd_grads(c["q"], c["k"], c["v"], c["g"].float(), c["beta"].float(), do, 0.05, **kw)
    gc = chunked_backward(c["q"], c["k"], c["v"], c["g"].float(), c["beta"].float(), do, 0.05, **kw)
    for n in (x for x in ga if x.startswith("d")):
        assert _rel(gc[n], ga[n]) < 1e-5, n


def test_recurrence_gradient_against_finite_differences():
    """The gold itself: autograd of the fp64 recurrence against central
    differences, every input including the gate parameters and h0."""
    torch.manual_seed(0)
    B, T, H, K = 1, 5, 1, 128
    gen = torch.Generator().manual_seed(11)
    q = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    k = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    v = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    g = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    beta = torch.randn(B, T, H, generator=gen, dtype=torch.float64)
    A_log = torch.log(torch.rand(H, generator=gen, dtype=torch.float64) * 15 + 1)
    dt_bias = torch.randn(H * K, generator=gen, dtype=torch.float64) * 0.1
    h0 = torch.randn(B, H, K, K, generator=gen, dtype=torch.float64) * 0.1
    w_o = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    w_h = torch.randn(B, H, K, K, generator=gen, dtype=torch.float64) * 0.1

    def f(q, k, v, g, beta, A_log, dt_bias, h0):
        o, ht = recurrent_gold(q, k, v, g, beta, 0.1, A_log=A_log, dt_bias=dt_bias,
                               initial_state=h0, dtype=torch.float64)
        return (o * w_o).sum() + (ht * w_h).sum()

    ins = [x.clone().requires_grad_(True) for x in (q, k, v, g, beta, A_log, dt_bias, h0)]
    assert torch.autograd.gradcheck(f, ins, eps=1e-6, atol=1e-6, rtol=1e-4, fast_mode=True)


def test_kernel_mode_error_is_bf16_sized():
    """The bf16 rounding points move the gradients by ~3e-3 (relative RMS):
    the level the HIP backward is held to."""
    args, fkw = _case(1, 64, 2, 2, seed=21)
    ga = autograd_grads(*args, 0.1, **fkw)
    gk = chunked_backward(*args, 0.1, mode="kernel", **fkw)
    for n in (x for x in ga if x.startswith("d")):
        assert 1e-4 < _rel(gk[n], ga[n]) < 1.5e-2, n


def test_planted_mistake_is_caught(monkeypatch):
    """Drop the reverse cumsum of the gate gradient (a plausible slip): the
    restatement must then disagree with the gold on dg."""
    args, fkw = _case(1, 40, 2, 2, seed=4)
    ga = autograd_grads(*args, 0.1, **fkw)
    monkeypatch.setattr(kda_oracle_bwd, "_revcumsum", lambda x, dim: x)
    gc = chunked_backward(*args, 0.1, **fkw)
    assert _rel(gc["dg"], ga["dg"]) > 1e-2

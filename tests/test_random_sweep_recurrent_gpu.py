"""A seeded random sweep of the token recurrence on the GPU
(kda_recurrent_fwd), beyond the hand-picked cases of
tests/test_recurrent_gpu.py: batch rows, lengths 1-40, grouped value heads,
packed sequences (some empty), both state layouts, fp32 or bf16 gates, with
and without an initial state, and three flag sets (every in-kernel flag;
no beta sigmoid; the raw per-token log decay without l2norm or sigmoid).
Each case checks the fp32 output and final state against the oracle's fp32
recurrence with the bars of tests/test_recurrent_gpu.py (relative RMS at
most 1e-5, max-abs at most 1e-4 of the output's scale; only the summation
order differs), and the bf16 output against the fp32 one rounded to
nearest even, bit for bit.  The case list is drawn from a fixed seed.
"""

from __future__ import annotations

import random

import pytest
import torch

from kda_bt16 import kda_recurrent_fwd
from kda_oracle import per_sequence, recurrent_gold
from kda_testlib import assert_close_rel, maxdiff
from test_recurrent_gpu import _inputs

pytestmark = pytest.mark.gpu

N_CASES = 40
FLAG_SETS = (dict(gate=True, l2=True, sig=True), dict(gate=True, l2=True, sig=False),
             dict(gate=False, l2=False, sig=False))


def _draw_cases():
    rng = random.Random(77)
    cases = []
    for i in range(N_CASES):
        varlen = rng.random() < 0.25
        H = rng.choice([1, 2])
        T = rng.randint(1, 40)
        c = dict(name=f"rec{i:03d}", B=1 if varlen else rng.choice([1, 2, 3]), T=T, H=H,
                 HV=H * rng.choice([1, 2]), seed=rng.randrange(1 << 30),
                 h0=rng.choice([0.0, 0.05]), svf=rng.random() < 0.5,
                 gate_dtype=rng.choice([torch.float32, torch.bfloat16]),
                 flags=rng.choice(FLAG_SETS), cu=None)
        if varlen:
            cuts = sorted(rng.randint(0, T) for _ in range(rng.randint(0, 4)))
            c["cu"] = [0] + cuts + [T]
        cases.append(c)
    return cases


CASES = _draw_cases()


@pytest.mark.parametrize("c", CASES, ids=[c["name"] for c in CASES])
def test_random_recurrent_case(c, gpu_device):
    dev = gpu_device
    print(f"recurrent sweep {c}", flush=True)
    f = c["flags"]
    S = c["B"] if c["cu"] is None else len(c["cu"]) - 1
    x = _inputs(c["B"], c["T"], c["H"], c["HV"], c["seed"], h0_std=0.0, gate_dtype=c["gate_dtype"],
                small=not f["l2"])
    h0 = None
    if c["h0"] > 0:
        gen = torch.Generator().manual_seed(c["seed"] + 1)
        h0 = torch.randn(S, c["HV"], 128, 128, generator=gen) * c["h0"]
        if not c["svf"]:
            h0 = h0.transpose(-1, -2).contiguous()
    # without the in-kernel gate, g is the per-token log decay (negative)
    if f["gate"]:
        g = x["g"]
    else:
        gen = torch.Generator().manual_seed(c["seed"] + 2)
        g = (-torch.rand(x["g"].shape, generator=gen) * 0.3).to(x["g"].dtype)
    cu = None if c["cu"] is None else torch.tensor(c["cu"], dtype=torch.int32, device=dev)
    kw = dict(scale=0.1, initial_state=None if h0 is None else h0.to(dev), output_final_state=True,
              use_qk_l2norm_in_kernel=f["l2"], use_gate_in_kernel=f["gate"],
              use_beta_sigmoid_in_kernel=f["sig"], lower_bound=-5.0, A_log=x["A_log"].to(dev),
              dt_bias=x["dt_bias"].to(dev), state_v_first=c["svf"], cu_seqlens=cu)
    ins = [t.to(dev) for t in (x["q"], x["k"], x["v"], g, x["beta"])]
    o, ht = kda_recurrent_fwd(*ins, output_dtype=torch.float32, **kw)
    o16, ht16 = kda_recurrent_fwd(*ins, output_dtype=torch.bfloat16, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o16, o.to(torch.bfloat16)) and torch.equal(ht16, ht), c["name"]
    gkw = dict(A_log=x["A_log"], dt_bias=x["dt_bias"], lower_bound=-5.0, state_v_first=c["svf"],
               use_gate=f["gate"], use_l2norm=f["l2"], use_beta_sigmoid=f["sig"],
               gate_log=not f["gate"], dtype=torch.float32)
    args = (x["q"], x["k"], x["v"], g.float(), x["beta"].float())
    if c["cu"] is None:
        o_g, ht_g = recurrent_gold(*args, 0.1, initial_state=h0, **gkw)
    else:
        o_g, ht_g = per_sequence(recurrent_gold, *args, c["cu"], 0.1, initial_state=h0, **gkw)
    o, ht = o.cpu(), ht.cpu()
    assert torch.isfinite(o).all() and torch.isfinite(ht).all(), c["name"]
    assert_close_rel(f"{c['name']} o", o_g, o, 1e-5)
    assert_close_rel(f"{c['name']} ht", ht_g, ht, 1e-5)
    assert maxdiff(o, o_g) <= 1e-4 * max(o_g.abs().max().item(), 1e-3), c["name"]
    assert maxdiff(ht, ht_g) <= 1e-4 * max(ht_g.abs().max().item(), 1e-3), c["name"]

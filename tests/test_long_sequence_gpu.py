"""One sequence of 2^20 tokens (65536 chunks, 1.1 GB of stage-1 records for
one value head), far beyond the BASELINE lengths: every index and buffer
size along a single sequence-head stream at that scale.

* the two stages and the fused kernel give the same o and final state, bit
  for bit;
* the resume invariant: the forward split at a chunk boundary (token 2^19,
  the first half's final state as the second half's initial state) equals
  the whole, bit for bit;
* the first 2^16 tokens of o equal a forward over those tokens alone, bit
  for bit, and that forward is within the reference tests' tolerance of the
  CPU oracle (relative RMS 0.006, tests/test_kda_bt16.py:78-79; the oracle
  over all 2^20 tokens would take minutes on the host);
* the whole o and final state against the fp32 token recurrence on the GPU
  (pinned against the CPU fp32 gold in tests/test_recurrent_gpu.py):
  relative RMS at most 0.006.
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import forward_choice, kda_bt16_fwd, kda_recurrent_fwd
from kda_oracle import chunked_reference, make_inputs
from kda_testlib import assert_close_rel

pytestmark = pytest.mark.gpu

T_LONG = 1 << 20
T_PREFIX = 1 << 16
LB = -5.0
SCALE = 128 ** -0.5


def test_one_sequence_of_a_million_tokens(gpu_device):
    dev = gpu_device
    print(f"long sequence: B=1 T={T_LONG} H=1", flush=True)
    c = make_inputs(1, T_LONG, 1, seed=2024, h0_std=0.05)
    x = [c[n].to(dev) for n in ("q", "k", "v", "g", "beta")]
    h0 = c["h0"].to(dev)
    kw = dict(scale=SCALE, output_final_state=True, use_qk_l2norm_in_kernel=True,
              use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, lower_bound=LB,
              A_log=c["A_log"].to(dev), dt_bias=c["dt_bias"].to(dev))

    with forward_choice(fused=False):
        o, ht = kda_bt16_fwd(*x, initial_state=h0, **kw)
    with forward_choice(fused=True):
        o_f, ht_f = kda_bt16_fwd(*x, initial_state=h0, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all() and torch.isfinite(ht).all()
    assert torch.equal(o, o_f) and torch.equal(ht, ht_f), "fused differs from two stages"
    del o_f, ht_f

    half = T_LONG // 2
    oa, hta = kda_bt16_fwd(*(t[:, :half].contiguous() for t in x), initial_state=h0, **kw)
    ob, htb = kda_bt16_fwd(*(t[:, half:].contiguous() for t in x), initial_state=hta, **kw)
    torch.cuda.synchronize()
    assert torch.equal(oa, o[:, :half]) and torch.equal(ob, o[:, half:]), "resume: o differs"
    assert torch.equal(htb, ht), "resume: final state differs"
    del oa, hta, ob, htb

    op, htp = kda_bt16_fwd(*(t[:, :T_PREFIX].contiguous() for t in x), initial_state=h0, **kw)
    torch.cuda.synchronize()
    assert torch.equal(op, o[:, :T_PREFIX]), "prefix: o differs from the long call's"
    o_r, ht_r, _ = chunked_reference(
        *(c[n][:, :T_PREFIX] for n in ("q", "k", "v")), c["g"][:, :T_PREFIX].float(),
        c["beta"][:, :T_PREFIX].float(), SCALE, A_log=c["A_log"], dt_bias=c["dt_bias"],
        lower_bound=LB, initial_state=c["h0"])
    assert_close_rel("prefix o vs oracle", o_r.float(), op.float().cpu(), 0.006)
    assert_close_rel("prefix ht vs oracle", ht_r, htp.cpu(), 0.006)
    del op, htp

    o_g, ht_g = kda_recurrent_fwd(*x, initial_state=h0, output_dtype=torch.float32, **kw)
    torch.cuda.synchronize()
    assert_close_rel("o vs fp32 recurrence", o_g.cpu(), o.float().cpu(), 0.006)
    assert_close_rel("ht vs fp32 recurrence", ht_g.cpu(), ht.cpu(), 0.006)

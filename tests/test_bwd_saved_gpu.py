"""GPU checks of the training forward that keeps its state
(kda_bt16_fwd_save_hip) and the backward that starts from it
(kda_bt16_bwd_saved_hip), the autograd node's default policy.

The oracle-parity of the gradients is covered by test_bwd_gpu.py through the
recompute entry point (kda_bt16_bwd_hip); this file pins the saved-state path
to that one and to the plain forward, bit for bit: the same kernels' math
runs in both, only the place of the per-chunk state differs.
"""

from __future__ import annotations

import pytest
import torch

from kda_oracle import make_inputs

pytestmark = pytest.mark.gpu

LEAVES = ("q", "k", "v", "g", "beta", "A_log", "dt_bias", "h0")

# name, B, T, H, HV, cu_seqlens, options
CASES = [
    ("fixed_T64", 2, 64, 2, 2, None, {}),
    ("ragged_T50_gva", 2, 50, 1, 2, None, {}),
    ("varlen_empty_seqs", 1, 120, 2, 2, [0, 0, 37, 53, 53, 120], {}),
    ("fp32_gate_kfirst_no_h0", 1, 40, 2, 2, None,
     {"gate_dtype": torch.float32, "svf": False, "h0": False}),
    ("no_bias", 1, 80, 2, 4, None, {"bias": False}),
]


def _setup(B, T, H, HV, cu, opts, dev):
    gdt = opts.get("gate_dtype", torch.bfloat16)
    N = B if cu is None else len(cu) - 1
    c = make_inputs(B, T, HV, seed=5, h0_std=0.05, gate_dtype=gdt)
    x = {n: c[n] for n in ("v", "g", "beta", "A_log", "dt_bias")}
    x["q"] = c["q"][:, :, :H].contiguous()
    x["k"] = c["k"][:, :, :H].contiguous()
    gen = torch.Generator().manual_seed(11)
    x["h0"] = None
    if opts.get("h0", True):
        h0 = torch.randn(N, HV, 128, 128, generator=gen) * 0.05
        x["h0"] = h0
    if not opts.get("bias", True):
        x["dt_bias"] = None
    dos = [torch.randn(B, T, HV, 128, generator=gen).to(torch.bfloat16).to(dev) for _ in range(2)]
    dhts = [(torch.randn(N, HV, 128, 128, generator=gen) * 0.1).to(dev) for _ in range(2)]
    return x, dos, dhts


def _forward(x, cu, opts, dev, grad):
    from kda_bt16 import kda_bt16_fwd

    leaves = {n: (None if t is None else t.to(dev).requires_grad_(grad)) for n, t in x.items()}
    o, ht = kda_bt16_fwd(
        leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["beta"], 0.1,
        initial_state=leaves["h0"], output_final_state=True, use_qk_l2norm_in_kernel=True,
        use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, lower_bound=-5.0,
        A_log=leaves["A_log"], dt_bias=leaves["dt_bias"], state_v_first=opts.get("svf", True),
        cu_seqlens=None if cu is None else torch.tensor(cu, dtype=torch.int32, device=dev))
    return leaves, o, ht


def _grads(leaves, o, ht, do, dht, retain):
    live = [n for n in LEAVES if leaves[n] is not None]
    loss = (o.float() * do.float()).sum() + (ht * dht).sum()
    gs = torch.autograd.grad(loss, [leaves[n] for n in live], retain_graph=retain)
    return dict(zip(live, gs))


@pytest.mark.parametrize("name,B,T,H,HV,cu,opts", CASES, ids=[c[0] for c in CASES])
def test_saved_state_matches_recompute(gpu_device, name, B, T, H, HV, cu, opts):
    """o and ht of the training forward equal the plain forward's; the
    gradients from the saved state equal the recompute path's, for two
    backward calls in a row over one saved state (dO differs between them)."""
    from kda_bt16 import set_backward_recompute

    dev = gpu_device
    print(f"[saved-state] {name}: B={B} T={T} H={H} HV={HV} cu={cu}", flush=True)
    x, dos, dhts = _setup(B, T, H, HV, cu, opts, dev)
    with torch.no_grad():
        _, o_ref, ht_ref = _forward(x, cu, opts, dev, grad=False)
    try:
        set_backward_recompute(False)
        leaves, o, ht = _forward(x, cu, opts, dev, grad=True)
        saved = [_grads(leaves, o, ht, dos[i], dhts[i], retain=(i == 0)) for i in range(2)]
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(ht, ht_ref)
        set_backward_recompute(True)
        leaves, o2, ht2 = _forward(x, cu, opts, dev, grad=True)
        recomputed = [_grads(leaves, o2, ht2, dos[i], dhts[i], retain=(i == 0)) for i in range(2)]
        torch.cuda.synchronize()
    finally:
        set_backward_recompute(False)
    assert torch.equal(o2, o_ref) and torch.equal(ht2, ht_ref)
    for i in range(2):
        for n, gr in recomputed[i].items():
            assert torch.isfinite(gr.float()).all(), (i, n)
            assert torch.equal(saved[i][n], gr), (i, n)


def test_saved_state_is_freed_after_backward_while_o_lives(gpu_device):
    """The per-chunk state goes through save_for_backward: autograd frees it
    when the backward has run, although o (and its grad_fn) stay alive."""
    from kda_bt16 import _hip, kda_bt16_fwd
    from kda_bt16.kernels import _flags, _make_args

    dev = gpu_device
    B, T, H = 1, 2048, 8
    c = make_inputs(B, T, H, seed=9)
    leaves = {n: c[n].to(dev).requires_grad_(True) for n in ("q", "k", "v", "g", "beta", "A_log")}
    args = _make_args(leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["beta"], 0.1,
                      -5.0, leaves["A_log"], None, None, leaves["v"], None, None, 0,
                      _flags(True, True, True, True))
    saved_bytes = _hip.saved_bytes(args)
    assert saved_bytes > 32 << 20  # ~55 KiB per record slot, 1024 slots
    torch.cuda.synchronize()
    o, _ = kda_bt16_fwd(leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["beta"], 0.1,
                        use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                        use_beta_sigmoid_in_kernel=True, lower_bound=-5.0, A_log=leaves["A_log"])
    torch.cuda.synchronize()
    state = [t for t in o.grad_fn.saved_tensors if t is not None and t.dtype == torch.uint8]
    assert len(state) == 1 and state[0].numel() == saved_bytes
    del state
    held = torch.cuda.memory_allocated(dev)
    o.backward(torch.ones_like(o))
    torch.cuda.synchronize()
    after = torch.cuda.memory_allocated(dev)
    # autograd has released what the node saved, the state included ...
    with pytest.raises(RuntimeError, match="freed"):
        _ = o.grad_fn.saved_tensors
    # ... and its memory: the gradients were allocated, the state freed
    # (2 MiB of slack for buffers torch keeps after a first backward)
    grads = sum(t.grad.numel() * t.grad.element_size() for t in leaves.values())
    assert held + grads - after >= saved_bytes - (1 << 21), (held, after, grads, saved_bytes)

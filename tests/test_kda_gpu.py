"""Parity of the HIP path (through kda_bt16_fwd / kda_bt16_debug -> C ABI ->
gfx950 kernels) with the CPU oracle and the fp32 recurrent gold.

Bars (the tolerance each test applies is written in it):
* vs the fp32 recurrent gold: max-abs error of o and ht no worse than 1.5x
  the reference chunked path's own error on the same inputs (the oracle in
  kernel mode restates that path), plus 1e-5 slack;
* vs the oracle: FLA-style relative-RMS ratio <= 0.006 on o and ht (the
  reference's own tolerance vs its gold, tests/test_kda_bt16.py:78-79) and
  max-abs <= 1e-2 (tests/test_torch_reference.py:289-290);
* stage-1 intermediates within a few bf16 ulps of the oracle's.
"""

from __future__ import annotations

import pytest
import torch

from kda_bt16 import kda_bt16_debug, kda_bt16_fwd
from kda_oracle import chunked_reference, make_inputs, recurrent_gold
from kda_testlib import GOLDEN_CASES, assert_close_rel, load_golden, maxdiff

pytestmark = pytest.mark.gpu


def _hip(c, dev, **over):
    cfg = dict(
        scale=c.get("scale", 0.1), initial_state=None, output_final_state=True,
        use_qk_l2norm_in_kernel=True, use_gate_in_kernel=c.get("use_gate", True),
        use_beta_sigmoid_in_kernel=True, lower_bound=c.get("lower_bound", -5.0),
        A_log=c["A_log"].to(dev), dt_bias=None if c["dt_bias"] is None else c["dt_bias"].to(dev),
        state_v_first=c.get("state_v_first", True),
    )
    if c.get("h0") is not None:
        cfg["initial_state"] = c["h0"].to(dev)
    cfg.update(over)
    args = [c[x].to(dev) for x in ("q", "k", "v", "g", "beta")]
    return args, cfg


def _oracle(c, *, mode="kernel", **over):
    cfg = dict(
        A_log=c["A_log"], dt_bias=c["dt_bias"], lower_bound=c.get("lower_bound", -5.0),
        initial_state=c.get("h0"), state_v_first=c.get("state_v_first", True),
        use_gate=c.get("use_gate", True),
    )
    cfg.update(over)
    return chunked_reference(c["q"], c["k"], c["v"], c["g"].float(), c["beta"].float(),
                             c.get("scale", 0.1), mode=mode, **cfg)


def _gold(c, **over):
    cfg = dict(
        A_log=c["A_log"], dt_bias=c["dt_bias"], lower_bound=c.get("lower_bound", -5.0),
        initial_state=c.get("h0"), state_v_first=c.get("state_v_first", True),
        use_gate=c.get("use_gate", True),
    )
    cfg.update(over)
    return recurrent_gold(c["q"], c["k"], c["v"], c["g"].float(), c["beta"].float(),
                          c.get("scale", 0.1), dtype=torch.float32, **cfg)


def _check_full(c, o, ht, *, gold=True, label=""):
    o_ref, ht_ref, _ = _oracle(c)
    o, ht = o.float().cpu(), ht.cpu()
    assert torch.isfinite(o).all() and torch.isfinite(ht).all(), label
    assert_close_rel(f"{label} o vs oracle", o_ref.float(), o, 0.006)
    assert_close_rel(f"{label} ht vs oracle", ht_ref, ht, 0.006)
    assert maxdiff(o, o_ref.float()) < 1e-2, label
    assert maxdiff(ht, ht_ref) < 1e-2, label
    if gold:
        o_g, ht_g = _gold(c)
        bar_o = 1.5 * maxdiff(o_ref.float(), o_g) + 1e-5
        bar_h = 1.5 * maxdiff(ht_ref, ht_g) + 1e-5
        do, dh = maxdiff(o, o_g), maxdiff(ht, ht_g)
        print(f"{label}: o {do:.3e} (bar {bar_o:.3e})  ht {dh:.3e} (bar {bar_h:.3e})", flush=True)
        assert do <= bar_o, f"{label}: o vs gold {do:.3e} > 1.5x reference-path error {bar_o:.3e}"
        assert dh <= bar_h, f"{label}: ht vs gold {dh:.3e} > 1.5x reference-path error {bar_h:.3e}"


@pytest.mark.parametrize("B,T,H", [(1, 1, 1), (1, 16, 1), (1, 17, 1), (1, 32, 2), (1, 33, 2),
                                   (2, 64, 4), (2, 1037, 4), (1, 512, 8)])
def test_shapes_vs_oracle_and_gold(B, T, H, gpu_device):
    c = make_inputs(B, T, H, seed=1000 + T, h0_std=0.05)
    args, cfg = _hip(c, gpu_device)
    o, ht = kda_bt16_fwd(*args, **cfg)
    torch.cuda.synchronize()
    _check_full(c, o, ht, label=f"B{B} T{T} H{H}")


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_golden_fixtures(name, gpu_device):
    c = load_golden(name)
    args, cfg = _hip(c, gpu_device, scale=c["scale"])
    o, ht = kda_bt16_fwd(*args, **cfg)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all() and torch.isfinite(ht).all()
    # reference tolerance vs gold: 0.006 (0.02 for the saturated gate,
    # tests/test_kda_bt16.py:170-171)
    tol = 0.02 if name.startswith("saturated") else 0.006
    assert_close_rel("o", c["o_gold"], o.float().cpu(), tol)
    assert_close_rel("ht", c["ht_gold"], ht.cpu(), tol)
    _check_full(c, o, ht, label=name)


def test_debug_intermediates_vs_oracle(gpu_device):
    c = make_inputs(2, 71, 3, seed=5, h0_std=0.05)
    args, cfg = _hip(c, gpu_device)
    o, ht, dbg = kda_bt16_debug(*args, **cfg)
    torch.cuda.synchronize()
    _, _, ref = _oracle(c)
    assert set(dbg) == {"Aqk", "A_inv", "w", "u", "g"}
    assert dbg["Aqk"].dtype == torch.bfloat16 and dbg["g"].dtype == torch.float32
    assert maxdiff(dbg["g"], ref["g"]) < 1e-4
    for key in ("Aqk", "A_inv", "w", "u"):
        got, want = dbg[key].float().cpu(), ref[key].float()
        assert got.shape == want.shape, key
        # a few bf16 ulps (2^-8 relative) of the largest element
        tol = 3 * 2.0 ** -8 * want.abs().max().item()
        assert maxdiff(got, want) <= tol, f"{key}: {maxdiff(got, want):.3e} > {tol:.3e}"
    o2, ht2 = kda_bt16_fwd(*args, **cfg)
    assert torch.equal(o, o2) and torch.equal(ht, ht2)


@pytest.mark.parametrize("T", [16, 17])
@pytest.mark.parametrize("state_v_first", [True, False])
def test_initial_state_layouts(T, state_v_first, gpu_device):
    """tests/test_torch_reference.py:390-476: non-zero h0 in both layouts."""
    c = make_inputs(1, T, 1, seed=456 + T, h0_std=1.0)
    if not state_v_first:
        c["h0"] = c["h0"].transpose(-1, -2).contiguous()
    c["state_v_first"] = state_v_first
    args, cfg = _hip(c, gpu_device)
    o, ht = kda_bt16_fwd(*args, **cfg)
    torch.cuda.synchronize()
    _check_full(c, o, ht, label=f"h0 T{T} vfirst={state_v_first}")


def test_kfirst_equals_vfirst_transposed(gpu_device):
    c = make_inputs(2, 80, 2, seed=77, h0_std=0.05)
    args, cfg = _hip(c, gpu_device)
    o1, ht1 = kda_bt16_fwd(*args, **cfg)
    cfg2 = dict(cfg, state_v_first=False,
                initial_state=cfg["initial_state"].transpose(-1, -2).contiguous())
    o2, ht2 = kda_bt16_fwd(*args, **cfg2)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert torch.equal(ht1, ht2.transpose(-1, -2))


@pytest.mark.parametrize("lower_bound", [-8.0, -10.0])
def test_saturated_gate_no_overflow(lower_bound, gpu_device):
    """tests/test_kda_bt16.py:128-171: sigmoid pinned to 1, gate = lower_bound."""
    c = make_inputs(1, 128, 4, seed=42)
    c["A_log"] = torch.zeros(4)
    c["dt_bias"] = torch.zeros(4 * 128)
    c["g"] = torch.full((1, 128, 4, 128), 20.0)
    c["beta"] = c["beta"].float()
    c["lower_bound"] = lower_bound
    args, cfg = _hip(c, gpu_device)
    o, ht = kda_bt16_fwd(*args, **cfg)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all() and torch.isfinite(ht).all()
    o_g, ht_g = _gold(c)
    assert_close_rel("o", o_g, o.float().cpu(), 0.02)
    assert_close_rel("ht", ht_g, ht.cpu(), 0.02)


def test_flag_combinations(gpu_device):
    """Every in-kernel flag off in turn, no dt_bias, fp32 and bf16 g/beta."""
    base = make_inputs(1, 50, 2, seed=8, h0_std=0.05)
    variants = [
        dict(),
        dict(use_qk_l2norm_in_kernel=False),
        dict(use_beta_sigmoid_in_kernel=False),
        dict(dt_bias=None),
        dict(fp32_gate=True),
    ]
    for var in variants:
        c = dict(base)
        over = dict(var)
        if over.pop("fp32_gate", False):
            c["g"] = c["g"].float()
            c["beta"] = c["beta"].float()
        if "dt_bias" in over:
            c["dt_bias"] = None
            over.pop("dt_bias")
        if over.get("use_qk_l2norm_in_kernel") is False:
            # unnormalised q/k of norm ~11 would blow the recurrence up; scale down
            c["q"] = (c["q"].float() / 12).bfloat16()
            c["k"] = (c["k"].float() / 12).bfloat16()
        if over.get("use_beta_sigmoid_in_kernel") is False:
            c["beta"] = torch.sigmoid(c["beta"].float())
        args, cfg = _hip(c, gpu_device, **over)
        o, ht = kda_bt16_fwd(*args, **cfg)
        torch.cuda.synchronize()
        ocfg = {}
        if over.get("use_qk_l2norm_in_kernel") is False:
            ocfg["use_l2norm"] = False
        if over.get("use_beta_sigmoid_in_kernel") is False:
            ocfg["use_beta_sigmoid"] = False
        o_ref, ht_ref, _ = _oracle(c, **ocfg)
        assert_close_rel(f"{var} o", o_ref.float(), o.float().cpu(), 0.006)
        assert_close_rel(f"{var} ht", ht_ref, ht.cpu(), 0.006)


def test_precomputed_gate_matches_in_kernel_gate(gpu_device):
    """use_gate_in_kernel=False fed with the stage-1 log2 cumsum (the debug
    'g' output) reproduces the in-kernel-gate result."""
    c = make_inputs(2, 96, 2, seed=12, h0_std=0.05)
    args, cfg = _hip(c, gpu_device)
    o1, ht1, dbg = kda_bt16_debug(*args, **cfg)
    args2 = list(args)
    args2[3] = dbg["g"]
    o2, ht2 = kda_bt16_fwd(*args2, **dict(cfg, use_gate_in_kernel=False))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert torch.equal(ht1, ht2)


def test_fused_flag_and_reuse_workspace(gpu_device):
    c = make_inputs(1, 64, 4, seed=2, h0_std=0.05)
    args, cfg = _hip(c, gpu_device)
    o1, ht1 = kda_bt16_fwd(*args, **cfg)
    o2, ht2 = kda_bt16_fwd(*args, use_fused_kernel=True, **cfg)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(ht1, ht2)
    # reuse_workspace=True: outputs alias a module cache (kernels.py:525-536)
    o3, ht3 = kda_bt16_fwd(*args, reuse_workspace=True, **cfg)
    o4, ht4 = kda_bt16_fwd(*args, reuse_workspace=True, **cfg)
    torch.cuda.synchronize()
    assert o3.data_ptr() == o4.data_ptr() and ht3.data_ptr() == ht4.data_ptr()
    assert torch.equal(o4, o1) and torch.equal(ht4, ht1)


def test_no_final_state_and_default_scale(gpu_device):
    c = make_inputs(2, 128, 4, seed=3)
    args, cfg = _hip(c, gpu_device, scale=None, output_final_state=False)
    o, ht = kda_bt16_fwd(*args, **cfg)
    torch.cuda.synchronize()
    assert ht is None
    o_ref, _, _ = chunked_reference(c["q"], c["k"], c["v"], c["g"].float(), c["beta"].float(), None,
                                    A_log=c["A_log"], dt_bias=c["dt_bias"])
    assert_close_rel("o", o_ref.float(), o.float().cpu(), 0.006)


def test_repeat_calls_bit_identical(gpu_device):
    """Stability: N calls on the same inputs are bit-identical and finite
    (pattern of the reference's stability gate)."""
    c = make_inputs(1, 300, 8, seed=4, h0_std=0.05)
    args, cfg = _hip(c, gpu_device)
    o0, ht0 = kda_bt16_fwd(*args, **cfg)
    for _ in range(10):
        o, ht = kda_bt16_fwd(*args, **cfg)
        assert torch.equal(o, o0) and torch.equal(ht, ht0)
    assert torch.isfinite(o0.float()).all()


def test_stream_ordering_on_side_stream(gpu_device):
    """The launch follows torch's current stream."""
    c = make_inputs(1, 200, 4, seed=6, h0_std=0.05)
    args, cfg = _hip(c, gpu_device)
    o_ref, ht_ref = kda_bt16_fwd(*args, **cfg)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        o, ht = kda_bt16_fwd(*args, **cfg)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(ht, ht_ref)


@pytest.mark.parametrize("dt", [torch.float16, torch.float64])
def test_precomputed_g_of_other_float_dtypes(dt, gpu_device):
    """kernels.py:673-674, 108: without the in-kernel gate the reference
    takes g of any dtype and widens it to fp32 at load.  The result equals
    the call with that widening done by hand, bit for bit, and the gradient
    comes back in g's dtype."""
    c = make_inputs(1, 70, 2, seed=31, h0_std=0.05)
    gen = torch.Generator().manual_seed(3)
    gate = -5.0 * torch.sigmoid(torch.randn(1, 80, 2, 128, generator=gen))
    g = (torch.cumsum(gate.view(1, 5, 16, 2, 128), 2) * 1.4426950216).view(1, 80, 2, 128)[:, :70]
    g = g.contiguous().to(dt)
    args, cfg = _hip(c, gpu_device, use_gate_in_kernel=False)
    args[3] = g.to(gpu_device)
    o1, ht1 = kda_bt16_fwd(*args, **cfg)
    args2 = list(args)
    args2[3] = g.to(gpu_device).float()
    o2, ht2 = kda_bt16_fwd(*args2, **cfg)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(ht1, ht2)
    gl = args[3].clone().requires_grad_(True)
    o3, _ = kda_bt16_fwd(args[0], args[1], args[2], gl, args[4], **cfg)
    o3.float().sum().backward()
    assert gl.grad.dtype == dt and torch.isfinite(gl.grad.double()).all()

"""Write ``tests/golden/kda_ref_fixtures.npz``: inputs and outputs of the
reference's own chunked path, produced by running its Triton kernels
(``/root/reference/src/kda_bt16/kernels.py``: ``kda_bt16_debug``, i.e.
``kda_bt16_kernel_k1`` and ``kda_bt16_kernel_k2``) on the CPU under Triton's
interpreter (``TRITON_INTERPRET=1``).

Run in the build container only (it needs /root/reference and Triton; the
GPU box never runs it, only the .npz travels):

    python tests/golden/make_ref_fixtures.py

What the fixtures pin: the oracle's restatement of the reference's rounding
points (``oracle/kda_oracle.py``, tests/test_oracle_ref.py) and the HIP
path's stage-1 intermediates and outputs (tests/test_ref_fixtures_gpu.py).

Two passes per case, stored under separate keys:

* ``interp/``: the interpreter as installed.  Its fp32 work is faithful, so
  ``g`` (the gate cumsum), ``Aqk`` and ``A_inv`` (fp32 grams and solve,
  stored bf16) are the reference's values.  Its bf16 ``tl.dot`` is not:
  Triton 3.6's interpreter stores bf16 tensors as their uint16 bit patterns
  and ``create_dot`` multiplies those patterns as integers
  (``triton/runtime/interpreter.py``, ``InterpreterBuilder.create_dot``), so
  ``w``, ``u`` (kernels.py:171-176) and everything stage 2 computes
  (kernels.py:261-291) come out near 1e10 and are not stored from this pass.
* ``dotfix/``: the same run with that one function corrected: bf16 operands
  of ``tl.dot`` are widened to fp32 (exact: a bf16 value is the top half of
  its fp32) before the interpreter's own fp32 matmul.  That is the bf16 dot
  the reference asks for (exact products, fp32 accumulation; only the
  summation order is numpy's).  Nothing else in Triton or the reference is
  touched.  ``w``, ``u``, ``o`` and ``ht`` are stored from this pass, and
  ``g``, ``Aqk``, ``A_inv`` must come out bit-identical to ``interp/``
  (checked here).

The reference validates fp32 ``g`` and ``beta`` (kernels.py:673-676): the
cases pass them as fp32, and bf16 q, k, v.  No bytecode is written into the
reference tree.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"
sys.dont_write_bytecode = True  # nothing may be written under /root/reference

import numpy as np  # noqa: E402
import torch  # noqa: E402

REF_SRC = Path("/root/reference/src")
OUT = Path(__file__).resolve().parent / "kda_ref_fixtures.npz"
RCP_LN2 = 1.4426950216


def _bits(x: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> its uint16 bit patterns."""
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


def _case(name, B, T, H, seed, *, lb=-5.0, g_std=1.0, h0_std=0.0, svf=True, use_gate=True,
          l2norm=True, bsig=True, scale=None):
    gen = torch.Generator().manual_seed(seed)
    qk_scale = 1.0 if l2norm else 128 ** -0.5  # unnormalised rows of norm ~1
    q = (torch.randn(B, T, H, 128, generator=gen) * qk_scale).to(torch.bfloat16)
    k = (torch.randn(B, T, H, 128, generator=gen) * qk_scale).to(torch.bfloat16)
    v = torch.randn(B, T, H, 128, generator=gen).to(torch.bfloat16)
    graw = torch.randn(B, T, H, 128, generator=gen) * g_std
    beta = torch.randn(B, T, H, generator=gen) if bsig else torch.rand(B, T, H, generator=gen)
    A_log = torch.log(torch.rand(H, generator=gen) * 15.0 + 1.0)
    dt_bias = torch.randn(H * 128, generator=gen) * 0.1
    h0 = None
    if h0_std:  # bf16-valued, so the fixture stores it in 2 bytes per element
        h0 = (torch.randn(B, H, 128, 128, generator=gen) * h0_std).bfloat16().float()
    if not use_gate:
        # the precomputed-gate contract: g is the chunk-local log2 cumsum of
        # per-token gates in [lb, 0]
        gate = lb * torch.sigmoid(graw)
        NT = -(-T // 16)
        pad = NT * 16 - T
        gp = torch.cat([gate, gate.new_zeros(B, pad, H, 128)], 1).view(B, NT, 16, H, 128)
        g = (torch.cumsum(gp, 2) * RCP_LN2).view(B, NT * 16, H, 128)[:, :T].contiguous()
    else:
        g = graw
    return dict(name=name, q=q, k=k, v=v, g=g.float(), beta=beta.float(), A_log=A_log,
                dt_bias=dt_bias, h0=h0, lb=lb, svf=svf, use_gate=use_gate, l2norm=l2norm,
                bsig=bsig, scale=0.1 if scale is None else scale)


CASES = [
    _case("t1", 1, 1, 1, seed=1, h0_std=0.05),
    _case("t16", 1, 16, 1, seed=2),
    _case("t17_h0", 1, 17, 1, seed=3, h0_std=0.05),
    _case("t37_b2_h0", 2, 37, 2, seed=4, h0_std=0.05),
    _case("t64_seed42", 1, 64, 2, seed=42, scale=128 ** -0.5),
    _case("sat_lb10", 1, 33, 2, seed=5, lb=-10.0, g_std=2.0, h0_std=0.05),
    _case("precomputed_g", 1, 37, 2, seed=6, use_gate=False, h0_std=0.05),
    _case("kfirst_h0", 1, 40, 2, seed=7, h0_std=0.05, svf=False),
    _case("no_l2norm_no_sigmoid", 1, 33, 2, seed=8, l2norm=False, bsig=False),
]


def _run(ref, c):
    h0 = c["h0"]
    if h0 is not None and not c["svf"]:
        h0 = h0.transpose(-1, -2).contiguous()  # the K-first layout's state
    o, ht, dbg = ref.kda_bt16_debug(
        c["q"], c["k"], c["v"], c["g"], c["beta"], scale=c["scale"], initial_state=h0,
        output_final_state=True, use_qk_l2norm_in_kernel=c["l2norm"],
        use_gate_in_kernel=c["use_gate"], use_beta_sigmoid_in_kernel=c["bsig"],
        lower_bound=c["lb"], A_log=c["A_log"], dt_bias=c["dt_bias"], state_v_first=c["svf"],
    )
    return o, ht, dbg, h0


def _fixed_dot(orig):
    """InterpreterBuilder.create_dot with bf16 operands widened to fp32."""
    from triton import language as tl
    from triton.runtime.interpreter import TensorHandle

    def widen(x):
        if x.dtype.scalar == tl.bfloat16:
            data = (x.data.astype(np.uint32) << 16).view(np.float32)
            return TensorHandle(data, tl.float32)
        return x

    def create_dot(self, a, b, d, input_precision, max_num_imprecise_acc):
        return orig(self, widen(a), widen(b), d, input_precision, max_num_imprecise_acc)

    return create_dot


def main() -> None:
    sys.path.insert(0, str(REF_SRC))
    from kda_bt16 import kernels as ref  # the reference itself, from /root/reference
    from triton.runtime import interpreter

    out: dict[str, np.ndarray] = {}
    for c in CASES:
        p = c["name"] + "/"
        o0, ht0, dbg0, h0 = _run(ref, c)
        orig = interpreter.InterpreterBuilder.create_dot
        interpreter.InterpreterBuilder.create_dot = _fixed_dot(orig)
        try:
            o1, ht1, dbg1, _ = _run(ref, c)
        finally:
            interpreter.InterpreterBuilder.create_dot = orig
        for key in ("g", "Aqk", "A_inv"):
            a, b = dbg0[key], dbg1[key]
            assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                               b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32)), \
                f"{c['name']}: {key} differs between the two passes"
        assert dbg1["w"].float().abs().max() < 1e3, "the dot fix did not take"
        # inputs
        for key in ("q", "k", "v"):
            out[p + key] = _bits(c[key])
        out[p + "g"] = c["g"].numpy()
        out[p + "beta"] = c["beta"].numpy()
        out[p + "A_log"] = c["A_log"].numpy()
        out[p + "dt_bias"] = c["dt_bias"].numpy()
        if h0 is not None:
            out[p + "h0"] = _bits(h0.bfloat16())  # in the case's state layout, bf16-exact
        out[p + "cfg"] = np.array([c["scale"], c["lb"], c["svf"], c["use_gate"], c["l2norm"],
                                   c["bsig"]], dtype=np.float64)
        # outputs of the unmodified interpreter
        out[p + "interp/g"] = dbg0["g"].numpy()
        out[p + "interp/Aqk"] = _bits(dbg0["Aqk"])
        out[p + "interp/A_inv"] = _bits(dbg0["A_inv"])
        # outputs of the bf16-dot-corrected interpreter
        out[p + "dotfix/w"] = _bits(dbg1["w"])
        out[p + "dotfix/u"] = _bits(dbg1["u"])
        out[p + "dotfix/o"] = _bits(o1)
        out[p + "dotfix/ht"] = ht1.numpy()
        print(f"{c['name']}: T={c['q'].shape[1]} |w| {dbg1['w'].float().abs().max():.3f} "
              f"|o| {o1.float().abs().max():.4f} |ht| {ht1.abs().max():.4f} "
              f"(buggy interpreter: |w| {dbg0['w'].float().abs().max():.3g})", flush=True)
    out["cases"] = np.array([c["name"] for c in CASES])
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()

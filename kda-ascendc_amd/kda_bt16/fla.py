"""FLA-convention entry points over the MI355X kernels: ``chunk_kda`` and
``fused_recurrent_kda`` with the arguments, defaults and return values of
flash-linear-attention's ``fla.ops.kda`` functions as the reference calls
them (``/root/reference/tests/test_kda_bt16.py:26-38, 84-99``,
``/root/reference/benchmarks/bench_fla_compare.py:100-111``).  The reference
lists the FLA integration as not yet done (``README.md:422-423, 510``).

FLA conventions that differ from :func:`kda_bt16.kda_bt16_fwd`:

* without ``use_gate_in_kernel``, ``g`` is the per-token natural-log decay
  (FLA forms its chunk-local log2 cumsum itself, ``kda_gate_chunk_cumsum``);
  here stage 1 forms it (``KDA_BT16_G_LOG_DECAY``);
* the state layout defaults to K-first (``state_v_first=False``), FLA's
  default, handled natively by stage 2;
* ``chunk_size`` is accepted for signature compatibility; the kernels use
  16-token chunks (results equal FLA's 64-token chunks to rounding, the
  reference's own check at 0.01, ``tests/test_kda_bt16.py:84-101``);
* ``cu_seqlens`` packs sequences along T with B == 1;
* ``chunk_kda`` is differentiable (autograd runs the HIP backward);
  ``fused_recurrent_kda`` is forward-only, like the token recurrence.

What this backend serves is :func:`verify_chunk_kda` /
:func:`verify_fused_recurrent_kda`'s bucket; outside it the functions raise
``NotImplementedError`` naming the reason, and the dispatcher
(:mod:`kda_bt16.dispatch`) routes such calls elsewhere.
"""

from __future__ import annotations

import torch

from .kernels import _check_max_seqlen, _fwd_maybe_autograd, _validate_kda_inputs, kda_recurrent_fwd

_LB_RANGE = (-11.0, 0.0)


def _lb_ok(lower_bound) -> bool:
    return lower_bound is not None and _LB_RANGE[0] < float(lower_bound) < _LB_RANGE[1]


def _common_reason(q, k, v, g, beta, allow_grad: bool = False) -> str | None:
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != torch.bfloat16:
            return f"{name} must be bfloat16, got {t.dtype}"
    if q.shape[-1] != 128 or v.shape[-1] != 128:
        return f"needs K=V=128, got K={q.shape[-1]}, V={v.shape[-1]}"
    if v.ndim != 4 or q.ndim != 4 or v.shape[2] % q.shape[2] != 0:
        return "needs HV a multiple of H"
    if g.dtype not in (torch.float32, torch.bfloat16) or beta.dtype not in (torch.float32, torch.bfloat16):
        return "g and beta must be float32 or bfloat16"
    if not allow_grad and torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (q, k, v, g, beta)):
        return "forward only: inputs require grad"
    return None


def _device_reason(q) -> str | None:
    return None if q.device.type == "cuda" else "tensors are not on a ROCm GPU"


def verify_chunk_kda(q, k, v, g, beta, *, use_gate_in_kernel=False, safe_gate=False,
                     lower_bound=None, A_log=None, return_intermediate_states=False,
                     cp_context=None, **_ignored) -> str | None:
    """``None`` if :func:`chunk_kda` serves this call, else the reason it
    does not.  The bucket: bf16 q/k/v, K = V = 128, HV a multiple of H
    (autograd included: the backward kernels serve it), no context
    parallelism or intermediate states, and a gate
    bounded below by ``lower_bound`` in (-11, 0): the in-kernel gate
    ``lower_bound * sigmoid(...)``, or a per-token log decay the caller
    guarantees to be >= lower_bound (FLA's ``safe_gate`` contract).  The
    unbounded softplus gate (``lower_bound=None``) is not served: a 16-token
    chunk's decay span would overflow fp32 (kernels.py:733-744)."""
    reason = _common_reason(q, k, v, g, beta, allow_grad=True)
    if reason:
        return reason
    if return_intermediate_states:
        return "return_intermediate_states is not supported"
    if cp_context is not None:
        return "context parallelism is not supported"
    if use_gate_in_kernel:
        if not _lb_ok(lower_bound):
            return "the in-kernel gate needs lower_bound in (-11, 0) (softplus gate not served)"
        if A_log is None:
            return "use_gate_in_kernel requires A_log"
    elif not (safe_gate and _lb_ok(lower_bound)):
        return "a precomputed log decay needs safe_gate=True and lower_bound in (-11, 0)"
    return _device_reason(q)


def verify_fused_recurrent_kda(q, k, v, g, beta, *, use_gate_in_kernel=False, lower_bound=None,
                               A_log=None, **_ignored) -> str | None:
    """``None`` if :func:`fused_recurrent_kda` serves this call, else the
    reason.  As :func:`verify_chunk_kda` without the chunk-span limit on a
    precomputed log decay (the token recurrence multiplies by exp(g) one
    token at a time); the softplus gate is still not served."""
    reason = _common_reason(q, k, v, g, beta)
    if reason:
        return reason
    if use_gate_in_kernel:
        if not _lb_ok(lower_bound):
            return "the in-kernel gate needs lower_bound in (-11, 0) (softplus gate not served)"
        if A_log is None:
            return "use_gate_in_kernel requires A_log"
    return _device_reason(q)


def _flat_dt_bias(dt_bias):
    # FLA takes dt_bias as [HV * K] or [HV, K] (bench_fla_compare.py:96, 105).
    return None if dt_bias is None else dt_bias.reshape(-1)


def chunk_kda(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    cu_seqlens: torch.Tensor | None = None,
    safe_gate: bool = False,
    lower_bound: float | None = None,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    use_beta_sigmoid_in_kernel: bool = False,
    state_v_first: bool = False,
    chunk_size: int = 64,
    return_intermediate_states: bool = False,
    cp_context=None,
    max_seqlen: int | None = None,
    **kwargs,
):
    """FLA ``chunk_kda`` on the MI355X chunked kernels.

    Returns ``(o, final_state)``: ``o`` ``[B, T, HV, 128]`` bf16 and the fp32
    final state (``None`` unless ``output_final_state``), K-first
    ``[N, HV, K, V]`` unless ``state_v_first``.  Raises
    ``NotImplementedError`` outside :func:`verify_chunk_kda`'s bucket.
    ``max_seqlen`` (with ``cu_seqlens``) is the longest sequence's length,
    a hint for the kernel choice (:func:`kda_bt16.kda_bt16_fwd`).
    """
    del chunk_size, kwargs  # 16-token chunks; other FLA options do not change the forward
    reason = verify_chunk_kda(
        q, k, v, g, beta, use_gate_in_kernel=use_gate_in_kernel, safe_gate=safe_gate,
        lower_bound=lower_bound, A_log=A_log,
        return_intermediate_states=return_intermediate_states, cp_context=cp_context)
    if reason:
        raise NotImplementedError(f"chunk_kda on MI355X: {reason}")
    dt_bias = _flat_dt_bias(dt_bias)
    B, T, H, K, HV, V = _validate_kda_inputs(
        q, k, v, g, beta, initial_state, use_gate_in_kernel, True, lower_bound,
        A_log, dt_bias, state_v_first, cu_seqlens,
    )
    _check_max_seqlen(max_seqlen)
    if scale is None:
        scale = K ** -0.5
    return _fwd_maybe_autograd(
        q, k, v, g, beta, scale, initial_state, output_final_state,
        use_qk_l2norm_in_kernel, use_gate_in_kernel, use_beta_sigmoid_in_kernel,
        lower_bound, A_log, dt_bias, state_v_first,
        cu_seqlens=cu_seqlens, g_log=not use_gate_in_kernel, max_seqlen=max_seqlen,
    )


def fused_recurrent_kda(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    use_qk_l2norm_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    use_beta_sigmoid_in_kernel: bool = False,
    lower_bound: float | None = None,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    cu_seqlens: torch.Tensor | None = None,
    state_v_first: bool = False,
    inplace_final_state: bool = False,
    **kwargs,
):
    """FLA ``fused_recurrent_kda`` (the decode path, and the reference
    tests' gold, tests/test_kda_bt16.py:26-38) on the MI355X token
    recurrence.  Returns ``(o, final_state)``; ``o`` has q's dtype."""
    del kwargs
    reason = verify_fused_recurrent_kda(
        q, k, v, g, beta, use_gate_in_kernel=use_gate_in_kernel, lower_bound=lower_bound,
        A_log=A_log)
    if reason:
        raise NotImplementedError(f"fused_recurrent_kda on MI355X: {reason}")
    return kda_recurrent_fwd(
        q, k, v, g, beta, scale=scale, initial_state=initial_state,
        output_final_state=output_final_state or inplace_final_state,
        use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel, use_gate_in_kernel=use_gate_in_kernel,
        use_beta_sigmoid_in_kernel=use_beta_sigmoid_in_kernel,
        lower_bound=lower_bound if use_gate_in_kernel else -5.0, A_log=A_log,
        dt_bias=_flat_dt_bias(dt_bias), state_v_first=state_v_first,
        output_dtype=q.dtype, inplace_final_state=inplace_final_state, cu_seqlens=cu_seqlens,
    )

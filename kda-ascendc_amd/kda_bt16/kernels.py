"""KDA BT=16 chunked forward on MI355X: the Python API and host driver.

Drop-in for ``/root/reference/src/kda_bt16/kernels.py``:

* :func:`kda_bt16_fwd` and :func:`kda_bt16_debug` keep the reference's
  signatures, defaults, validation order, messages and exception types
  (kernels.py:609-850);
* the two stages run as hand-written gfx950 HIP kernels in
  ``libkda_bt16_hip.so`` (``csrc/kda_k1.hip``, ``csrc/kda_k2.hip``), called
  through the C ABI declared in ``include/kda_bt16_hip.h`` on the caller's
  current stream, with no host synchronisation.

Differences from the reference, all supersets of its contract:

* ``g`` and ``beta`` may be bfloat16 as well as float32 (the kernels widen
  them to fp32 at load, exactly as the reference's ``.to(tl.float32)``);
* ``state_v_first=False`` is handled by stage 2 reading/writing the
  ``[K, V]`` state directly instead of transposing at the boundary
  (kernels.py:499-510); the values are identical;
* ``use_fused_kernel=True`` runs the fused kernel (one work-group per
  sequence and value head, stage 1's records kept in LDS: the reference's
  single-kernel variant, kernels.py:305-472) whatever the geometry; without
  it the forward fuses when the (sequence, head) pairs are more than half
  the CUs (with ``cu_seqlens``: at least as many as the CUs).  Both give
  the two-stage results bit for bit (the reference's own test requires the
  two to agree, tests/test_kda_bt16.py:174-200);
* ``HV`` may be any multiple of ``H`` (grouped value heads: value head hv
  reads q/k head hv // (HV // H), the indexing of kernels.py:88, which the
  reference's validation does not yet admit, kernels.py:729-730);
* ``cu_seqlens`` (keyword, default None) packs N variable-length sequences
  along T with B == 1, FLA's varlen convention; the states are then
  ``[N, HV, ...]`` (the reference lists varlen as a limitation,
  README.md:420-421);
* the forward is differentiable: when an input requires grad,
  :func:`kda_bt16_fwd` records an autograd node whose backward runs the
  HIP backward (:func:`kda_bt16_bwd`; the reference is forward-only,
  README.md:420).
"""

from __future__ import annotations

import contextlib
import ctypes
import threading

import torch

from . import _hip, workspace

# Module-level cache for ``reuse_workspace=True`` (kernels.py:35, 525-536):
# o / ht alias this cache and are overwritten by the next call with the
# same geometry.  Not thread safe, like the reference's.
_WORKSPACE_CACHE: dict[tuple, dict[str, torch.Tensor]] = {}

# Training memory policy of the autograd node.  True (the default): the
# forward keeps its per-chunk state (kda_bt16_fwd_save_hip, ~55 KiB per
# 16-token chunk and value head) and the backward starts from it; False:
# the forward keeps only its inputs and the backward recomputes the state.
# The two give the same gradients, bit for bit.
_SAVE_STATE = [True]


def set_backward_recompute(recompute: bool) -> None:
    """Choose the training memory policy: ``True`` recomputes the chunk
    states in the backward (memory of the inputs only), ``False`` (the
    default) keeps them from the forward."""
    _SAVE_STATE[0] = not recompute


# Kernel choices forced by :func:`forward_choice` on this thread.
_CHOICE = threading.local()


@contextlib.contextmanager
def forward_choice(*, fused: bool | None = None, k2_tiles: int = 0, k2_wave_tiles: int = 0):
    """Force the forward's kernel choices for the calls this thread makes
    inside the block (no counterpart in the reference, whose ``_run``
    always launches its two stages, kernels.py:581-602):

    * ``fused``: True runs the fused kernel, False stage 1 then stage 2,
      None (default) leaves it to the library; an explicit
      ``use_fused_kernel=True`` still wins;
    * ``k2_tiles``: stage-2 value tiles per work-group (1, 2, 4 or 8);
    * ``k2_wave_tiles``: with 2-8 tiles, 1 or 2 forces compute waves that
      each run that many whole tiles (0: the library's kernel, a state
      wave per tile at 2 tiles);

    0 leaves the choice to the library.  They reach the C ABI as the
    ``KDA_BT16_FUSED_KERNEL`` / ``KDA_BT16_TWO_STAGE`` flags and the
    ``k2_tiles`` / ``k2_wave_tiles`` fields.  Every choice gives the same
    results bit for bit: this is for measurement and tests."""
    if k2_tiles not in (0, 1, 2, 4, 8):
        raise ValueError(f"k2_tiles must be 0, 1, 2, 4 or 8, got {k2_tiles}")
    if k2_wave_tiles not in (0, 1, 2):
        raise ValueError(f"k2_wave_tiles must be 0, 1 or 2, got {k2_wave_tiles}")
    prev = getattr(_CHOICE, "value", None)
    _CHOICE.value = (fused, k2_tiles, k2_wave_tiles)
    try:
        yield
    finally:
        _CHOICE.value = prev


def fused_abort_count(reset: bool = False, device: torch.device | int | None = None) -> int:
    """Fused-kernel work-groups on ``device`` (default: the current one)
    that gave up a bounded wait since the library was loaded or the count
    last reset (``kda_bt16_fused_aborts``).  Such a work-group writes NaN
    over the o columns and final-state rows of its compute waves that had
    not finished, instead of hanging the GPU.  Waits for the device's work
    to finish."""
    with torch.cuda.device(torch.cuda.current_device() if device is None else device):
        return _hip.fused_aborts(reset)

_RCP_LN2 = 1.4426950216
_EPS = 1e-6
_BT = 16


def _validate_kda_inputs(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    initial_state: torch.Tensor | None,
    use_gate_in_kernel: bool,
    safe_gate: bool,
    lower_bound: float | None,
    A_log: torch.Tensor | None,
    dt_bias: torch.Tensor | None,
    state_v_first: bool,
    cu_seqlens: torch.Tensor | None = None,
) -> tuple[int, int, int, int, int, int]:
    """Input contract of kernels.py:609-749, same order and messages, with
    two widenings: HV may be any multiple of H (grouped value heads; the
    reference requires HV == H, kernels.py:729-730), and ``cu_seqlens``
    packs N sequences along T (FLA's varlen convention and messages: B must
    be 1 and the states have N rows).

    Returns ``(B, T, H, K, HV, V)``; raises ``ValueError`` / ``TypeError``.
    """
    if q.ndim != 4:
        raise ValueError(f"q must be 4D [B, T, H, D], got {q.ndim}D with shape {q.shape}")
    if k.ndim != 4:
        raise ValueError(f"k must be 4D [B, T, H, D], got {k.ndim}D with shape {k.shape}")
    if v.ndim != 4:
        raise ValueError(f"v must be 4D [B, T, HV, V], got {v.ndim}D with shape {v.shape}")
    if g.ndim != 4:
        raise ValueError(f"g must be 4D [B, T, HV, D], got {g.ndim}D with shape {g.shape}")
    if beta.ndim != 3:
        raise ValueError(f"beta must be 3D [B, T, HV], got {beta.ndim}D with shape {beta.shape}")

    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[-1]

    if B <= 0 or T <= 0 or H <= 0 or K <= 0:
        raise ValueError(f"q dimensions must be positive, got B={B}, T={T}, H={H}, K={K}")
    if HV <= 0 or V <= 0:
        raise ValueError(f"v dimensions must be positive, got HV={HV}, V={V}")

    if not q.is_contiguous():
        raise ValueError("q must be contiguous (kernel assumes stride [H*K, K, 1])")
    if not k.is_contiguous():
        raise ValueError("k must be contiguous")
    if not v.is_contiguous():
        raise ValueError("v must be contiguous")
    if not g.is_contiguous():
        raise ValueError("g must be contiguous")
    if not beta.is_contiguous():
        raise ValueError("beta must be contiguous")

    if q.dtype != torch.bfloat16:
        raise TypeError(f"q must be bfloat16, got {q.dtype}")
    if k.dtype != torch.bfloat16:
        raise TypeError(f"k must be bfloat16, got {k.dtype}")
    if v.dtype != torch.bfloat16:
        raise TypeError(f"v must be bfloat16, got {v.dtype}")
    if use_gate_in_kernel and g.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"g must be float32 when use_gate_in_kernel=True, got {g.dtype}")
    # Without the in-kernel gate the reference takes g of any dtype and
    # widens it to fp32 at load (kernels.py:673-674, 108); _gate_f32 does
    # that on the host for dtypes other than fp32 / bf16.
    if beta.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"beta must be float32 or bfloat16, got {beta.dtype}")

    if k.shape != q.shape:
        raise ValueError(f"k.shape {k.shape} must match q.shape {q.shape}")
    if v.shape != (B, T, HV, V):
        raise ValueError(f"v.shape {v.shape} must be [B={B}, T={T}, HV={HV}, V={V}]")
    if g.shape != (B, T, HV, K):
        raise ValueError(f"g.shape {g.shape} must be [B={B}, T={T}, HV={HV}, K={K}]")
    if beta.shape != (B, T, HV):
        raise ValueError(f"beta.shape {beta.shape} must be [B={B}, T={T}, HV={HV}]")

    if not all(x.device == q.device for x in [k, v, g, beta]):
        raise ValueError(f"All tensors must be on same device as q ({q.device})")

    S = B
    if cu_seqlens is not None:
        if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
            raise ValueError(f"cu_seqlens must be 1D with at least 2 entries, got shape {tuple(cu_seqlens.shape)}")
        if cu_seqlens.dtype not in (torch.int32, torch.int64):
            raise TypeError(f"cu_seqlens must be int32 or int64, got {cu_seqlens.dtype}")
        if not cu_seqlens.is_contiguous():
            raise ValueError("cu_seqlens must be contiguous")
        if cu_seqlens.device != q.device:
            raise ValueError(f"cu_seqlens device {cu_seqlens.device} must match q ({q.device})")
        if B != 1:
            raise ValueError(
                f"The batch size is expected to be 1 rather than {B} when using `cu_seqlens`. "
                "Please flatten variable-length inputs before processing."
            )
        S = cu_seqlens.numel() - 1
        if initial_state is not None and initial_state.shape[0] != S:
            raise ValueError(
                "The number of initial states is expected to be equal to the number of input "
                f"sequences, i.e., {S} rather than {initial_state.shape[0]}."
            )

    if initial_state is not None:
        if not initial_state.is_contiguous():
            raise ValueError("initial_state must be contiguous")
        if initial_state.dtype != torch.float32:
            raise TypeError(f"initial_state must be float32, got {initial_state.dtype}")
        if initial_state.device != q.device:
            raise ValueError(f"initial_state device {initial_state.device} must match q ({q.device})")
        expected_shape = (S, HV, V, K) if state_v_first else (S, HV, K, V)
        if initial_state.shape != expected_shape:
            raise ValueError(
                f"initial_state.shape {initial_state.shape} must be {expected_shape} "
                f"(state_v_first={state_v_first})"
            )

    if A_log is not None:
        if not A_log.is_contiguous():
            raise ValueError("A_log must be contiguous")
        if A_log.dtype != torch.float32:
            raise TypeError(f"A_log must be float32, got {A_log.dtype}")
        if A_log.device != q.device:
            raise ValueError("A_log device must match q")
        if A_log.shape != (HV,):
            raise ValueError(f"A_log.shape {A_log.shape} must be (HV={HV},)")

    if dt_bias is not None:
        if not dt_bias.is_contiguous():
            raise ValueError("dt_bias must be contiguous")
        if dt_bias.dtype != torch.float32:
            raise TypeError(f"dt_bias must be float32, got {dt_bias.dtype}")
        if dt_bias.device != q.device:
            raise ValueError("dt_bias device must match q")
        if dt_bias.shape != (HV * K,):
            raise ValueError(f"dt_bias.shape {dt_bias.shape} must be (HV*K={HV * K},)")

    if K != 128 or V != 128:
        raise ValueError(f"prototype targets K=V=128, got K={K}, V={V}")
    if HV % H != 0:
        raise ValueError(f"HV must be a multiple of H (grouped value heads), got HV={HV}, H={H}")

    if use_gate_in_kernel:
        if not safe_gate:
            raise ValueError("use_gate_in_kernel requires safe_gate=True")
        if lower_bound is None:
            raise ValueError("use_gate_in_kernel requires lower_bound")
        if not (-11.0 < lower_bound < 0.0):
            raise ValueError(
                f"lower_bound must be in range (-11, 0) to prevent fp32 exp2 overflow "
                f"(BT=16 can amplify exponent by ~8x), got {lower_bound}"
            )
        if A_log is None:
            raise ValueError("use_gate_in_kernel requires A_log")

    return B, T, H, K, HV, V


def _gate_f32(g: torch.Tensor) -> torch.Tensor:
    """g as the kernels read it: fp32 or bf16 as given, any other dtype
    widened to fp32 (the reference's ``.to(tl.float32)`` at load,
    kernels.py:108)."""
    if g.dtype in (torch.float32, torch.bfloat16):
        return g
    return g.to(torch.float32)


def _require_gpu(q: torch.Tensor) -> None:
    if q.device.type != "cuda":
        raise ValueError(
            f"kda_bt16 runs on a ROCm GPU (torch 'cuda' device); got tensors on {q.device}"
        )


def _aligned(t: torch.Tensor | None, align: int = 16) -> torch.Tensor | None:
    """The kernels use 16-byte vector loads: copy the rare contiguous view
    whose storage offset breaks that alignment."""
    if t is None or t.data_ptr() % align == 0:
        return t
    return t.clone()


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _dtype_tag(t: torch.Tensor) -> int:
    return _hip.DTYPE_BF16 if t.dtype == torch.bfloat16 else _hip.DTYPE_F32


def _make_args(
    q, k, v, g, beta, scale, lower_bound, A_log, dt_bias, h0, o, ht, ws, ws_bytes,
    flags, dbg=None, cu_seqlens=None, max_seqlen=None,
) -> _hip.KdaBt16Args:
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[-1]
    a = _hip.KdaBt16Args()
    a.abi_version = _hip.ABI_VERSION
    a.B, a.T, a.H, a.HV, a.K, a.V = B, T, H, HV, K, V
    a.flags = flags
    a.scale = float(scale)
    a.lower_bound = float(lower_bound) if lower_bound is not None else 0.0
    a.g_dtype = _dtype_tag(g)
    a.beta_dtype = _dtype_tag(beta)
    a.q, a.k, a.v, a.g, a.beta = (x.data_ptr() for x in (q, k, v, g, beta))
    a.A_log = _ptr(A_log)
    a.dt_bias = _ptr(dt_bias)
    a.h0 = _ptr(h0)
    a.o = _ptr(o)
    a.ht = _ptr(ht)
    a.workspace = _ptr(ws)
    a.workspace_bytes = ws_bytes
    if dbg is not None:
        a.dbg_Aqk = dbg["Aqk"].data_ptr()
        a.dbg_A_inv = dbg["A_inv"].data_ptr()
        a.dbg_w = dbg["w"].data_ptr()
        a.dbg_u = dbg["u"].data_ptr()
        a.dbg_g = dbg["g"].data_ptr()
    if cu_seqlens is not None:
        a.cu_seqlens = cu_seqlens.data_ptr()
        a.cu_seqlens_dtype = _hip.DTYPE_I64 if cu_seqlens.dtype == torch.int64 else _hip.DTYPE_I32
        a.N = cu_seqlens.numel() - 1
        a.max_seqlen = int(max_seqlen or 0)
    choice = getattr(_CHOICE, "value", None)
    if choice is not None:
        fused, a.k2_tiles, a.k2_wave_tiles = choice
        if fused is False and not flags & _hip.FUSED_KERNEL:
            a.flags |= _hip.TWO_STAGE
        elif fused is True:
            a.flags |= _hip.FUSED_KERNEL
    return a


def _flags(use_gate: bool, use_l2norm: bool, use_beta_sigmoid: bool, state_v_first: bool,
           g_log: bool = False, fused: bool = False) -> int:
    f = _hip.FUSED_KERNEL if fused else 0
    if g_log and not use_gate:
        f |= _hip.G_LOG_DECAY
    if use_gate:
        f |= _hip.USE_GATE
    if use_l2norm:
        f |= _hip.USE_QK_L2NORM
    if use_beta_sigmoid:
        f |= _hip.USE_BETA_SIGMOID
    if state_v_first:
        f |= _hip.STATE_V_FIRST
    return f


def _run(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    scale: float,
    initial_state: torch.Tensor | None,
    output_final_state: bool,
    use_qk_l2norm_in_kernel: bool,
    use_gate_in_kernel: bool,
    use_beta_sigmoid_in_kernel: bool,
    lower_bound: float,
    A_log: torch.Tensor | None,
    dt_bias: torch.Tensor | None,
    state_v_first: bool,
    return_intermediates: bool,
    use_fused: bool = False,
    reuse_workspace: bool = False,
    cu_seqlens: torch.Tensor | None = None,
    g_log: bool = False,
    save_state: bool = False,
    max_seqlen: int | None = None,
):
    """Host driver, the counterpart of kernels.py:475-606: allocate outputs,
    lease the workspace when the forward runs its two stages (the fused
    kernel keeps the records in LDS), launch through the C ABI.

    ``save_state``: run the training forward (``kda_bt16_fwd_save_hip``)
    and return ``(o, ht, saved)``, ``saved`` the uint8 state tensor the
    backward starts from."""
    _require_gpu(q)
    g = _gate_f32(g)
    q, k, v, g, initial_state, dt_bias = (
        _aligned(x) for x in (q, k, v, g, initial_state, dt_bias))
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[-1]
    S = B if cu_seqlens is None else cu_seqlens.numel() - 1
    dev = q.device

    cache_key = (dev, B, T, H, HV, K, V, S, k.dtype, return_intermediates)
    cache = _WORKSPACE_CACHE.get(cache_key) if reuse_workspace else None

    def alloc(name, shape, dtype):
        if cache is not None:
            t = cache.get(name)
            if t is not None and t.shape == shape and t.dtype == dtype:
                return t
        t = torch.empty(shape, dtype=dtype, device=dev)
        if reuse_workspace:
            _WORKSPACE_CACHE.setdefault(cache_key, {})[name] = t
        return t

    o = alloc("o", (B, T, HV, V), k.dtype)
    ht = None
    if output_final_state:
        ht = alloc("ht", (S, HV, V, K) if state_v_first else (S, HV, K, V), torch.float32)

    dbg = None
    if return_intermediates:
        dbg = {
            "Aqk": torch.empty((B, T, HV, _BT), dtype=k.dtype, device=dev),
            "A_inv": torch.empty((B, T, HV, _BT), dtype=k.dtype, device=dev),
            "w": torch.empty((B, T, HV, K), dtype=k.dtype, device=dev),
            "u": torch.empty((B, T, HV, V), dtype=k.dtype, device=dev),
            "g": torch.empty((B, T, HV, K), dtype=torch.float32, device=dev),
        }

    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        args = _make_args(
            q, k, v, g, beta, scale, lower_bound if use_gate_in_kernel else None,
            A_log, dt_bias, initial_state, o, ht, None, 0,
            _flags(use_gate_in_kernel, use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel,
                   state_v_first, g_log, use_fused),
            dbg, cu_seqlens, max_seqlen,
        )
        if save_state or _hip.fwd_plan(args) == 0:
            ws_bytes = _hip.workspace_bytes_args(args)
            ws = workspace.lease(dev, stream, ws_bytes)
            args.workspace, args.workspace_bytes = ws.data_ptr(), ws_bytes
        if save_state:
            nbytes = _hip.saved_bytes(args)
            saved = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            _hip.call_saved("kda_bt16_fwd_save_hip", args, saved.data_ptr(), nbytes, stream)
            return o, ht, saved
        _hip.call("kda_bt16_fwd_hip", args, stream)

    if return_intermediates:
        return o, ht, dbg
    return o, ht


def _bwd_run(
    do: torch.Tensor,
    dht: torch.Tensor | None,
    q, k, v, g, beta, scale, initial_state, use_qk_l2norm_in_kernel, use_gate_in_kernel,
    use_beta_sigmoid_in_kernel, lower_bound, A_log, dt_bias, state_v_first, cu_seqlens, g_log,
    need_gate_grads: bool = True, need_dh0: bool = True, saved: torch.Tensor | None = None,
):
    """Host driver of the backward: allocate the gradients, lease the
    workspace, launch ``kda_bt16_bwd_hip`` on the current stream (or
    ``kda_bt16_bwd_saved_hip`` from a training forward's ``saved`` state).

    Returns ``(dq, dk, dv, dg, dbeta, dA_log, ddt_bias, dh0)``; dA_log /
    ddt_bias are None without the in-kernel gate (or dt_bias), dh0 is None
    without an initial state."""
    _require_gpu(q)
    g_dtype = g.dtype
    g = _gate_f32(g)
    q, k, v, g, initial_state, dt_bias = (
        _aligned(x) for x in (q, k, v, g, initial_state, dt_bias))
    dev = q.device
    do = _aligned(do.to(torch.bfloat16).contiguous())
    if dht is not None:
        dht = _aligned(dht.to(torch.float32).contiguous())
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dg = torch.empty_like(g)
    dbeta = torch.empty_like(beta)
    gate_grads = need_gate_grads and use_gate_in_kernel
    dA_log = torch.empty_like(A_log) if gate_grads and A_log is not None else None
    ddt_bias = torch.empty_like(dt_bias) if gate_grads and dt_bias is not None else None
    dh0 = torch.empty_like(initial_state) if (need_dh0 and initial_state is not None) else None
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        fa = _make_args(
            q, k, v, g, beta, scale, lower_bound if use_gate_in_kernel else None,
            A_log, dt_bias, initial_state, None, None, None, 0,
            _flags(use_gate_in_kernel, use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel,
                   state_v_first, g_log),
            None, cu_seqlens,
        )
        ws_bytes = (_hip.bwd_workspace_bytes(fa) if saved is None
                    else _hip.bwd_saved_workspace_bytes(fa))
        # Not pooled: a backward's workspace (up to ~106 KiB per record slot)
        # goes back to torch's caching allocator when the call's work is
        # done, instead of staying leased to every later forward.
        ws = workspace.scratch(dev, ws_bytes)
        ba = _hip.KdaBt16BwdArgs()
        ba.fwd = ctypes.pointer(fa)
        ba.dout = do.data_ptr()
        ba.dht = _ptr(dht)
        ba.dq, ba.dk, ba.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
        ba.dg, ba.dbeta = dg.data_ptr(), dbeta.data_ptr()
        ba.dA_log = _ptr(dA_log)
        ba.ddt_bias = _ptr(ddt_bias)
        ba.dh0 = _ptr(dh0)
        ba.workspace, ba.workspace_bytes = ws.data_ptr(), ws_bytes
        if saved is None:
            _hip.call("kda_bt16_bwd_hip", ba, stream)
        else:
            _hip.call_saved("kda_bt16_bwd_saved_hip", ba, saved.data_ptr(), saved.numel(), stream)
    return dq, dk, dv, dg.to(g_dtype), dbeta, dA_log, ddt_bias, dh0


class _KdaBt16Fn(torch.autograd.Function):
    """Autograd node of the chunked forward.  By default the forward is the
    training forward (``kda_bt16_fwd_save_hip``: the same o and ht, plus
    the per-chunk state) and the backward starts from that state
    (``kda_bt16_bwd_saved_hip``).  With :func:`set_backward_recompute` the
    forward is :func:`_run` and the backward recomputes the chunk states
    (``kda_bt16_bwd_hip``)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, A_log, dt_bias, initial_state, cu_seqlens, cfg):
        (scale, output_final_state, l2, use_gate, bsig, lower_bound, svf, g_log, reuse) = cfg
        save = _SAVE_STATE[0]
        res = _run(
            q, k, v, g, beta, scale, initial_state, output_final_state, l2, use_gate, bsig,
            lower_bound, A_log, dt_bias, svf, return_intermediates=False,
            reuse_workspace=reuse, cu_seqlens=cu_seqlens, g_log=g_log, save_state=save,
        )
        o, ht = res[0], res[1]
        # The per-chunk state goes through save_for_backward with the inputs:
        # autograd frees it once the backward has run (and saved-tensor
        # hooks such as checkpointing see it), while o may live on.
        ctx.save_for_backward(q, k, v, g, beta, A_log, dt_bias, initial_state, cu_seqlens,
                              res[2] if save else None)
        ctx.cfg = cfg
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g, beta, A_log, dt_bias, h0, cu, state = ctx.saved_tensors
        (scale, _ofs, l2, use_gate, bsig, lower_bound, svf, g_log, _reuse) = ctx.cfg
        if do is None:
            do = torch.zeros(v.shape, dtype=torch.bfloat16, device=v.device)
        need = ctx.needs_input_grad
        dq, dk, dv, dg, dbeta, dA_log, ddt_bias, dh0 = _bwd_run(
            do, dht, q, k, v, g, beta, scale, h0, l2, use_gate, bsig, lower_bound, A_log,
            dt_bias, svf, cu, g_log, need_gate_grads=need[5] or need[6], need_dh0=need[7],
            saved=state,
        )
        return (dq, dk, dv, dg, dbeta, dA_log if need[5] else None,
                ddt_bias if need[6] else None, dh0 if need[7] else None, None, None)


def _wants_grad(*ts) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def _check_max_seqlen(max_seqlen) -> None:
    if max_seqlen is not None and (not isinstance(max_seqlen, int) or max_seqlen < 0):
        raise ValueError(f"max_seqlen must be a non-negative int or None, got {max_seqlen!r}")


def _fwd_maybe_autograd(
    q, k, v, g, beta, scale, initial_state, output_final_state, l2, use_gate, bsig,
    lower_bound, A_log, dt_bias, svf, reuse_workspace=False, cu_seqlens=None, g_log=False,
    use_fused=False, max_seqlen=None,
):
    """:func:`_run`, through :class:`_KdaBt16Fn` when an input requires grad
    (whose training forward keeps its per-chunk state for the backward and so
    always runs the two stages)."""
    if _wants_grad(q, k, v, g, beta, A_log, dt_bias, initial_state):
        cfg = (scale, output_final_state, l2, use_gate, bsig, lower_bound, svf, g_log,
               reuse_workspace)
        return _KdaBt16Fn.apply(q, k, v, g, beta, A_log, dt_bias, initial_state, cu_seqlens, cfg)
    return _run(
        q, k, v, g, beta, scale, initial_state, output_final_state, l2, use_gate, bsig,
        lower_bound, A_log, dt_bias, svf, return_intermediates=False,
        reuse_workspace=reuse_workspace, cu_seqlens=cu_seqlens, g_log=g_log, use_fused=use_fused,
        max_seqlen=max_seqlen,
    )


def kda_bt16_bwd(
    do: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    dht: torch.Tensor | None = None,
    use_qk_l2norm_in_kernel: bool = False,
    use_gate_in_kernel: bool = False,
    use_beta_sigmoid_in_kernel: bool = False,
    safe_gate: bool = True,
    lower_bound: float = -5.0,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    state_v_first: bool = True,
    *,
    cu_seqlens: torch.Tensor | None = None,
    g_log: bool = False,
) -> dict:
    """Backward of :func:`kda_bt16_fwd` (no counterpart in the reference,
    which is forward-only, README.md:420): the gradients of
    ``sum(o * do) + sum(ht * dht)`` with respect to every input, for the
    forward's arguments.  ``g_log`` selects FLA's per-token log decay for
    ``g`` (as :func:`kda_bt16.fla.chunk_kda` uses it).

    Returns a dict with ``dq, dk, dv`` (bf16), ``dg``, ``dbeta`` (the dtypes
    of g and beta), ``dA_log``, ``ddt_bias`` (fp32, with the in-kernel gate)
    and ``dh0`` (with an initial state, in its layout).  The same math runs
    when :func:`kda_bt16_fwd`'s inputs require grad and autograd calls it.
    """
    B, T, H, K, HV, V = _validate_kda_inputs(
        q, k, v, g, beta, initial_state, use_gate_in_kernel, safe_gate, lower_bound,
        A_log, dt_bias, state_v_first, cu_seqlens,
    )
    S = B if cu_seqlens is None else cu_seqlens.numel() - 1
    if do.shape != (B, T, HV, V):
        raise ValueError(f"do.shape {tuple(do.shape)} must be [B={B}, T={T}, HV={HV}, V={V}]")
    if dht is not None and dht.shape != ((S, HV, V, K) if state_v_first else (S, HV, K, V)):
        raise ValueError(f"dht.shape {tuple(dht.shape)} must match the final state's")
    if scale is None:
        scale = K ** -0.5
    dq, dk, dv, dg, dbeta, dA_log, ddt_bias, dh0 = _bwd_run(
        do, dht, q, k, v, g, beta, scale, initial_state, use_qk_l2norm_in_kernel,
        use_gate_in_kernel, use_beta_sigmoid_in_kernel, lower_bound, A_log, dt_bias,
        state_v_first, cu_seqlens, g_log,
    )
    return {"dq": dq, "dk": dk, "dv": dv, "dg": dg, "dbeta": dbeta, "dA_log": dA_log,
            "ddt_bias": ddt_bias, "dh0": dh0}


def kda_bt16_fwd(
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
    safe_gate: bool = True,
    lower_bound: float = -5.0,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    state_v_first: bool = True,
    use_fused_kernel: bool = False,
    reuse_workspace: bool = False,
    *,
    cu_seqlens: torch.Tensor | None = None,
    max_seqlen: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """KDA forward (reference: kernels.py:752-810).

    Args:
        q/k: ``[B, T, H, K]``, bf16, ``K == 128``.
        v: ``[B, T, HV, V]``, bf16, ``HV`` a multiple of ``H``, ``V == 128``.
        g: ``[B, T, HV, K]`` fp32 or bf16: the raw gate if
            ``use_gate_in_kernel``, else the precomputed chunk-local cumsum
            in the log2 domain.
        beta: ``[B, T, HV]`` fp32 or bf16; raw logits if
            ``use_beta_sigmoid_in_kernel``.
        initial_state: fp32 ``[B, HV, V, K]`` (``state_v_first=True``) or
            ``[B, HV, K, V]``; ``N`` rows instead of ``B`` with ``cu_seqlens``.
        cu_seqlens: optional int32/int64 ``[N + 1]`` offsets of N sequences
            packed along T (B must be 1).
        max_seqlen: with ``cu_seqlens``, the longest sequence's length if
            the caller knows it (FLA's varlen convention).  A hint for the
            choice between the fused kernel and the two stages, which it
            makes from estimated times: one long sequence among short ones
            keeps the two stages.  The results are the same either way.

    Returns:
        ``o`` of shape ``[B, T, HV, V]`` (bf16) and, if
        ``output_final_state``, the fp32 final state in the same layout as
        ``initial_state``.
    """
    B, T, H, K, HV, V = _validate_kda_inputs(
        q, k, v, g, beta, initial_state,
        use_gate_in_kernel, safe_gate, lower_bound,
        A_log, dt_bias, state_v_first, cu_seqlens,
    )
    _check_max_seqlen(max_seqlen)
    if scale is None:
        scale = K ** -0.5
    return _fwd_maybe_autograd(
        q, k, v, g, beta, scale, initial_state, output_final_state,
        use_qk_l2norm_in_kernel, use_gate_in_kernel, use_beta_sigmoid_in_kernel,
        lower_bound, A_log, dt_bias, state_v_first,
        reuse_workspace=reuse_workspace, cu_seqlens=cu_seqlens, use_fused=use_fused_kernel,
        max_seqlen=max_seqlen,
    )


def kda_bt16_debug(
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
    safe_gate: bool = True,
    lower_bound: float = -5.0,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    state_v_first: bool = True,
    *,
    cu_seqlens: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None, dict]:
    """Like :func:`kda_bt16_fwd`, and also return the stage-1 intermediates
    ``{Aqk, A_inv, w, u, g}`` in the reference's layouts (kernels.py:813-850):
    ``Aqk``/``A_inv`` ``[B,T,HV,16]`` bf16, ``w``/``u`` ``[B,T,HV,128]`` bf16,
    ``g`` ``[B,T,HV,128]`` fp32."""
    B, T, H, K, HV, V = _validate_kda_inputs(
        q, k, v, g, beta, initial_state,
        use_gate_in_kernel, safe_gate, lower_bound,
        A_log, dt_bias, state_v_first, cu_seqlens,
    )
    if scale is None:
        scale = K ** -0.5
    return _run(
        q, k, v, g, beta, scale, initial_state, output_final_state,
        use_qk_l2norm_in_kernel, use_gate_in_kernel, use_beta_sigmoid_in_kernel,
        lower_bound, A_log, dt_bias, state_v_first,
        return_intermediates=True,
        use_fused=False,
        reuse_workspace=False,
        cu_seqlens=cu_seqlens,
    )


def kda_bt16_stage_launchers(
    q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
    use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True,
    lower_bound=-5.0, A_log=None, dt_bias=None, state_v_first=True, cu_seqlens=None,
    g_log=False,
):
    """Return ``(k1, k2, o, ht)``: zero-argument callables that launch only
    stage 1 or only stage 2 on the current stream, over buffers allocated
    once here.  The per-kernel breakdown of bench_bt16.py:85-118 uses the
    raw Triton kernels for the same purpose."""
    B, T, H, K, HV, V = _validate_kda_inputs(
        q, k, v, g, beta, initial_state, use_gate_in_kernel, True, lower_bound,
        A_log, dt_bias, state_v_first, cu_seqlens,
    )
    _require_gpu(q)
    if scale is None:
        scale = K ** -0.5
    dev = q.device
    S = B if cu_seqlens is None else cu_seqlens.numel() - 1
    o = torch.empty((B, T, HV, V), dtype=torch.bfloat16, device=dev)
    ht = None
    if output_final_state:
        ht = torch.empty((S, HV, V, K) if state_v_first else (S, HV, K, V),
                         dtype=torch.float32, device=dev)
    args = _make_args(
        q, k, v, g, beta, scale, lower_bound if use_gate_in_kernel else None,
        A_log, dt_bias, initial_state, o, ht, None, 0,
        _flags(use_gate_in_kernel, use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel,
               state_v_first, g_log),
        None, cu_seqlens,
    )
    ws_bytes = _hip.workspace_bytes_args(args)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws_bytes
    keep = (q, k, v, g, beta, A_log, dt_bias, initial_state, ws, cu_seqlens)

    def k1():
        _ = keep
        _hip.call("kda_bt16_k1_hip", args, torch.cuda.current_stream(dev).cuda_stream)

    # which kernels kda_bt16_fwd runs for these arguments: "fused" or
    # "two-stage", and for the two stages in how many chunk ranges (these
    # launchers run one pass over all chunks)
    k1.forward_plan = "fused" if _hip.fwd_plan(args) == 1 else "two-stage"
    k1.forward_segments = _hip.fwd_segments(args)

    def k2():
        _ = keep
        _hip.call("kda_bt16_k2_hip", args, torch.cuda.current_stream(dev).cuda_stream)

    return k1, k2, o, ht


def kda_recurrent_fwd(
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
    lower_bound: float | None = -5.0,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    state_v_first: bool = True,
    output_dtype: torch.dtype = torch.bfloat16,
    inplace_final_state: bool = False,
    cu_seqlens: torch.Tensor | None = None,
):
    """Token-by-token KDA recurrence on the GPU, fp32 state: the decode
    step (T == 1) and the fused-recurrent forward for any T.

    Arguments are those of FLA's ``fused_recurrent_kda`` as the reference's
    tests call it for their gold (``tests/test_kda_bt16.py:26-38``); the
    reference itself has no recurrent kernel (its roadmap lists the decode
    step, ``README.md:503-505``).  Differences from :func:`kda_bt16_fwd`:

    * without ``use_gate_in_kernel``, ``g`` is the per-token log decay
      (``alpha_t = exp(g_t)``), not a chunk-local cumsum;
    * ``output_dtype`` is bf16 or fp32 (fp32 makes this an on-GPU gold);
    * ``inplace_final_state`` writes the final state into ``initial_state``
      and returns it as ``ht`` (a decode step that allocates no state).

    Returns ``(o [B, T, HV, V], ht or None)``.
    """
    B, T, H, K, HV, V = _validate_kda_inputs(
        q, k, v, g, beta, initial_state, use_gate_in_kernel, True, lower_bound,
        A_log, dt_bias, state_v_first, cu_seqlens,
    )
    S = B if cu_seqlens is None else cu_seqlens.numel() - 1
    if output_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"output_dtype must be bfloat16 or float32, got {output_dtype}")
    if inplace_final_state and initial_state is None:
        raise ValueError("inplace_final_state requires initial_state")
    _require_gpu(q)
    if scale is None:
        scale = K ** -0.5
    dev = q.device
    q, k, v, g = (_aligned(x) for x in (q, k, v, g))
    h0 = initial_state
    if h0 is not None and h0.data_ptr() % 16 != 0:
        if inplace_final_state:
            raise ValueError("inplace_final_state needs a 16-byte aligned initial_state")
        h0 = h0.clone()
    o = torch.empty((B, T, HV, V), dtype=output_dtype, device=dev)
    ht = None
    if inplace_final_state:
        ht = initial_state
    elif output_final_state:
        ht = torch.empty((S, HV, V, K) if state_v_first else (S, HV, K, V),
                         dtype=torch.float32, device=dev)
    flags = _flags(use_gate_in_kernel, use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel,
                   state_v_first, g_log=True)
    if output_dtype == torch.float32:
        flags |= _hip.O_FP32
    args = _make_args(
        q, k, v, g, beta, scale, lower_bound if use_gate_in_kernel else None,
        A_log, dt_bias, h0, o, ht, None, 0, flags, None, cu_seqlens,
    )
    _hip.call("kda_recurrent_fwd_hip", args, torch.cuda.current_stream(dev).cuda_stream)
    return o, ht


def kda_decode_step(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    state: torch.Tensor,
    **kwargs,
) -> torch.Tensor:
    """One decode step (``q``, ``k``, ... with T == 1; any T works): updates
    ``state`` in place and returns ``o``.  Keyword arguments are those of
    :func:`kda_recurrent_fwd`."""
    o, _ = kda_recurrent_fwd(q, k, v, g, beta, initial_state=state,
                             inplace_final_state=True, **kwargs)
    return o


def kda_bt16_kernel_fused(*_args, **_kwargs):
    """The reference exports its single-kernel variant as a raw Triton kernel
    (kernels.py:305-472) launched with grid syntax; here the fused kernel is
    reached through ``kda_bt16_fwd(use_fused_kernel=True)``."""
    raise NotImplementedError(
        "kda_bt16_kernel_fused is not a launchable object on MI355X; "
        "kda_bt16_fwd(use_fused_kernel=True) runs the fused HIP kernel"
    )

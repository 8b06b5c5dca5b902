"""ctypes binding of ``libkda_bt16_hip.so`` (C ABI in ``include/kda_bt16_hip.h``).

The library is loaded lazily on first use.  There is no fallback: if the
library is missing or fails to load, every call raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkda_bt16_hip.so"

ABI_VERSION = 4

USE_GATE = 1 << 0
USE_QK_L2NORM = 1 << 1
USE_BETA_SIGMOID = 1 << 2
STATE_V_FIRST = 1 << 3
O_FP32 = 1 << 4  # token recurrence only
G_LOG_DECAY = 1 << 5  # without USE_GATE: g is the per-token natural-log decay
FUSED_KERNEL = 1 << 6  # forward entries: the fused kernel whatever the geometry
TWO_STAGE = 1 << 7  # forward entries: stage 1 then stage 2 whatever the geometry

# Bytes of the static scratch of kda_bt16_fwd_noalloc_hip, and the code it
# returns for a geometry whose records do not fit.
NOALLOC_MAX_WORKSPACE = 96 << 20
ESCRATCH = -7

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_I32 = 2
DTYPE_I64 = 3

EXPORTED_SYMBOLS = (
    "kda_bt16_workspace_bytes",
    "kda_bt16_workspace_bytes_args",
    "kda_bt16_fwd_hip",
    "kda_bt16_fwd_plan",
    "kda_bt16_fwd_segments",
    "kda_bt16_fwd_noalloc_hip",
    "kda_bt16_k1_hip",
    "kda_bt16_k2_hip",
    "kda_recurrent_fwd_hip",
    "kda_bt16_bwd_workspace_bytes",
    "kda_bt16_bwd_hip",
    "kda_bt16_saved_bytes",
    "kda_bt16_fwd_save_hip",
    "kda_bt16_bwd_saved_workspace_bytes",
    "kda_bt16_bwd_saved_hip",
    "kda_bt16_fused_aborts",
    "kda_bt16_strerror",
    "kda_bt16_abi_version",
)


class KdaBt16Args(ctypes.Structure):
    """Mirror of ``struct KdaBt16Args``."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("B", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("HV", ctypes.c_int32),
        ("K", ctypes.c_int32),
        ("V", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("scale", ctypes.c_float),
        ("lower_bound", ctypes.c_float),
        ("g_dtype", ctypes.c_int32),
        ("beta_dtype", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("g", ctypes.c_void_p),
        ("beta", ctypes.c_void_p),
        ("A_log", ctypes.c_void_p),
        ("dt_bias", ctypes.c_void_p),
        ("h0", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("ht", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("dbg_Aqk", ctypes.c_void_p),
        ("dbg_A_inv", ctypes.c_void_p),
        ("dbg_w", ctypes.c_void_p),
        ("dbg_u", ctypes.c_void_p),
        ("dbg_g", ctypes.c_void_p),
        ("cu_seqlens", ctypes.c_void_p),
        ("cu_seqlens_dtype", ctypes.c_int32),
        ("N", ctypes.c_int32),
        ("k2_tiles", ctypes.c_int32),
        ("k2_wave_tiles", ctypes.c_int32),
        ("max_seqlen", ctypes.c_int32),
    ]


class KdaBt16BwdArgs(ctypes.Structure):
    """Mirror of ``struct KdaBt16BwdArgs``."""

    _fields_ = [
        ("fwd", ctypes.POINTER(KdaBt16Args)),
        ("dout", ctypes.c_void_p),
        ("dht", ctypes.c_void_p),
        ("dq", ctypes.c_void_p),
        ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p),
        ("dg", ctypes.c_void_p),
        ("dbeta", ctypes.c_void_p),
        ("dA_log", ctypes.c_void_p),
        ("ddt_bias", ctypes.c_void_p),
        ("dh0", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class KdaHipError(RuntimeError):
    """A non-zero return code from the HIP library."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with code {code}: {msg}")
        self.code = code


_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH.name} is not built; run `python -m kda_bt16._build` "
                "(or __graft_entry__.build()) first"
            )
        h = ctypes.CDLL(str(LIB_PATH))
        h.kda_bt16_workspace_bytes.restype = ctypes.c_size_t
        h.kda_bt16_workspace_bytes.argtypes = [ctypes.c_int32] * 5
        h.kda_bt16_workspace_bytes_args.restype = ctypes.c_size_t
        h.kda_bt16_workspace_bytes_args.argtypes = [ctypes.POINTER(KdaBt16Args)]
        for name in ("kda_bt16_fwd_hip", "kda_bt16_fwd_noalloc_hip", "kda_bt16_k1_hip",
                     "kda_bt16_k2_hip", "kda_recurrent_fwd_hip"):
            fn = getattr(h, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.POINTER(KdaBt16Args), ctypes.c_void_p]
        h.kda_bt16_bwd_workspace_bytes.restype = ctypes.c_size_t
        h.kda_bt16_bwd_workspace_bytes.argtypes = [ctypes.POINTER(KdaBt16Args)]
        h.kda_bt16_bwd_hip.restype = ctypes.c_int
        h.kda_bt16_bwd_hip.argtypes = [ctypes.POINTER(KdaBt16BwdArgs), ctypes.c_void_p]
        for fn in (h.kda_bt16_saved_bytes, h.kda_bt16_bwd_saved_workspace_bytes):
            fn.restype = ctypes.c_size_t
            fn.argtypes = [ctypes.POINTER(KdaBt16Args)]
        h.kda_bt16_fwd_save_hip.restype = ctypes.c_int
        h.kda_bt16_fwd_save_hip.argtypes = [ctypes.POINTER(KdaBt16Args), ctypes.c_void_p,
                                            ctypes.c_size_t, ctypes.c_void_p]
        h.kda_bt16_bwd_saved_hip.restype = ctypes.c_int
        h.kda_bt16_bwd_saved_hip.argtypes = [ctypes.POINTER(KdaBt16BwdArgs), ctypes.c_void_p,
                                             ctypes.c_size_t, ctypes.c_void_p]
        h.kda_bt16_fwd_plan.restype = ctypes.c_int
        h.kda_bt16_fwd_plan.argtypes = [ctypes.POINTER(KdaBt16Args)]
        h.kda_bt16_fwd_segments.restype = ctypes.c_int
        h.kda_bt16_fwd_segments.argtypes = [ctypes.POINTER(KdaBt16Args)]
        h.kda_bt16_fused_aborts.restype = ctypes.c_int
        h.kda_bt16_fused_aborts.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.c_int32]
        h.kda_bt16_strerror.restype = ctypes.c_char_p
        h.kda_bt16_strerror.argtypes = [ctypes.c_int]
        h.kda_bt16_abi_version.restype = ctypes.c_int
        h.kda_bt16_abi_version.argtypes = []
        got = h.kda_bt16_abi_version()
        if got != ABI_VERSION:
            raise ImportError(f"{LIB_PATH.name} has ABI version {got}, expected {ABI_VERSION}")
        _lib = h
        return _lib


def workspace_bytes(B: int, T: int, HV: int, K: int, V: int) -> int:
    """Fixed-length workspace bytes (``kda_bt16_workspace_bytes``)."""
    return int(lib().kda_bt16_workspace_bytes(B, T, HV, K, V))


def workspace_bytes_args(args: KdaBt16Args) -> int:
    """Workspace bytes for any arguments, varlen included."""
    return int(lib().kda_bt16_workspace_bytes_args(ctypes.byref(args)))


def fwd_plan(args: KdaBt16Args) -> int:
    """``kda_bt16_fwd_plan``: 1 if the forward runs fused on the current
    device, 0 if stage 1 then stage 2; raises on invalid arguments."""
    rc = int(lib().kda_bt16_fwd_plan(ctypes.byref(args)))
    if rc < 0:
        raise RuntimeError(f"kda_bt16_fwd_plan: {lib().kda_bt16_strerror(rc).decode()}")
    return rc


def fwd_segments(args: KdaBt16Args) -> int:
    """``kda_bt16_fwd_segments``: 0 if the forward runs fused, else the
    number of chunk ranges its two stages run in turn (1-4); raises on
    invalid arguments."""
    rc = int(lib().kda_bt16_fwd_segments(ctypes.byref(args)))
    if rc < 0:
        raise RuntimeError(f"kda_bt16_fwd_segments: {lib().kda_bt16_strerror(rc).decode()}")
    return rc


def fused_aborts(reset: bool = False) -> int:
    """``kda_bt16_fused_aborts``: fused-kernel work-groups on the current
    device that gave up a bounded wait (the o columns and final-state rows
    of their compute waves still running are NaN) since load or the last
    reset.  Waits for the device's work."""
    n = ctypes.c_uint32(0)
    rc = int(lib().kda_bt16_fused_aborts(ctypes.byref(n), 1 if reset else 0))
    if rc != 0:
        raise KdaHipError("kda_bt16_fused_aborts", rc, lib().kda_bt16_strerror(rc).decode())
    return int(n.value)


def bwd_workspace_bytes(args: KdaBt16Args) -> int:
    """Backward workspace bytes (``kda_bt16_bwd_workspace_bytes``)."""
    return int(lib().kda_bt16_bwd_workspace_bytes(ctypes.byref(args)))


def saved_bytes(args: KdaBt16Args) -> int:
    """Bytes of a training forward's saved state (``kda_bt16_saved_bytes``)."""
    return int(lib().kda_bt16_saved_bytes(ctypes.byref(args)))


def bwd_saved_workspace_bytes(args: KdaBt16Args) -> int:
    """Workspace bytes of the backward from saved state."""
    return int(lib().kda_bt16_bwd_saved_workspace_bytes(ctypes.byref(args)))


def call_saved(name: str, args, saved: int, nbytes: int, stream: int) -> None:
    """``kda_bt16_fwd_save_hip`` / ``kda_bt16_bwd_saved_hip``: args, the
    saved-state buffer, its size, the stream."""
    rc = getattr(lib(), name)(ctypes.byref(args), ctypes.c_void_p(saved),
                              ctypes.c_size_t(nbytes), ctypes.c_void_p(stream))
    if rc != 0:
        raise KdaHipError(name, rc, lib().kda_bt16_strerror(rc).decode())


def call(name: str, args, stream: int) -> None:
    rc = getattr(lib(), name)(ctypes.byref(args), ctypes.c_void_p(stream))
    if rc != 0:
        raise KdaHipError(name, rc, lib().kda_bt16_strerror(rc).decode())

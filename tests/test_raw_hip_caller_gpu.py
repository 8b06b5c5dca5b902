"""The C ABI driven the way a caller without torch drives it: device buffers
from hipMalloc, inputs copied in with hipMemcpy, a workspace sized by
kda_bt16_workspace_bytes_args, kda_bt16_fwd_hip on a stream of the caller's
own (hipStreamCreate), results copied back after hipStreamSynchronize.  Only
ctypes, the HIP runtime library and the header's argument struct are
involved; the outputs equal kda_bt16_fwd's (the torch path) bit for bit for
a two-stage geometry with a partial last chunk and an initial state, the
fused kernel on the same inputs, and packed sequences of grouped value
heads with an empty sequence and 32-bit offsets.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from kda_bt16 import _hip, kda_bt16_fwd
from kda_bt16.kernels import _flags

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2  # hipMemcpyHostToDevice, hipMemcpyDeviceToHost


def _loaded_hip_runtime() -> str:
    """The HIP runtime this process already has mapped (the one
    libkda_bt16_hip.so resolved its libamdhip64 dependency to: inside a
    torch process, torch's own), so that the raw calls and the library
    share one runtime."""
    _hip.lib()
    with open("/proc/self/maps") as f:
        paths = {ln.split()[-1] for ln in f if "libamdhip64" in ln}
    assert len(paths) == 1, f"expected one HIP runtime in the process, found {sorted(paths)}"
    return paths.pop()


LB, SCALE = -5.0, 128 ** -0.5


class RawHip:
    """hipMalloc / hipMemcpy / streams through ctypes, every buffer freed at
    close()."""

    def __init__(self):
        h = ctypes.CDLL(_loaded_hip_runtime())
        h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        h.hipFree.argtypes = [ctypes.c_void_p]
        h.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        h.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
        h.hipStreamDestroy.argtypes = [ctypes.c_void_p]
        for f in (h.hipMalloc, h.hipMemcpy, h.hipFree, h.hipStreamCreate, h.hipStreamSynchronize,
                  h.hipStreamDestroy):
            f.restype = ctypes.c_int
        self.h = h
        self.bufs: list[int] = []

    def _ok(self, rc: int, what: str) -> None:
        if rc != 0:
            raise RuntimeError(f"{what} returned HIP error {rc}")

    def alloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        self._ok(self.h.hipMalloc(ctypes.byref(p), max(nbytes, 1)), "hipMalloc")
        self.bufs.append(p.value)
        return p.value

    def upload(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        p = self.alloc(a.nbytes)
        self._ok(self.h.hipMemcpy(p, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return p

    def download(self, p: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        self._ok(self.h.hipMemcpy(out.ctypes.data, p, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def close(self) -> None:
        for p in self.bufs:
            self.h.hipFree(p)
        self.bufs = []


def _bits(t: torch.Tensor) -> np.ndarray:
    """A CPU tensor's bytes as numpy (bf16 as its int16 bit patterns)."""
    t = t.contiguous()
    return (t.view(torch.int16) if t.dtype == torch.bfloat16 else t).numpy()


def _inputs(B, T, H, HV, seed, h0):
    gen = torch.Generator().manual_seed(seed)
    c = dict(
        q=torch.randn(B, T, H, 128, generator=gen).bfloat16(),
        k=torch.randn(B, T, H, 128, generator=gen).bfloat16(),
        v=torch.randn(B, T, HV, 128, generator=gen).bfloat16(),
        g=torch.randn(B, T, HV, 128, generator=gen).bfloat16(),
        beta=torch.randn(B, T, HV, generator=gen).bfloat16(),
        A_log=torch.log(torch.rand(HV, generator=gen) * 15 + 1),
        dt_bias=torch.randn(HV * 128, generator=gen) * 0.1,
    )
    c["h0"] = torch.randn(B, HV, 128, 128, generator=gen) * 0.05 if h0 else None
    return c


def _raw_forward(c, fused, cu=None):
    """o (bf16 bits) and ht through kda_bt16_fwd_hip on raw HIP memory."""
    hip = RawHip()
    stream = ctypes.c_void_p()
    hip._ok(hip.h.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")
    try:
        B, T, H = c["q"].shape[:3]
        HV = c["v"].shape[2]
        S = B if cu is None else len(cu) - 1
        a = _hip.KdaBt16Args()
        a.abi_version = _hip.ABI_VERSION
        a.B, a.T, a.H, a.HV, a.K, a.V = B, T, H, HV, 128, 128
        a.flags = _flags(True, True, True, True, fused=fused)
        a.scale, a.lower_bound = SCALE, LB
        a.g_dtype = a.beta_dtype = _hip.DTYPE_BF16
        a.q, a.k, a.v, a.g, a.beta = (hip.upload(_bits(c[x])) for x in ("q", "k", "v", "g", "beta"))
        a.A_log = hip.upload(_bits(c["A_log"]))
        a.dt_bias = hip.upload(_bits(c["dt_bias"]))
        if c["h0"] is not None:
            a.h0 = hip.upload(_bits(c["h0"]))
        a.o = hip.alloc(B * T * HV * 128 * 2)
        a.ht = hip.alloc(S * HV * 128 * 128 * 4)
        if cu is not None:
            a.cu_seqlens = hip.upload(np.asarray(cu, dtype=np.int32))
            a.cu_seqlens_dtype = _hip.DTYPE_I32
            a.N = S
        need = _hip.workspace_bytes_args(a)
        plan = _hip.fwd_plan(a)
        if plan == 0:  # the fused forward reads no workspace
            a.workspace = hip.alloc(need)
            a.workspace_bytes = need
        rc = _hip.lib().kda_bt16_fwd_hip(ctypes.byref(a), stream)
        assert rc == 0, _hip.lib().kda_bt16_strerror(rc).decode()
        hip._ok(hip.h.hipStreamSynchronize(stream), "hipStreamSynchronize")
        o = hip.download(a.o, (B, T, HV, 128), np.int16)
        ht = hip.download(a.ht, (S, HV, 128, 128), np.float32)
        return plan, o, ht
    finally:
        hip.h.hipStreamSynchronize(stream)
        hip.h.hipStreamDestroy(stream)
        hip.close()


CASES = {
    # B=2 T=1037 H=4: 8 (row, head) pairs, two stages; a partial last chunk, h0
    "two_stage": dict(shape=(2, 1037, 4, 4), seed=3, h0=True, fused=False, cu=None, plan=0),
    "fused": dict(shape=(2, 1037, 4, 4), seed=3, h0=True, fused=True, cu=None, plan=1),
    # packed sequences (one empty), grouped value heads, 32-bit offsets
    "varlen_gva": dict(shape=(1, 300, 2, 4), seed=5, h0=False, fused=False,
                       cu=[0, 37, 37, 160, 300], plan=0),
}


@pytest.mark.parametrize("name", list(CASES))
def test_raw_hip_caller_equals_torch_path(name, gpu_device):
    case = CASES[name]
    print(f"raw HIP caller case {name}", flush=True)
    B, T, H, HV = case["shape"]
    c = _inputs(B, T, H, HV, case["seed"], case["h0"])
    plan, o, ht = _raw_forward(c, case["fused"], case["cu"])
    assert plan == case["plan"], name

    dev = gpu_device
    cu = None if case["cu"] is None else torch.tensor(case["cu"], dtype=torch.int32, device=dev)
    h0 = None if c["h0"] is None else c["h0"].to(dev)
    o_ref, ht_ref = kda_bt16_fwd(
        *(c[x].to(dev) for x in ("q", "k", "v", "g", "beta")), scale=SCALE, initial_state=h0,
        output_final_state=True, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
        use_beta_sigmoid_in_kernel=True, lower_bound=LB, A_log=c["A_log"].to(dev),
        dt_bias=c["dt_bias"].to(dev), state_v_first=True, cu_seqlens=cu,
        use_fused_kernel=case["fused"])
    torch.cuda.synchronize()
    assert np.isfinite(ht).all(), name
    assert np.array_equal(o, _bits(o_ref.cpu())), f"{name}: o differs"
    assert np.array_equal(ht.view(np.int32), ht_ref.cpu().numpy().view(np.int32)), f"{name}: ht differs"

"""kda_bt16_fwd_noalloc_hip: the forward whose records live in the library's
static device scratch instead of a workspace.  It must give what
kda_bt16_fwd_hip gives, bit for bit, on consecutive calls that leave the
scratch holding the previous call's records (each call here is smaller than
the one before), take a fused geometry of any size (the fused forward keeps
its records in LDS), run a fixed-length two-stage geometry whose records
outgrow the scratch in chunk ranges that fit, and refuse one that cannot
fit even so before any launch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from kda_bt16 import _hip, kda_bt16_fwd
from kda_bt16.kernels import _flags, _make_args


def _args(**kw):
    a = _hip.KdaBt16Args()
    a.abi_version = _hip.ABI_VERSION
    a.B, a.T, a.H, a.HV, a.K, a.V = 1, 16, 1, 1, 128, 128
    a.scale = 0.1
    a.lower_bound = -5.0
    for name, val in kw.items():
        setattr(a, name, val)
    return a


@pytest.mark.skipif(torch.cuda.is_available(),
                    reason="stand-in device pointers are passed to a launching entry point only "
                           "where no GPU is present")
def test_noalloc_refuses_oversized_geometry_without_launching():
    fake = 1 << 40  # never dereferenced: the size check fails before any launch
    full = dict(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake)
    f = _hip.lib().kda_bt16_fwd_noalloc_hip
    # on the two-stage path (a fused geometry would launch: checked first)
    # 1280 (row, value head) pairs carry 80 MiB of state between chunk
    # ranges: with one chunk's records it outgrows the scratch
    a = _args(B=1, T=2048, H=1280, HV=1280, flags=_hip.TWO_STAGE, **full)
    assert _hip.workspace_bytes_args(a) > _hip.NOALLOC_MAX_WORKSPACE
    assert 1280 * (17408 + 128 * 128 * 4) > _hip.NOALLOC_MAX_WORKSPACE
    assert _hip.fwd_plan(a) == 0
    assert f(ctypes.byref(a), None) == _hip.ESCRATCH
    # packed sequences run in one pass: 272 MiB of records do not fit
    v = _args(B=1, T=8192, H=32, HV=32, N=8, cu_seqlens=fake, cu_seqlens_dtype=_hip.DTYPE_I32,
              flags=_hip.TWO_STAGE, **full)
    assert _hip.workspace_bytes_args(v) > _hip.NOALLOC_MAX_WORKSPACE
    assert f(ctypes.byref(v), None) == _hip.ESCRATCH
    assert b"static" in _hip.lib().kda_bt16_strerror(_hip.ESCRATCH)
    # the ordinary argument checks come first
    assert f(None, None) == -1
    assert f(ctypes.byref(_args(K=64, **full)), None) == -2
    assert f(ctypes.byref(_args()), None) == -1  # missing tensors


def _case(B, T, H, HV, seed, *, h0, svf, varlen=None):
    """q/k [B, T, H], the rest [B, T, HV] (the BASELINE generators); states
    for B rows, or for the sequences of ``varlen``."""
    gen = torch.Generator().manual_seed(seed)
    S = B if varlen is None else len(varlen) - 1
    c = dict(
        q=torch.randn(B, T, H, 128, generator=gen).bfloat16(),
        k=torch.randn(B, T, H, 128, generator=gen).bfloat16(),
        v=torch.randn(B, T, HV, 128, generator=gen).bfloat16(),
        g=torch.randn(B, T, HV, 128, generator=gen).bfloat16(),
        beta=torch.randn(B, T, HV, generator=gen).bfloat16(),
        A_log=torch.log(torch.rand(HV, generator=gen) * 15 + 1),
        dt_bias=torch.randn(HV * 128, generator=gen) * 0.1,
        h0=torch.randn(S, HV, 128, 128, generator=gen) * 0.05 if h0 else None,
    )
    c["cu"] = None if varlen is None else torch.tensor(varlen, dtype=torch.int32)
    c["svf"] = svf
    return c


def _run_both(c, dev):
    q, k, v, g, beta = (c[x].to(dev) for x in ("q", "k", "v", "g", "beta"))
    A_log, dt_bias = c["A_log"].to(dev), c["dt_bias"].to(dev)
    h0 = None if c.get("h0") is None else c["h0"].to(dev)
    cu = None if c["cu"] is None else c["cu"].to(dev)
    kw = dict(scale=0.1, initial_state=h0, output_final_state=True,
              use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              use_beta_sigmoid_in_kernel=True, lower_bound=-5.0, A_log=A_log,
              dt_bias=dt_bias, state_v_first=c["svf"], cu_seqlens=cu)
    o_ref, ht_ref = kda_bt16_fwd(q, k, v, g, beta, **kw)
    B, T, H, _ = q.shape
    HV = v.shape[2]
    S = B if cu is None else cu.numel() - 1
    o = torch.full((B, T, HV, 128), float("nan"), dtype=torch.bfloat16, device=dev)
    ht = torch.full((S, HV, 128, 128), float("nan"), dtype=torch.float32, device=dev)
    args = _make_args(q, k, v, g, beta, 0.1, -5.0, A_log, dt_bias, h0, o, ht, None, 0,
                      _flags(True, True, True, c["svf"]), None, cu)
    # a two-stage geometry fits the scratch, or runs in chunk ranges that
    # do (fixed length); a fused one needs none
    assert (_hip.workspace_bytes_args(args) <= _hip.NOALLOC_MAX_WORKSPACE
            or _hip.fwd_plan(args) == 1 or cu is None)
    _hip.call("kda_bt16_fwd_noalloc_hip", args, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize(dev)
    return (o_ref, ht_ref), (o, ht)


@pytest.mark.gpu
def test_noalloc_equals_fwd_on_consecutive_calls(gpu_device):
    cases = [
        # two stages, 272 MiB of records: in chunk ranges that fit the
        # scratch (3 of 171 chunks, 95 MB of records and the state)
        ("B1_T8192_H32_ranges", _case(1, 8192, 32, 32, seed=8, h0=True, svf=True)),
        # fused (512 (sequence, head) pairs): 16384 records' worth (272 MiB),
        # more than the scratch holds, which the fused forward does not use
        ("B16_T512_H32_fused", _case(16, 512, 32, 32, seed=7, h0=True, svf=True)),
        # near the scratch's size: 4096 records (68 MiB), h0, V-first
        ("B2_T4096_H8", _case(2, 4096, 8, 8, seed=3, h0=True, svf=True)),
        # smaller: 8 rows x 8 value heads, so stage 2 runs several sequences
        # per work-group
        ("B8_T300_HV8", _case(8, 300, 2, 8, seed=6, h0=True, svf=True)),
        # smaller, partial last chunk, K-first state
        ("B2_T1037_H4_kfirst", _case(2, 1037, 4, 4, seed=4, h0=True, svf=False)),
        # smaller again: grouped value heads, packed sequences with an empty one
        ("varlen_gva", _case(1, 300, 2, 4, seed=5, h0=False, svf=True,
                             varlen=[0, 37, 37, 160, 300])),
    ]
    for name, c in cases:
        print(f"noalloc case {name}", flush=True)
        (o_ref, ht_ref), (o, ht) = _run_both(c, gpu_device)
        assert torch.isfinite(o_ref.float()).all(), name
        assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16)), f"{name}: o differs"
        assert torch.equal(ht.view(torch.int32), ht_ref.view(torch.int32)), f"{name}: ht differs"


@pytest.mark.gpu
@pytest.mark.parametrize("B,T,H", [(2, 1024, 4), (16, 256, 32)], ids=["two_stage", "fused"])
def test_noalloc_graph_replays_equal_fwd(B, T, H, gpu_device):
    """kda_bt16_fwd_noalloc_hip captured into a HIP graph (torch.cuda.CUDAGraph)
    after one eager call on the device (which looks up the scratch's
    address), replayed on new inputs copied into the captured buffers, with
    eager work and a synchronisation between replays: every replay equals
    kda_bt16_fwd on the same inputs, bit for bit."""
    dev = gpu_device
    print(f"[noalloc graph] B={B} T={T} H={H}", flush=True)
    cases = [_case(B, T, H, H, seed=20 + i, h0=True, svf=True) for i in range(3)]
    for c in cases:
        for x in ("q", "k", "v", "g", "beta", "A_log", "dt_bias", "h0"):
            c[x] = c[x].to(dev)
    kw = dict(scale=0.1, output_final_state=True, use_qk_l2norm_in_kernel=True,
              use_gate_in_kernel=True, use_beta_sigmoid_in_kernel=True, lower_bound=-5.0)
    eager = []
    for c in cases:
        o, ht = kda_bt16_fwd(c["q"], c["k"], c["v"], c["g"], c["beta"], initial_state=c["h0"],
                             A_log=c["A_log"], dt_bias=c["dt_bias"], **kw)
        eager.append((o.clone(), ht.clone()))
    names = ("q", "k", "v", "g", "beta", "A_log", "dt_bias", "h0")
    st = {x: cases[0][x].clone() for x in names}
    o = torch.empty(B, T, H, 128, dtype=torch.bfloat16, device=dev)
    ht = torch.empty(B, H, 128, 128, dtype=torch.float32, device=dev)
    args = _make_args(st["q"], st["k"], st["v"], st["g"], st["beta"], 0.1, -5.0, st["A_log"],
                      st["dt_bias"], st["h0"], o, ht, None, 0, _flags(True, True, True, True))
    fused = _hip.fwd_plan(args) == 1
    assert fused == (B * H * 2 > torch.cuda.get_device_properties(dev).multi_processor_count)
    # the eager call first: on the two-stage path it looks up the scratch
    _hip.call("kda_bt16_fwd_noalloc_hip", args, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize(dev)
    assert torch.equal(o, eager[0][0]) and torch.equal(ht, eager[0][1])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _hip.call("kda_bt16_fwd_noalloc_hip", args, torch.cuda.current_stream(dev).cuda_stream)
    for i, c in enumerate(cases):
        for x in names:
            st[x].copy_(c[x])
        o.fill_(float("nan"))
        ht.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize(dev)
        _ = float(torch.randn(4096, device=dev).square().sum())  # eager work between replays
        assert torch.equal(o.view(torch.int16), eager[i][0].view(torch.int16)), f"replay {i}: o"
        assert torch.equal(ht.view(torch.int32), eager[i][1].view(torch.int32)), f"replay {i}: ht"

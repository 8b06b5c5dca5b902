"""The C ABI library loads and exports what include/kda_bt16_hip.h declares;
host-side argument checks return their error codes without launching (CPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from kda_bt16 import _hip

HEADER = Path(__file__).resolve().parents[1] / "include" / "kda_bt16_hip.h"

# Tests that hand a launching entry point stand-in device pointers (1 << 40)
# rely on its argument checks failing before any launch.  Without a GPU no
# launch can happen whatever the checks do; on a GPU box they are skipped,
# so that a regressed check can never launch a kernel on such an address.
fake_pointers = pytest.mark.skipif(
    torch.cuda.is_available(),
    reason="stand-in device pointers are passed to launching entry points only where no GPU is present")


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kda_\w+)\s*\(", text)))


def test_header_declares_the_binding_symbols():
    assert _declared_functions() == sorted(_hip.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _hip.lib()
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_header_constants_match_binding():
    text = HEADER.read_text()
    consts = dict(re.findall(r"#define\s+(KDA_BT16_\w+)\s+\(?([^\s/]+)", text))
    assert int(consts["KDA_BT16_ABI_VERSION"]) == _hip.ABI_VERSION
    assert consts["KDA_BT16_USE_GATE"] == "1u" or "1u << 0" in text
    assert _hip.lib().kda_bt16_abi_version() == _hip.ABI_VERSION


def test_struct_layout_matches_header_field_order():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct KdaBt16Args \{(.*?)\} KdaBt16Args;", text, re.S).group(1)
    names = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        names += [n.strip().lstrip("*") for n in re.sub(r"^.*?\b(?=\w+\s*(,|$))", "", decl).split(",")]
    fields = [f for f, _ in _hip.KdaBt16Args._fields_]
    assert names == fields


def test_workspace_bytes():
    ws = _hip.workspace_bytes
    assert ws(1, 8192, 32, 128, 128) == 32 * 512 * 17408
    assert ws(2, 1037, 4, 128, 128) == 2 * 4 * 65 * 17408
    assert ws(1, 16, 1, 64, 128) == 0
    assert ws(0, 16, 1, 128, 128) == 0
    # by arguments: value heads count, and varlen takes HV * (T // 16 + N) slots
    assert _hip.workspace_bytes_args(_args(B=2, T=1037, H=2, HV=4)) == 2 * 4 * 65 * 17408
    fake = 1 << 40
    a = _args(T=1000, H=2, HV=4, cu_seqlens=fake, cu_seqlens_dtype=_hip.DTYPE_I64, N=7)
    assert _hip.workspace_bytes_args(a) == 4 * (1000 // 16 + 7) * 17408
    assert _hip.workspace_bytes_args(_args(cu_seqlens=fake, N=0)) == 0


@fake_pointers
def test_varlen_argument_checks():
    fake = 1 << 40  # never dereferenced: argument checks fail first
    vl = dict(cu_seqlens=fake, cu_seqlens_dtype=_hip.DTYPE_I64, N=3)
    for fn in ("kda_bt16_fwd_hip", "kda_recurrent_fwd_hip"):
        f = getattr(_hip.lib(), fn)
        assert f(ctypes.byref(_args(B=2, **vl)), None) == -1  # packed sequences need B == 1
        assert f(ctypes.byref(_args(**{**vl, "N": 0})), None) == -1
        assert f(ctypes.byref(_args(**{**vl, "cu_seqlens_dtype": 0})), None) == -1
        assert f(ctypes.byref(_args(**{**vl, "cu_seqlens": fake + 4})), None) == -1
        assert f(ctypes.byref(_args(**{**vl, "cu_seqlens": fake + 4,
                                       "cu_seqlens_dtype": _hip.DTYPE_I32})), None) == -1  # no tensors
    # workspace sized for the fixed-length layout is too small for varlen
    full = dict(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake, workspace=fake)
    a = _args(T=64, **full, **vl, workspace_bytes=4 * 17408)
    assert _hip.lib().kda_bt16_fwd_hip(ctypes.byref(a), None) == -3


def test_strerror_codes():
    lib = _hip.lib()
    for code in (0, -1, -2, -3, -4, -5, -6, -7):
        assert lib.kda_bt16_strerror(code)
    assert lib.kda_bt16_strerror(-99) == b"unknown error"


def _args(**kw):
    a = _hip.KdaBt16Args()
    a.abi_version = _hip.ABI_VERSION
    a.B, a.T, a.H, a.HV, a.K, a.V = 1, 16, 1, 1, 128, 128
    a.scale = 0.1
    a.lower_bound = -5.0
    for name, val in kw.items():
        setattr(a, name, val)
    return a


@pytest.mark.parametrize("fn", ["kda_bt16_fwd_hip", "kda_bt16_k1_hip", "kda_bt16_k2_hip"])
@fake_pointers
def test_argument_checks_return_codes_without_launching(fn):
    f = getattr(_hip.lib(), fn)
    assert f(None, None) == -1
    assert f(ctypes.byref(_args(abi_version=99)), None) == -5
    assert f(ctypes.byref(_args(K=64)), None) == -2
    assert f(ctypes.byref(_args(H=2, HV=3)), None) == -2  # HV not a multiple of H
    assert f(ctypes.byref(_args(T=1973776 + 1)), None) == -2  # 32-bit per-head record size
    assert f(ctypes.byref(_args(T=0)), None) == -1
    assert f(ctypes.byref(_args(g_dtype=7)), None) == -1
    assert f(ctypes.byref(_args(flags=_hip.USE_GATE, lower_bound=-12.0)), None) == -6
    # missing tensors (stage 1 / full) or output (stage 2)
    assert f(ctypes.byref(_args()), None) == -1
    with pytest.raises(_hip.KdaHipError, match="code -1"):
        _hip.call(fn, _args(), 0)


def test_forward_plan_reads_no_device_memory():
    """kda_bt16_fwd_plan: argument checks, the caller's choice through the
    flags, and the two stages whenever debug outputs are asked for (they
    come from stage 1).  Pointers are never dereferenced and nothing is
    launched."""
    f = _hip.lib().kda_bt16_fwd_plan
    fake = 1 << 40
    ten = dict(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake)
    assert f(None) == -1
    assert f(ctypes.byref(_args(K=64, **ten))) == -2
    assert f(ctypes.byref(_args())) == -1  # missing tensors
    assert f(ctypes.byref(_args(B=16, H=32, HV=32, **ten))) == 1
    assert f(ctypes.byref(_args(B=16, H=32, HV=32, flags=_hip.TWO_STAGE, **ten))) == 0
    assert f(ctypes.byref(_args(**ten))) == 0
    assert f(ctypes.byref(_args(flags=_hip.FUSED_KERNEL, **ten))) == 1
    dbg = dict(dbg_Aqk=fake, dbg_A_inv=fake, dbg_w=fake, dbg_u=fake, dbg_g=fake)
    # debug outputs win over the caller's request
    assert f(ctypes.byref(_args(flags=_hip.FUSED_KERNEL, **ten, **dbg))) == 0
    assert _hip.fwd_plan(_args(flags=_hip.FUSED_KERNEL, **ten)) == 1
    # both requests at once, and kernel choices out of range, are refused
    assert f(ctypes.byref(_args(flags=_hip.FUSED_KERNEL | _hip.TWO_STAGE, **ten))) == -1
    for bad in (dict(k2_tiles=3), dict(k2_tiles=16), dict(k2_tiles=-1), dict(k2_wave_tiles=3),
                dict(k2_wave_tiles=-1), dict(max_seqlen=-1)):
        assert f(ctypes.byref(_args(**ten, **bad))) == -1, bad
    for ok in (dict(k2_tiles=1), dict(k2_tiles=8, k2_wave_tiles=1), dict(max_seqlen=16)):
        assert f(ctypes.byref(_args(**ten, **ok))) == 0, ok


@pytest.mark.parametrize("env", [{"KDA_BT16_FUSED": "1"}, {"KDA_BT16_FUSED": "0"},
                                 {"KDA_BT16_K2_TILES": "2", "KDA_BT16_K2_WAVE_TILES": "2"}])
def test_forward_plan_ignores_the_environment(monkeypatch, env):
    """The choice depends on the arguments only: variables that once
    overrode it change nothing."""
    f = _hip.lib().kda_bt16_fwd_plan
    fake = 1 << 40
    ten = dict(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake)
    shapes = [dict(), dict(B=16, H=32, HV=32), dict(B=1, H=129, HV=129),
              dict(N=8, H=32, HV=32, T=4096, cu_seqlens=fake, cu_seqlens_dtype=_hip.DTYPE_I32)]
    before = [f(ctypes.byref(_args(**ten, **sh))) for sh in shapes]
    for name, val in env.items():
        monkeypatch.setenv(name, val)
    assert [f(ctypes.byref(_args(**ten, **sh))) for sh in shapes] == before


def test_forward_plan_thresholds():
    """Without the caller's choice, fixed length fuses once the (sequence,
    value head) pairs are more than half the CUs, cu_seqlens once they are
    at least as many as the CUs.  Without a GPU the library counts 256 CUs,
    the MI355X's count."""
    f = _hip.lib().kda_bt16_fwd_plan
    fake = 1 << 40
    ten = dict(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake)

    def plan(**kw):
        return f(ctypes.byref(_args(**ten, **kw)))

    assert plan(B=1, H=128, HV=128) == 0
    assert plan(B=1, H=129, HV=129) == 1
    assert plan(B=2, H=32, HV=64) == 0  # 128 pairs through grouped value heads
    assert plan(B=5, H=32, HV=32) == 1
    cu = dict(cu_seqlens=fake, cu_seqlens_dtype=_hip.DTYPE_I32, T=4096)
    assert plan(N=7, H=32, HV=32, **cu) == 0  # 224 pairs
    assert plan(N=8, H=32, HV=32, **cu) == 1  # 256 pairs
    # max_seqlen is only read with cu_seqlens
    assert plan(B=5, H=32, HV=32, max_seqlen=16) == 1


def test_forward_segments():
    """kda_bt16_fwd_segments: 0 when the forward runs fused; for the two
    stages, one pass up to 200 MB of records, above that one chunk range
    per ~150 MB of records (at most 64, each of at least 64 chunks), at any
    number of stage-2 value tiles per work-group; one pass with packed
    sequences or debug outputs.  Without a GPU the library counts 256 CUs.  Pointers are
    never dereferenced and nothing is launched."""
    f = _hip.lib().kda_bt16_fwd_segments
    fake = 1 << 40
    ten = dict(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake)

    def segs(**kw):
        return f(ctypes.byref(_args(**ten, **kw)))

    assert f(None) == -1
    assert segs(K=64) == -2
    assert segs(B=16, T=2048, H=32, HV=32) == 0                  # fused
    assert segs(B=1, T=8192, H=32, HV=32) == 2                    # 285 MB of records
    assert segs(B=2, T=8192, H=16, HV=16) == 2                    # the same records, two rows
    assert segs(B=1, T=8192, H=16, HV=32) == 2                    # grouped value heads
    assert segs(B=1, T=8192, H=16, HV=16) == 1                    # 143 MB
    assert segs(B=1, T=8192, H=20, HV=20) == 1                    # 178 MB
    assert segs(B=1, T=4096, H=40, HV=40) == 1                    # 178 MB, 2 value tiles
    assert segs(B=1, T=8192, H=24, HV=24) == 2                    # 214 MB
    assert segs(B=2, T=4096, H=8, HV=8) == 1
    assert segs(B=1, T=16384, H=32, HV=32) == 4                   # 570 MB
    assert segs(B=1, T=8192, H=48, HV=48) == 3                    # 2 value tiles per work-group
    assert segs(B=1, T=8192, H=96, HV=96) == 6                    # 856 MB, 4 value tiles per work-group
    assert segs(B=1, T=8192, H=32, HV=32, k2_tiles=4) == 2        # forced wider work-groups
    assert segs(B=1, T=1 << 20, H=1, HV=1) == 8                   # 1.14 GB
    assert segs(B=1, T=16384, H=128, HV=128) == 16                # 2.28 GB
    assert segs(B=1, T=1 << 20, H=16, HV=16) == 64                # 18.3 GB: at most 64
    assert segs(B=1, T=8192, H=1, HV=1) == 1                      # 8.9 MB
    assert segs(B=1, T=4096, H=64, HV=64) == 2                    # 2 tiles, 285 MB
    assert segs(B=1, T=2048, H=128, HV=128) == 2                  # 285 MB, 4 tiles, 128 chunks
    assert segs(B=1, T=1024, H=256, HV=256, flags=_hip.TWO_STAGE) == 1  # 64 chunks: no room for two ranges
    assert segs(B=1, T=8192, H=32, HV=32, flags=_hip.TWO_STAGE,
                dbg_Aqk=fake, dbg_A_inv=fake, dbg_w=fake, dbg_u=fake, dbg_g=fake) == 1
    cu = dict(N=8, T=8192, cu_seqlens=fake, cu_seqlens_dtype=_hip.DTYPE_I32)
    assert segs(H=16, HV=16, **cu) == 1                           # packed: one pass
    assert _hip.fwd_segments(_args(B=1, T=8192, H=32, HV=32, **ten)) == 2


def test_forward_plan_with_max_seqlen():
    """With cu_seqlens and the longest sequence's length, the choice follows
    the estimated times: the fused kernel's is set by the longest sequence
    (~1.85 us a chunk) or the chunks per CU, the two stages' by all chunks
    (stage 1) plus the longest chain (stage 2, ~0.65 us a step).  Measured
    at 192 pairs (HV = 32): lengths 19456 + 5 x 1024, fused 2188 us against
    1146; 6 x 4096, 480 against 590."""
    f = _hip.lib().kda_bt16_fwd_plan
    fake = 1 << 40
    ten = dict(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake)

    def plan(N, T, longest, HV=32):
        cu = dict(cu_seqlens=fake, cu_seqlens_dtype=_hip.DTYPE_I32)
        return f(ctypes.byref(_args(N=N, T=T, H=HV, HV=HV, max_seqlen=longest, **cu, **ten)))

    assert plan(6, 24576, 19456) == 0  # skewed: two stages
    assert plan(6, 24576, 4096) == 1   # equal lengths: fused, below the pair-count threshold too
    assert plan(8, 16384 + 7 * 1024, 16384) == 0  # 256 pairs, one long sequence
    assert plan(8, 8 * 2944, 2944) == 1  # 256 pairs, equal
    assert plan(16, 8192, 1527) == 1  # bench's 16 packed sequences (512 pairs)
    assert plan(16, 16 * 2048, 2048) == 1  # c4's shape packed
    # a hint longer than T is read as T
    assert plan(6, 24576, 1 << 30) == plan(6, 24576, 24576)


@fake_pointers
def test_workspace_checked_before_launch():
    fake = 1 << 40  # never dereferenced: the size check fails first
    a = _args(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake, workspace=fake, workspace_bytes=100)
    assert _hip.lib().kda_bt16_fwd_hip(ctypes.byref(a), None) == -3
    a = _args(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake, workspace=fake + 8,
              workspace_bytes=17408)
    assert _hip.lib().kda_bt16_fwd_hip(ctypes.byref(a), None) == -3


@fake_pointers
def test_recurrent_entry_argument_checks():
    f = _hip.lib().kda_recurrent_fwd_hip
    assert f(None, None) == -1
    assert f(ctypes.byref(_args(abi_version=99)), None) == -5
    assert f(ctypes.byref(_args(K=64)), None) == -2
    assert f(ctypes.byref(_args(H=2, HV=3)), None) == -2  # HV not a multiple of H
    assert f(ctypes.byref(_args(T=0)), None) == -1
    assert f(ctypes.byref(_args(flags=_hip.USE_GATE, lower_bound=-12.0)), None) == -6
    assert f(ctypes.byref(_args()), None) == -1  # missing tensors
    fake = 1 << 40  # never dereferenced: argument checks fail first
    full = dict(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake)
    assert f(ctypes.byref(_args(H=2, HV=4, **full, dbg_Aqk=fake)), None) == -1  # debug outputs
    assert f(ctypes.byref(_args(**full, ht=fake + 8)), None) == -1  # 16-byte state alignment
    # q, k, v and g are read in 4-column pieces: 16-byte aligned rows
    for name in ("q", "k", "v", "g"):
        assert f(ctypes.byref(_args(**{**full, name: fake + 8})), None) == -1, name
    assert f(ctypes.byref(_args(**{**full, "o": fake + 2}, flags=_hip.O_FP32)), None) == -1


@fake_pointers
def test_o_fp32_is_refused_on_chunked_entries():
    fake = 1 << 40
    a = _args(q=fake, k=fake, v=fake, g=fake, beta=fake, o=fake, flags=_hip.O_FP32)
    assert _hip.lib().kda_bt16_fwd_hip(ctypes.byref(a), None) == -2


def test_bwd_struct_layout_matches_header_field_order():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct KdaBt16BwdArgs \{(.*?)\} KdaBt16BwdArgs;", text, re.S).group(1)
    names = [re.findall(r"(\w+)\s*$", d.strip())[0] for d in body.split(";") if d.strip()]
    assert names == [f for f, _ in _hip.KdaBt16BwdArgs._fields_]


def test_bwd_workspace_bytes():
    # per record slot: forward and backward records, bf16 h and dh, v_new and
    # dv_new, gate partials;
    # each region 256-byte aligned
    R = 32 * 512
    per = [17408, 17408, 32768, 4096, 32768, 4096, 132 * 4]
    assert _hip.bwd_workspace_bytes(_args(B=1, T=8192, H=32, HV=32)) == sum(
        (R * x + 255) // 256 * 256 for x in per)
    assert _hip.bwd_workspace_bytes(_args(K=64)) == 0


def _bwd(fwd, **kw):
    b = _hip.KdaBt16BwdArgs()
    b.fwd = ctypes.pointer(fwd)
    for name, val in kw.items():
        setattr(b, name, val)
    return b


@fake_pointers
def test_bwd_argument_checks_return_codes_without_launching():
    f = _hip.lib().kda_bt16_bwd_hip
    fake = 1 << 40  # never dereferenced: the checks fail first
    ins = dict(q=fake, k=fake, v=fake, g=fake, beta=fake)
    grads = dict(dout=fake, dq=fake, dk=fake, dv=fake, dg=fake, dbeta=fake)
    assert f(None, None) == -1
    assert f(ctypes.byref(_bwd(_args(abi_version=99), **grads)), None) == -5
    assert f(ctypes.byref(_bwd(_args(K=64, **ins), **grads)), None) == -2
    assert f(ctypes.byref(_bwd(_args(**ins), **{**grads, "dq": None})), None) == -1
    assert f(ctypes.byref(_bwd(_args(**ins, dbg_Aqk=fake), **grads)), None) == -1
    # gate-parameter gradients need the in-kernel gate (and dt_bias for ddt_bias)
    assert f(ctypes.byref(_bwd(_args(**ins), **grads, dA_log=fake)), None) == -1
    gate = _args(**ins, flags=_hip.USE_GATE, A_log=fake)
    assert f(ctypes.byref(_bwd(gate, **grads, ddt_bias=fake)), None) == -1
    assert f(ctypes.byref(_bwd(_args(**ins), **{**grads, "dv": fake + 8})), None) == -1
    # workspace missing, too small or misaligned
    assert f(ctypes.byref(_bwd(_args(**ins), **grads)), None) == -3
    assert f(ctypes.byref(_bwd(_args(**ins), **grads, workspace=fake, workspace_bytes=100)),
             None) == -3
    need = _hip.bwd_workspace_bytes(_args())
    assert f(ctypes.byref(_bwd(_args(**ins), **grads, workspace=fake + 8,
                               workspace_bytes=need)), None) == -3

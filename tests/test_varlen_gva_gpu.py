"""Grouped value heads, per-token log decay, varlen (cu_seqlens), the FLA
adapters and the dispatch on the GPU.

Bars:
* against the CPU oracle: FLA-style relative RMS <= 0.006 and max-abs
  <= 1e-2, as for the fixed-length path, and o/ht vs the fp32 gold within
  1.5x the oracle's own error plus 1e-5;
* bit for bit where the definition fixes the result exactly: a varlen call
  equals one call per sequence, a grouped-value-head call equals the
  multi-head call with q/k repeated per group, an adapter equals the entry
  point it wraps.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from kda_bt16 import (_hip, chunk_kda, dispatch, forward_choice, fused_recurrent_kda, kda_bt16_fwd,
                      kda_recurrent_fwd)
from kda_oracle import RCP_LN2, chunked_reference, per_sequence, recurrent_gold
from kda_testlib import assert_close_rel, maxdiff

pytestmark = pytest.mark.gpu

LB = -5.0


def _inputs(T, H, HV, seed, *, B=1, S=None, h0_std=0.05, log_decay=False):
    """q/k [B,T,H], the rest [B,T,HV]; states for S sequences (default B)."""
    gen = torch.Generator().manual_seed(seed)
    S = B if S is None else S
    c = dict(
        q=torch.randn(B, T, H, 128, generator=gen).bfloat16(),
        k=torch.randn(B, T, H, 128, generator=gen).bfloat16(),
        v=torch.randn(B, T, HV, 128, generator=gen).bfloat16(),
        g=torch.randn(B, T, HV, 128, generator=gen),
        beta=torch.randn(B, T, HV, generator=gen),
        A_log=torch.log(torch.rand(HV, generator=gen) * 15 + 1),
        dt_bias=torch.randn(HV * 128, generator=gen) * 0.1,
        h0=torch.randn(S, HV, 128, 128, generator=gen) * h0_std if h0_std else None,
    )
    if log_decay:  # FLA's benchmark gate: logsigmoid, clamped at the bound
        c["g"] = F.logsigmoid(c["g"]).clamp_min(LB)
        c["beta"] = c["beta"].sigmoid()
    return c


def _dev(c, dev):
    return {n: (t.to(dev) if isinstance(t, torch.Tensor) else t) for n, t in c.items()}


def _gated_kw(c, dev=None):
    mv = (lambda t: t.to(dev)) if dev else (lambda t: t)
    return dict(use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                use_beta_sigmoid_in_kernel=True, lower_bound=LB,
                A_log=mv(c["A_log"]), dt_bias=mv(c["dt_bias"]))


def _check(label, o, ht, o_ref, ht_ref, o_g, ht_g):
    o, ht = o.float().cpu(), ht.cpu()
    assert torch.isfinite(o).all() and torch.isfinite(ht).all(), label
    assert_close_rel(f"{label} o vs oracle", o_ref.float(), o, 0.006)
    assert_close_rel(f"{label} ht vs oracle", ht_ref.float(), ht, 0.006)
    assert maxdiff(o, o_ref.float()) < 1e-2 and maxdiff(ht, ht_ref) < 1e-2, label
    bar_o = 1.5 * maxdiff(o_ref.float(), o_g) + 1e-5
    bar_h = 1.5 * maxdiff(ht_ref, ht_g) + 1e-5
    do, dh = maxdiff(o, o_g), maxdiff(ht, ht_g)
    print(f"{label}: o {do:.3e} (bar {bar_o:.3e})  ht {dh:.3e} (bar {bar_h:.3e})", flush=True)
    assert do <= bar_o and dh <= bar_h, label


# ---- grouped value heads ---------------------------------------------------

@pytest.mark.parametrize("vfirst", [True, False])
def test_chunked_gva_vs_oracle_and_gold(vfirst, gpu_device):
    c = _inputs(53, 2, 4, seed=31, B=2)
    h0 = c["h0"] if vfirst else c["h0"].transpose(-1, -2).contiguous()
    d = _dev(c, gpu_device)
    o, ht = kda_bt16_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], scale=0.1,
                         initial_state=h0.to(gpu_device), output_final_state=True,
                         state_v_first=vfirst, **_gated_kw(c, gpu_device))
    kw = dict(A_log=c["A_log"], dt_bias=c["dt_bias"], lower_bound=LB, initial_state=h0,
              state_v_first=vfirst)
    o_ref, ht_ref, _ = chunked_reference(c["q"], c["k"], c["v"], c["g"], c["beta"], 0.1, **kw)
    o_g, ht_g = recurrent_gold(c["q"], c["k"], c["v"], c["g"], c["beta"], 0.1, **kw)
    _check(f"gva vfirst={vfirst}", o, ht, o_ref, ht_ref, o_g, ht_g)


def test_chunked_gva_equals_repeated_heads(gpu_device):
    """HV = 4 over H = 2 equals HV = H = 4 with q/k repeated per group."""
    c = _dev(_inputs(70, 2, 4, seed=37, B=2), gpu_device)
    kw = dict(scale=0.1, initial_state=c["h0"], output_final_state=True, **_gated_kw(c))
    o, ht = kda_bt16_fwd(c["q"], c["k"], c["v"], c["g"], c["beta"], **kw)
    qr = c["q"].repeat_interleave(2, dim=2).contiguous()
    kr = c["k"].repeat_interleave(2, dim=2).contiguous()
    o2, ht2 = kda_bt16_fwd(qr, kr, c["v"], c["g"], c["beta"], **kw)
    assert torch.equal(o, o2) and torch.equal(ht, ht2)


# ---- per-token log decay (FLA convention) ----------------------------------

@pytest.mark.parametrize("T", [16, 45])
def test_chunk_kda_log_decay_vs_oracle_and_gold(T, gpu_device):
    """chunk_kda without the in-kernel gate: g is logsigmoid(.) >= -5 per
    token and beta is already a probability (FLA's benchmark inputs,
    bench_fla_compare.py:77-79); K-first state by default."""
    c = _inputs(T, 2, 2, seed=41, B=2, log_decay=True)
    h0 = c["h0"].transpose(-1, -2).contiguous()  # K-first
    d = _dev(c, gpu_device)
    o, ht = chunk_kda(d["q"], d["k"], d["v"], d["g"], d["beta"], scale=0.1,
                      initial_state=h0.to(gpu_device), output_final_state=True,
                      use_qk_l2norm_in_kernel=True, safe_gate=True, lower_bound=LB)
    kw = dict(use_gate=False, use_beta_sigmoid=False, initial_state=h0, state_v_first=False)
    o_ref, ht_ref, _ = chunked_reference(c["q"], c["k"], c["v"], c["g"], c["beta"], 0.1,
                                         gate_log=True, **kw)
    o_g, ht_g = recurrent_gold(c["q"], c["k"], c["v"], c["g"], c["beta"], 0.1, gate_log=True, **kw)
    _check(f"log decay T{T}", o, ht, o_ref, ht_ref, o_g, ht_g)


def test_log_decay_equals_precomputed_cumsum(gpu_device):
    """Stage 1 forming the cumsum equals the caller passing it: the same
    cumsum-then-scale in fp32 is done on the host here (16-token chunks)."""
    c = _inputs(50, 2, 2, seed=43, B=1, log_decay=True)
    G = torch.zeros_like(c["g"])
    for c0 in range(0, 50, 16):
        G[:, c0:c0 + 16] = torch.cumsum(c["g"][:, c0:c0 + 16], dim=1) * RCP_LN2
    d = _dev(c, gpu_device)
    common = dict(scale=0.1, initial_state=d["h0"], output_final_state=True,
                  use_qk_l2norm_in_kernel=True, state_v_first=True)
    o1, ht1 = chunk_kda(d["q"], d["k"], d["v"], d["g"], d["beta"], safe_gate=True,
                        lower_bound=LB, **common)
    o2, ht2 = kda_bt16_fwd(d["q"], d["k"], d["v"], G.to(gpu_device), d["beta"], **common)
    # the device scan and torch's cumsum may sum in a different order: a few ulps of G
    assert maxdiff(o1.float(), o2.float()) < 2e-2 and maxdiff(ht1, ht2) < 1e-3
    assert_close_rel("log decay vs precomputed o", o2.float(), o1.float(), 2e-3)


# ---- varlen ----------------------------------------------------------------

CU = [0, 5, 5, 37, 100, 117, 160]  # an empty sequence, short ones, partial chunks


@pytest.mark.parametrize("cu_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("vfirst", [True, False])
def test_chunked_varlen_equals_per_sequence_calls(cu_dtype, vfirst, gpu_device):
    N, T = len(CU) - 1, CU[-1]
    c = _inputs(T, 2, 4, seed=47, S=N)
    h0 = c["h0"] if vfirst else c["h0"].transpose(-1, -2).contiguous()
    d = _dev(c, gpu_device)
    h0d = h0.to(gpu_device)
    cu = torch.tensor(CU, dtype=cu_dtype, device=gpu_device)
    kw = dict(scale=0.1, output_final_state=True, state_v_first=vfirst, **_gated_kw(c, gpu_device))
    o, ht = kda_bt16_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=h0d,
                         cu_seqlens=cu, **kw)
    assert o.shape == (1, T, 4, 128) and ht.shape == (N, 4, 128, 128)
    for n in range(N):
        a, b = CU[n], CU[n + 1]
        if a == b:
            assert torch.equal(ht[n], h0d[n]), "empty sequence must pass its state through"
            continue
        on, htn = kda_bt16_fwd(*(d[x][:, a:b].contiguous() for x in ("q", "k", "v", "g", "beta")),
                               initial_state=h0d[n:n + 1].contiguous(), **kw)
        assert torch.equal(o[:, a:b], on), f"sequence {n}: o differs"
        assert torch.equal(ht[n:n + 1], htn), f"sequence {n}: ht differs"


def test_chunked_varlen_vs_oracle_and_gold(gpu_device):
    N, T = len(CU) - 1, CU[-1]
    c = _inputs(T, 2, 2, seed=53, S=N)
    d = _dev(c, gpu_device)
    cu = torch.tensor(CU, dtype=torch.int64, device=gpu_device)
    o, ht = kda_bt16_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], scale=0.1,
                         initial_state=d["h0"], output_final_state=True, cu_seqlens=cu,
                         **_gated_kw(c, gpu_device))
    kw = dict(A_log=c["A_log"], dt_bias=c["dt_bias"], lower_bound=LB, initial_state=c["h0"])
    args = (c["q"], c["k"], c["v"], c["g"], c["beta"], CU, 0.1)
    o_ref, ht_ref = per_sequence(chunked_reference, *args, **kw)
    o_g, ht_g = per_sequence(recurrent_gold, *args, **kw)
    _check("varlen", o, ht, o_ref, ht_ref, o_g, ht_g)


def test_chunked_varlen_many_sequences(gpu_device):
    """150 sequences (0-40 tokens): stage 1's sequence search takes two
    rounds of its 64-way ballot; every sequence equals its own call."""
    gen = torch.Generator().manual_seed(59)
    lens = torch.randint(0, 41, (150,), generator=gen)
    cu_list = [0] + torch.cumsum(lens, 0).tolist()
    N, T = 150, cu_list[-1]
    c = _inputs(T, 1, 1, seed=61, S=N)
    d = _dev(c, gpu_device)
    cu = torch.tensor(cu_list, dtype=torch.int32, device=gpu_device)
    kw = dict(scale=0.1, output_final_state=True, **_gated_kw(c, gpu_device))
    o, ht = kda_bt16_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["h0"],
                         cu_seqlens=cu, **kw)
    for n in range(N):
        a, b = cu_list[n], cu_list[n + 1]
        if a == b:
            assert torch.equal(ht[n], d["h0"][n])
            continue
        on, htn = kda_bt16_fwd(*(d[x][:, a:b].contiguous() for x in ("q", "k", "v", "g", "beta")),
                               initial_state=d["h0"][n:n + 1].contiguous(), **kw)
        assert torch.equal(o[:, a:b], on) and torch.equal(ht[n:n + 1], htn), n


# More (sequence, value head, value tile) triples than the GPU has CUs:
# stage 2 then runs several sequences per work-group, in groups, through one
# record ring (k2_kernel's multi-sequence mode).  Its results must equal one
# call per sequence bit for bit, with empty sequences first, inside and last
# in a group, and with or without initial and final states.
MS_LENS = [0, 33, 16, 0, 0, 129, 1, 47, 0, 200, 15, 17, 0, 64, 3, 90, 31, 0, 48, 2,
           77, 0, 16, 5, 250, 0, 12, 33, 8, 0, 0, 61, 19, 140, 4, 0, 28, 56, 9, 0]


@pytest.mark.parametrize("with_h0,with_ht,vfirst",
                         [(True, True, True), (False, True, True), (True, False, True),
                          (True, True, False)])
@pytest.mark.parametrize("k2_tiles", ["1", None], ids=["one_tile_ms", "default"])
def test_varlen_multi_sequence_work_groups(with_h0, with_ht, vfirst, k2_tiles, gpu_device):
    """Several sequences per stage-2 work-group (k2_tiles=1 forces the
    one-tile kernel, which then groups sequences) and the default, which
    takes several value tiles per work-group here; each sequence equals its
    own call.  fused=False keeps the two stages: with 320 (sequence, head)
    pairs the forward would otherwise run the fused kernel."""
    with forward_choice(fused=False, k2_tiles=int(k2_tiles or 0)):
        _multi_sequence_case(with_h0, with_ht, vfirst, gpu_device)


def _multi_sequence_case(with_h0, with_ht, vfirst, gpu_device):
    cu_list = [0]
    for n in MS_LENS:
        cu_list.append(cu_list[-1] + n)
    N, T, HV = len(MS_LENS), cu_list[-1], 8
    props = torch.cuda.get_device_properties(gpu_device)
    assert N * HV * 8 > props.multi_processor_count, "the case must exceed one work-group per CU"
    print(f"[ms] N={N} T={T} HV={HV} h0={with_h0} ht={with_ht} vfirst={vfirst}", flush=True)
    c = _inputs(T, 4, HV, seed=71, S=N)
    d = _dev(c, gpu_device)
    h0 = None
    if with_h0:
        h0 = d["h0"] if vfirst else d["h0"].transpose(-1, -2).contiguous()
    cu = torch.tensor(cu_list, dtype=torch.int64, device=gpu_device)
    kw = dict(scale=0.1, output_final_state=with_ht, state_v_first=vfirst,
              **_gated_kw(c, gpu_device))
    o, ht = kda_bt16_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=h0,
                         cu_seqlens=cu, **kw)
    assert (ht is None) == (not with_ht)
    for n in range(N):
        a, b = cu_list[n], cu_list[n + 1]
        if a == b:
            if with_ht:
                want = h0[n] if with_h0 else torch.zeros_like(ht[n])
                assert torch.equal(ht[n], want), f"empty sequence {n}"
            continue
        on, htn = kda_bt16_fwd(*(d[x][:, a:b].contiguous() for x in ("q", "k", "v", "g", "beta")),
                               initial_state=None if h0 is None else h0[n:n + 1].contiguous(), **kw)
        assert torch.equal(o[:, a:b], on), f"sequence {n}: o differs"
        if with_ht:
            assert torch.equal(ht[n:n + 1], htn), f"sequence {n}: ht differs"


@pytest.mark.parametrize("k2_tiles", ["1", None], ids=["one_tile_ms", "default"])
def test_fixed_length_batch_multi_sequence_work_groups(k2_tiles, gpu_device):
    """B = 8 rows of 300 tokens, HV = 8: 512 triples, so stage 2 takes two
    or more rows per work-group (k2_tiles=1), or several value tiles per
    work-group (the default); each row equals its own call."""
    with forward_choice(k2_tiles=int(k2_tiles or 0)):
        _fixed_length_rows_case(gpu_device)


def _fixed_length_rows_case(gpu_device):
    B, T, HV = 8, 300, 8
    c = _inputs(T, 2, HV, seed=73, B=B)
    d = _dev(c, gpu_device)
    kw = dict(scale=0.1, output_final_state=True, **_gated_kw(c, gpu_device))
    o, ht = kda_bt16_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["h0"], **kw)
    for b in range(B):
        ob, htb = kda_bt16_fwd(*(d[x][b:b + 1] for x in ("q", "k", "v", "g", "beta")),
                               initial_state=d["h0"][b:b + 1], **kw)
        assert torch.equal(o[b:b + 1], ob), f"row {b}: o differs"
        assert torch.equal(ht[b:b + 1], htb), f"row {b}: ht differs"


@pytest.mark.parametrize("T", [300, 64])
def test_varlen_single_sequence_equals_fixed_length(T, gpu_device):
    """T = 64: the fixed-length call runs stage 1's full-chunk variant and
    the varlen call its general one; they must agree bit for bit."""
    c = _dev(_inputs(T, 2, 2, seed=67), gpu_device)
    kw = dict(scale=0.1, initial_state=c["h0"], output_final_state=True, **_gated_kw(c))
    o, ht = kda_bt16_fwd(c["q"], c["k"], c["v"], c["g"], c["beta"], **kw)
    cu = torch.tensor([0, T], dtype=torch.int64, device=gpu_device)
    o2, ht2 = kda_bt16_fwd(c["q"], c["k"], c["v"], c["g"], c["beta"], cu_seqlens=cu, **kw)
    assert torch.equal(o, o2) and torch.equal(ht, ht2)


@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_recurrent_varlen_equals_per_sequence_and_gold(out, gpu_device):
    N, T = len(CU) - 1, CU[-1]
    c = _inputs(T, 2, 4, seed=71, S=N)
    d = _dev(c, gpu_device)
    cu = torch.tensor(CU, dtype=torch.int64, device=gpu_device)
    kw = dict(scale=0.1, output_final_state=True, output_dtype=out, **_gated_kw(c, gpu_device))
    o, ht = kda_recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["h0"],
                              cu_seqlens=cu, **kw)
    for n in range(N):
        a, b = CU[n], CU[n + 1]
        if a == b:
            assert torch.equal(ht[n], d["h0"][n])
            continue
        on, htn = kda_recurrent_fwd(*(d[x][:, a:b].contiguous() for x in ("q", "k", "v", "g", "beta")),
                                    initial_state=d["h0"][n:n + 1].contiguous(), **kw)
        assert torch.equal(o[:, a:b], on) and torch.equal(ht[n:n + 1], htn), n
    if out == torch.float32:
        o_g, ht_g = per_sequence(recurrent_gold, c["q"], c["k"], c["v"], c["g"], c["beta"], CU,
                                 0.1, A_log=c["A_log"], dt_bias=c["dt_bias"], lower_bound=LB,
                                 initial_state=c["h0"])
        assert_close_rel("recurrent varlen o", o_g, o.cpu(), 1e-5)
        assert_close_rel("recurrent varlen ht", ht_g, ht.cpu(), 1e-5)


def test_recurrent_chunk_cumsum_form_through_c_abi(gpu_device):
    """The recurrence with neither USE_GATE nor G_LOG_DECAY takes the
    chunk-local log2 cumsum, as the chunked entries do."""
    c = _inputs(37, 2, 2, seed=73, log_decay=True)
    G = torch.zeros_like(c["g"])
    for c0 in range(0, 37, 16):
        G[:, c0:c0 + 16] = torch.cumsum(c["g"][:, c0:c0 + 16], dim=1) * RCP_LN2
    d = _dev(c, gpu_device)
    Gd = G.to(gpu_device)
    o = torch.empty(1, 37, 2, 128, dtype=torch.float32, device=gpu_device)
    ht = torch.empty(1, 2, 128, 128, dtype=torch.float32, device=gpu_device)
    a = _hip.KdaBt16Args()
    a.abi_version = _hip.ABI_VERSION
    a.B, a.T, a.H, a.HV, a.K, a.V = 1, 37, 2, 2, 128, 128
    a.flags = _hip.STATE_V_FIRST | _hip.O_FP32
    a.scale, a.lower_bound = 0.1, 0.0
    a.g_dtype, a.beta_dtype = _hip.DTYPE_F32, _hip.DTYPE_F32
    a.q, a.k, a.v, a.g, a.beta = (t.data_ptr() for t in (d["q"], d["k"], d["v"], Gd, d["beta"]))
    a.h0, a.o, a.ht = d["h0"].data_ptr(), o.data_ptr(), ht.data_ptr()
    _hip.call("kda_recurrent_fwd_hip", a, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    kw = dict(use_gate=False, use_l2norm=False, use_beta_sigmoid=False, initial_state=c["h0"])
    o_g, ht_g = recurrent_gold(c["q"], c["k"], c["v"], G, c["beta"], 0.1, **kw)
    assert_close_rel("cumsum-form o", o_g, o.cpu(), 1e-5)
    assert_close_rel("cumsum-form ht", ht_g, ht.cpu(), 1e-5)


# ---- adapters and dispatch -------------------------------------------------

def test_chunk_kda_adapter_equals_kda_bt16_fwd(gpu_device):
    """The reference test's chunk_kda call (tests/test_kda_bt16.py:84-99) on
    this backend equals kda_bt16_fwd with the same arguments."""
    c = _dev(_inputs(130, 2, 2, seed=79, B=2), gpu_device)
    kw = dict(scale=0.1, initial_state=c["h0"], output_final_state=True, state_v_first=True,
              **_gated_kw(c))
    o1, ht1 = chunk_kda(c["q"], c["k"], c["v"], c["g"], c["beta"], safe_gate=True,
                        chunk_size=64, **kw)
    o2, ht2 = kda_bt16_fwd(c["q"], c["k"], c["v"], c["g"], c["beta"], **kw)
    assert torch.equal(o1, o2) and torch.equal(ht1, ht2)


def test_fused_recurrent_kda_adapter(gpu_device):
    c = _dev(_inputs(20, 2, 4, seed=83, log_decay=True), gpu_device)
    h0 = c["h0"].transpose(-1, -2).contiguous()  # FLA's K-first default
    o1, ht1 = fused_recurrent_kda(c["q"], c["k"], c["v"], c["g"], c["beta"], scale=0.1,
                                  initial_state=h0, output_final_state=True)
    o2, ht2 = kda_recurrent_fwd(c["q"], c["k"], c["v"], c["g"], c["beta"], scale=0.1,
                                initial_state=h0, output_final_state=True, state_v_first=False)
    assert o1.dtype == torch.bfloat16
    assert torch.equal(o1, o2) and torch.equal(ht1, ht2)


def test_dispatch_routes_bucket_calls_to_this_backend(gpu_device):
    """A stand-in FLA module wrapped by install_into_fla: calls in the
    bucket run here (same bits as chunk_kda), others fall back."""
    import types

    fallback_calls = []

    def chunk_kda_fla(q, k, v, g, beta, scale=None, initial_state=None,
                      output_final_state=False, **kw):
        fallback_calls.append(kw)
        return "fallback", None

    mod = types.SimpleNamespace(chunk_kda=chunk_kda_fla)
    dispatch.install_into_fla(mod)
    assert dispatch.MI355X_BACKEND.is_available()
    c = _dev(_inputs(64, 2, 2, seed=89), gpu_device)
    kw = dict(scale=0.1, initial_state=None, output_final_state=True, state_v_first=True,
              safe_gate=True, **_gated_kw(c))
    o1, ht1 = mod.chunk_kda(c["q"], c["k"], c["v"], c["g"], c["beta"], **kw)
    o2, ht2 = chunk_kda(c["q"], c["k"], c["v"], c["g"], c["beta"], **kw)
    assert torch.equal(o1, o2) and torch.equal(ht1, ht2) and not fallback_calls
    # the softplus gate (no lower_bound) is declined and goes to FLA's own function
    kw2 = dict(kw, lower_bound=None)
    assert mod.chunk_kda(c["q"], c["k"], c["v"], c["g"], c["beta"], **kw2)[0] == "fallback"
    assert len(fallback_calls) == 1

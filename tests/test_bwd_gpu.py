"""GPU parity of the HIP backward (csrc/kda_bwd.hip through kda_bt16_bwd_hip)
against the CPU oracle (oracle/kda_oracle_bwd.py).

The reference is forward-only (/root/reference/README.md:420), so the gold is
the exact gradient of the op: fp64 autograd through the token recurrence
(pinned against finite differences in tests/test_oracle_bwd.py), or at full
length the fp64 chunked restatement pinned against it.  The bar for each
gradient: relative RMS error against the gold at most 1.5x that of the CPU
restatement with the HIP path's bf16 rounding points (``mode="kernel"``) plus
1e-3, the backward counterpart of the forward's north-star bar (1.5x the
reference chunk path's error against the fp32 gold).
"""

from __future__ import annotations

import pytest
import torch

from kda_oracle import k1_reference, make_inputs
from kda_oracle_bwd import autograd_grads, chunked_backward

pytestmark = pytest.mark.gpu

GRADS = ("dq", "dk", "dv", "dg", "dbeta", "dA_log", "ddt_bias", "dh0")


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).pow(2).mean().sqrt() / b.pow(2).mean().sqrt().clamp_min(1e-300)).item()


def _inputs(B, T, H, HV, *, seed=3, gate=True, glog=False, svf=True, h0=True, dht=True,
            gate_dtype=torch.bfloat16):
    c = make_inputs(B, T, HV, seed=seed, h0_std=0.05, gate_dtype=gate_dtype)
    q = c["q"][:, :, :H].contiguous()
    k = c["k"][:, :, :H].contiguous()
    g = c["g"]
    if glog:
        gen = torch.Generator().manual_seed(seed + 100)
        g = (-torch.rand(B, T, HV, 128, generator=gen) * 0.7).to(gate_dtype)
    elif not gate:
        st = k1_reference(q, k, c["v"], c["g"].float(), c["beta"].float(), 0.1,
                          A_log=c["A_log"], dt_bias=c["dt_bias"], mode="exact")
        NT = -(-T // 16)
        g = st["G"].reshape(B, HV, NT * 16, 128)[:, :, :T].movedim(1, 2).contiguous().float()
    gen = torch.Generator().manual_seed(seed + 7)
    do = torch.randn(B, T, HV, 128, generator=gen).to(torch.bfloat16)
    h0t = c["h0"] if h0 else None
    if h0t is not None and not svf:
        h0t = h0t.transpose(-1, -2).contiguous()
    dhtt = torch.randn(B, HV, 128, 128, generator=gen) * 0.1 if dht else None
    return dict(q=q, k=k, v=c["v"], g=g, beta=c["beta"], do=do, h0=h0t, dht=dhtt,
                A_log=c["A_log"], dt_bias=c["dt_bias"])


def _hip_bwd(x, dev, *, gate=True, glog=False, svf=True, l2=True, bsig=True, cu=None, scale=0.1):
    from kda_bt16 import kda_bt16_bwd

    D = (lambda t: None if t is None else t.to(dev))
    out = kda_bt16_bwd(D(x["do"]), D(x["q"]), D(x["k"]), D(x["v"]), D(x["g"]), D(x["beta"]), scale,
                       initial_state=D(x["h0"]), dht=D(x["dht"]), use_qk_l2norm_in_kernel=l2,
                       use_gate_in_kernel=gate, use_beta_sigmoid_in_kernel=bsig, lower_bound=-5.0,
                       A_log=D(x["A_log"]), dt_bias=D(x["dt_bias"]), state_v_first=svf,
                       cu_seqlens=D(cu), g_log=glog)
    torch.cuda.synchronize()
    return out


def _oracle_kw(x, *, gate=True, glog=False, svf=True, l2=True, bsig=True):
    return dict(A_log=x["A_log"], dt_bias=x["dt_bias"], initial_state=x["h0"], dht=x["dht"],
                state_v_first=svf, use_gate=gate, use_l2norm=l2, use_beta_sigmoid=bsig,
                gate_log=glog)


CASES = [
    # name, (B, T, H, HV), flags
    ("gate_h0_dht_partial", (1, 40, 2, 2), {}),
    ("gva", (1, 50, 2, 4), {}),
    ("fla_log_decay", (2, 33, 2, 2), {"gate": False, "glog": True}),
    ("precomputed_cumsum", (1, 40, 2, 2), {"gate": False}),
    ("k_first_state", (1, 37, 2, 2), {"svf": False}),
    ("no_l2norm_no_sigmoid", (1, 32, 1, 1), {"l2": False, "bsig": False}),
    ("fp32_gates", (1, 64, 2, 2), {"gate_dtype": torch.float32}),
    ("one_token", (1, 1, 1, 1), {}),
    ("zero_state_no_dht", (2, 100, 2, 2), {"h0": False, "dht": False}),
    ("multi_chunk", (2, 512, 4, 4), {}),
]


@pytest.mark.parametrize("name,shape,flags", CASES, ids=[c[0] for c in CASES])
def test_bwd_against_gold(gpu_device, name, shape, flags):
    gate = flags.get("gate", True)
    glog = flags.get("glog", False)
    svf = flags.get("svf", True)
    l2 = flags.get("l2", True)
    bsig = flags.get("bsig", True)
    x = _inputs(*shape, gate=gate, glog=glog, svf=svf, h0=flags.get("h0", True),
                dht=flags.get("dht", True), gate_dtype=flags.get("gate_dtype", torch.bfloat16))
    print(f"[bwd] {name} B,T,H,HV={shape}", flush=True)
    out = _hip_bwd(x, gpu_device, gate=gate, glog=glog, svf=svf, l2=l2, bsig=bsig)
    okw = _oracle_kw(x, gate=gate, glog=glog, svf=svf, l2=l2, bsig=bsig)
    args = (x["q"], x["k"], x["v"], x["g"].float(), x["beta"].float(), x["do"].float(), 0.1)
    gold = autograd_grads(*args, **okw)
    ker = chunked_backward(*args, mode="kernel", **okw)
    checked = 0
    for n in GRADS:
        if n not in gold:
            assert out[n] is None or n == "dh0", n
            continue
        got = out[n]
        assert got is not None, n
        assert got.shape == gold[n].shape, n
        assert torch.isfinite(got).all(), n
        err, bar = _rel(got, gold[n]), 1.5 * _rel(ker[n], gold[n]) + 1e-3
        assert err <= bar, f"{n}: {err:.3e} > {bar:.3e}"
        checked += 1
    assert checked >= 6


def test_bwd_dtypes_follow_inputs(gpu_device):
    x = _inputs(1, 20, 1, 1, gate_dtype=torch.float32)
    out = _hip_bwd(x, gpu_device)
    assert out["dq"].dtype == out["dk"].dtype == out["dv"].dtype == torch.bfloat16
    assert out["dg"].dtype == out["dbeta"].dtype == torch.float32
    assert out["dA_log"].dtype == out["ddt_bias"].dtype == out["dh0"].dtype == torch.float32
    x = _inputs(1, 20, 1, 1, gate_dtype=torch.bfloat16)
    out = _hip_bwd(x, gpu_device)
    assert out["dg"].dtype == out["dbeta"].dtype == torch.bfloat16


def test_bwd_is_deterministic(gpu_device):
    x = _inputs(1, 300, 2, 4, seed=12)
    a = _hip_bwd(x, gpu_device)
    b = _hip_bwd(x, gpu_device)
    for n in GRADS:
        assert torch.equal(a[n], b[n]), n


@pytest.mark.parametrize("cu_dtype", [torch.int32, torch.int64])
def test_bwd_varlen_equals_per_sequence(gpu_device, cu_dtype):
    """Packed sequences (an empty one included) against one call per
    sequence: bit-identical per-token gradients and dh0; the gate-parameter
    sums (added in another order) to fp32 rounding; and the fp64 gold."""
    from kda_bt16 import kda_bt16_bwd

    cu = [0, 17, 17, 60, 93]
    N, T, H, HV = len(cu) - 1, cu[-1], 2, 4
    c = make_inputs(1, T, HV, seed=31, h0_std=0.05)
    q, k = c["q"][:, :, :H].contiguous(), c["k"][:, :, :H].contiguous()
    gen = torch.Generator().manual_seed(5)
    do = torch.randn(1, T, HV, 128, generator=gen).to(torch.bfloat16)
    h0 = torch.randn(N, HV, 128, 128, generator=gen) * 0.05
    dht = torch.randn(N, HV, 128, 128, generator=gen) * 0.1
    dev = gpu_device
    kw = dict(use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              use_beta_sigmoid_in_kernel=True, A_log=c["A_log"].to(dev),
              dt_bias=c["dt_bias"].to(dev))
    packed = kda_bt16_bwd(do.to(dev), q.to(dev), k.to(dev), c["v"].to(dev), c["g"].to(dev),
                          c["beta"].to(dev), 0.1, initial_state=h0.to(dev), dht=dht.to(dev),
                          cu_seqlens=torch.tensor(cu, dtype=cu_dtype, device=dev), **kw)
    torch.cuda.synchronize()
    dA, ddt = torch.zeros(HV, dtype=torch.float64), torch.zeros(HV * 128, dtype=torch.float64)
    for n in range(N):
        a, b = cu[n], cu[n + 1]
        if a == b:
            assert torch.equal(packed["dh0"][n].cpu(), dht[n]), "an empty sequence passes dht"
            continue
        sl = lambda t: t[:, a:b].contiguous().to(dev)
        one = kda_bt16_bwd(sl(do), sl(q), sl(k), sl(c["v"]), sl(c["g"]), sl(c["beta"]), 0.1,
                           initial_state=h0[n:n + 1].to(dev), dht=dht[n:n + 1].to(dev), **kw)
        torch.cuda.synchronize()
        for name in ("dq", "dk", "dv", "dg", "dbeta"):
            assert torch.equal(packed[name][:, a:b], one[name]), (n, name)
        assert torch.equal(packed["dh0"][n:n + 1], one["dh0"]), n
        dA += one["dA_log"].double().cpu()
        ddt += one["ddt_bias"].double().cpu()
        gold = autograd_grads(q[:, a:b], k[:, a:b], c["v"][:, a:b], c["g"][:, a:b].float(),
                              c["beta"][:, a:b].float(), do[:, a:b].float(), 0.1,
                              A_log=c["A_log"], dt_bias=c["dt_bias"], initial_state=h0[n:n + 1],
                              dht=dht[n:n + 1])
        for name in ("dq", "dk", "dv", "dg", "dbeta", "dh0"):
            assert _rel(one[name], gold[name]) < 1e-2, (n, name)
    assert _rel(packed["dA_log"], dA) < 1e-5
    assert _rel(packed["ddt_bias"], ddt) < 1e-5


@pytest.mark.parametrize("T", [16, 5])
def test_bwd_single_chunk(gpu_device, T):
    """Sequences of one chunk (a full one and a partial one), with and
    without h0 and dht, against the fp64 gold: the reverse chain then runs a
    single step, which is both its first and its last."""
    for h0, dht in ((True, True), (False, False), (True, False)):
        x = _inputs(1, T, 1, 1, seed=5, h0=h0, dht=dht)
        out = _hip_bwd(x, gpu_device)
        gold = autograd_grads(x["q"], x["k"], x["v"], x["g"].float(), x["beta"].float(),
                              x["do"].float(), 0.1, A_log=x["A_log"], dt_bias=x["dt_bias"],
                              initial_state=x["h0"], dht=x["dht"])
        for n in ("dq", "dk", "dv", "dg", "dbeta", "dh0"):
            if gold.get(n) is None or out.get(n) is None:
                continue
            assert _rel(out[n], gold[n]) < 1e-2, (T, h0, dht, n)


@pytest.mark.parametrize("fill", [0x7F, 0xFF])
def test_bwd_single_chunk_on_poisoned_workspace(gpu_device, monkeypatch, fill):
    """One-chunk sequences (a full and a partial chunk; two heads; one and
    two batch rows) on a workspace whose bytes all start as `fill` (0x7f: a
    huge finite pattern, 0xff: NaN), each run twice: the same bits, finite,
    and the fp64 gold.  The reverse chain's single step once accumulated a
    16x16x32 MFMA onto a 16x16x16 one with no wait state between and read
    two stale accumulator registers, whose values depend on what ran before
    (the shapes are now never mixed in one chain, kda_common.h)."""
    from kda_bt16 import workspace

    def poisoned(device, nbytes):
        return torch.full((max(256, (nbytes + 255) // 256 * 256),), fill, dtype=torch.uint8,
                          device=device)

    monkeypatch.setattr(workspace, "scratch", poisoned)
    for B, T in ((1, 16), (2, 5)):
        x = _inputs(B, T, 2, 2, seed=7 + T)
        a = _hip_bwd(x, gpu_device)
        b = _hip_bwd(x, gpu_device)
        gold = autograd_grads(x["q"], x["k"], x["v"], x["g"].float(), x["beta"].float(),
                              x["do"].float(), 0.1, A_log=x["A_log"], dt_bias=x["dt_bias"],
                              initial_state=x["h0"], dht=x["dht"])
        for n in GRADS:
            assert torch.equal(a[n], b[n]), (B, T, n)
            assert torch.isfinite(a[n]).all(), (B, T, n)
        for n in ("dq", "dk", "dv", "dg", "dbeta", "dh0"):
            assert _rel(a[n], gold[n]) < 1e-2, (B, T, n)


def test_autograd_matches_explicit_backward(gpu_device):
    """kda_bt16_fwd and chunk_kda record an autograd node whose backward is
    kda_bt16_bwd: the same bits."""
    from kda_bt16 import chunk_kda, kda_bt16_bwd, kda_bt16_fwd

    dev = gpu_device
    c = make_inputs(1, 48, 2, seed=1, h0_std=0.05)
    names = ("q", "k", "v", "g", "beta", "A_log", "dt_bias", "h0")
    ins = {n: c[n].to(dev).requires_grad_(True) for n in names}
    o, ht = kda_bt16_fwd(ins["q"], ins["k"], ins["v"], ins["g"], ins["beta"], 0.1,
                         initial_state=ins["h0"], output_final_state=True,
                         use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                         use_beta_sigmoid_in_kernel=True, A_log=ins["A_log"],
                         dt_bias=ins["dt_bias"])
    assert o.requires_grad and ht.requires_grad
    gen = torch.Generator().manual_seed(9)
    do = torch.randn(o.shape, generator=gen).to(torch.bfloat16).to(dev)
    dht = torch.randn(ht.shape, generator=gen).to(dev)
    ((o.float() * do.float()).sum() + (ht * dht).sum()).backward()
    ref = kda_bt16_bwd(do, *(c[n].to(dev) for n in names[:5]), 0.1, initial_state=c["h0"].to(dev),
                       dht=dht, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                       use_beta_sigmoid_in_kernel=True, A_log=c["A_log"].to(dev),
                       dt_bias=c["dt_bias"].to(dev))
    torch.cuda.synchronize()
    for n, r in zip(names, ("dq", "dk", "dv", "dg", "dbeta", "dA_log", "ddt_bias", "dh0")):
        assert torch.equal(ins[n].grad, ref[r]), n

    # FLA convention: per-token log decay, K-first state
    gl = (-torch.rand(1, 48, 2, 128, generator=gen) * 0.5).to(dev)
    q2 = c["q"].to(dev).requires_grad_(True)
    g2 = gl.clone().requires_grad_(True)
    o2, _ = chunk_kda(q2, c["k"].to(dev), c["v"].to(dev), g2, c["beta"].float().to(dev),
                      use_qk_l2norm_in_kernel=True, safe_gate=True, lower_bound=-5.0)
    (o2.float() * do.float()).sum().backward()
    ref2 = kda_bt16_bwd(do, c["q"].to(dev), c["k"].to(dev), c["v"].to(dev), gl,
                        c["beta"].float().to(dev), use_qk_l2norm_in_kernel=True,
                        state_v_first=False, g_log=True)
    torch.cuda.synchronize()
    assert torch.equal(q2.grad, ref2["dq"])
    assert torch.equal(g2.grad, ref2["dg"])


def test_bwd_headline_shape(gpu_device):
    """B=1 T=8192 H=32: every gradient finite, and two
    heads (the op is independent per head) against the fp64 chunked
    restatement of the full 8192 tokens."""
    B, T, H = 1, 8192, 32
    c = make_inputs(B, T, H, seed=42)
    gen = torch.Generator().manual_seed(3)
    do = torch.randn(B, T, H, 128, generator=gen).to(torch.bfloat16)
    x = dict(q=c["q"], k=c["k"], v=c["v"], g=c["g"], beta=c["beta"], do=do, h0=None, dht=None,
             A_log=c["A_log"], dt_bias=c["dt_bias"])
    print("[bwd] headline B=1 T=8192 H=32", flush=True)
    out = _hip_bwd(x, gpu_device, scale=None)
    for n in ("dq", "dk", "dv", "dg", "dbeta", "dA_log", "ddt_bias"):
        assert torch.isfinite(out[n]).all(), n
    hs = [0, 17]
    sl = lambda t: t[:, :, hs].contiguous()
    gold = chunked_backward(sl(c["q"]), sl(c["k"]), sl(c["v"]), sl(c["g"]).float(),
                            sl(c["beta"]).float(), sl(do).float(), None, A_log=c["A_log"][hs],
                            dt_bias=c["dt_bias"].view(H, 128)[hs].reshape(-1))
    for n in ("dq", "dk", "dv", "dg", "dbeta"):
        assert _rel(sl(out[n]), gold[n]) < 1e-2, n
    assert _rel(out["dA_log"][hs], gold["dA_log"]) < 1e-2
    assert _rel(out["ddt_bias"].view(H, 128)[hs].reshape(-1), gold["ddt_bias"]) < 1e-2


BWD_CONFIGS = {
    # BASELINE configs[1] and configs[4] (configs[2] is test_bwd_headline_shape)
    "c1_B2_T4096_H8": dict(B=2, T=4096, H=8, h0_std=0.05),
    "c4_B16_T2048_H32": dict(B=16, T=2048, H=32, h0_std=0.05, g_std=2.0),
}


@pytest.mark.parametrize("name", list(BWD_CONFIGS))
def test_bwd_baseline_configs(name, gpu_device):
    """The backward at BASELINE sizes, with an initial state and dht: every
    gradient finite, and two (batch, head) pairs (the op is independent per
    pair) against the fp64 chunked restatement, gate parameters included
    through their per-head slices.  configs[4] has strong decay (g ~N(0, 2))."""
    cfg = dict(BWD_CONFIGS[name])
    B, T, H = cfg.pop("B"), cfg.pop("T"), cfg.pop("H")
    c = make_inputs(B, T, H, seed=42, **cfg)
    gen = torch.Generator().manual_seed(17)
    do = torch.randn(B, T, H, 128, generator=gen).to(torch.bfloat16)
    dht = torch.randn(B, H, 128, 128, generator=gen) * 0.05
    x = dict(q=c["q"], k=c["k"], v=c["v"], g=c["g"], beta=c["beta"], do=do, h0=c["h0"], dht=dht,
             A_log=c["A_log"], dt_bias=c["dt_bias"])
    print(f"[bwd] {name}", flush=True)
    out = _hip_bwd(x, gpu_device, scale=None)
    for n in GRADS:
        assert torch.isfinite(out[n]).all(), n
    for b, h in ((0, 0), (B - 1, H - 1)):
        sl = lambda t: t[b:b + 1, :, h:h + 1].contiguous()
        gold = chunked_backward(
            sl(c["q"]), sl(c["k"]), sl(c["v"]), sl(c["g"]).float(), sl(c["beta"]).float(),
            sl(do).float(), None, dht=dht[b:b + 1, h:h + 1], A_log=c["A_log"][h:h + 1],
            dt_bias=c["dt_bias"][h * 128:(h + 1) * 128], initial_state=c["h0"][b:b + 1, h:h + 1])
        for n in ("dq", "dk", "dv", "dg", "dbeta"):
            assert _rel(sl(out[n]), gold[n]) < 1e-2, (b, h, n)
        assert _rel(out["dh0"][b:b + 1, h:h + 1], gold["dh0"]) < 1e-2, (b, h)

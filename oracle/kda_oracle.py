"""CPU oracle for the KDA BT=16 chunked forward.

TEST INFRASTRUCTURE ONLY.  Nothing on the product path imports this module:
it is used by ``tests/``, ``__graft_entry__.smoke()`` (as the checker) and
``bench.py``'s ``cpu_baseline`` leg (as the timed CPU restatement).

Two independent formulations:

* :func:`chunked_reference` restates the reference's two-stage chunked path
  -- ``kda_bt16_kernel_k1`` (/root/reference/src/kda_bt16/kernels.py:53-184)
  and ``kda_bt16_kernel_k2`` (kernels.py:187-302) -- vectorised over
  (batch, head, chunk) in torch on the CPU.  In ``mode="kernel"`` it keeps the
  reference's fp32 arithmetic and every bf16 rounding point; in
  ``mode="exact"`` it runs the same algebra in fp64 with no rounding.
* :func:`recurrent_gold` is the token-by-token KDA recurrence (the role FLA's
  ``fused_recurrent_kda`` plays in /root/reference/tests/test_kda_bt16.py:26-39),
  in fp32 or fp64.

How each part is pinned (tests/test_oracle.py):

* the chunked algebra (gate cumsum, mid recentring, both grams and masks,
  forward substitution, W/U, the state recurrence) -- ``mode="exact"``
  against the fp64 recurrence to ~1e-10 on shapes with partial chunks,
  non-zero states and both state layouts; two different formulations that
  agree in exact arithmetic;
* the solve -- against ``torch.linalg.inv(I + L)`` in fp64;
* l2norm and gate -- unit row norms; cumsum monotone, chunk-local and
  bounded by ``16 * lower_bound * RCP_LN2``;
* special cases with closed forms -- T=1 from a zero state gives
  ``o = scale * beta * (k^.q^) * v``; beta = 0 gives pure decay of h0;
* the bf16 rounding points -- ``mode="kernel"`` against the fp32 gold on the
  reference README's precision case (B=2 T=1024 H=4, seed 42), whose
  published errors are o 4.9e-4 and ht 1.8e-3 (/root/reference/README.md:55-57).
"""

from __future__ import annotations

import contextlib
import math

import torch
import torch.nn.functional as F

RCP_LN2 = 1.4426950216  # kernels.py:38
EPS = 1e-6  # kernels.py:39
BT = 16  # kernels.py:40


# How fp32 values are rounded to bf16: "rtne" (round to nearest, ties to
# even) is what the reference's `.to(tl.bfloat16)` does on GPUs and NPUs;
# "rtz" (truncation) is what Triton's CPU interpreter does for the same
# cast (triton/runtime/interpreter.py, _convert_float with no rounding
# mode), used only to compare with fixtures that interpreter wrote.
_BF16_ROUNDING = ["rtne"]


@contextlib.contextmanager
def bf16_rounding(mode: str):
    """Within the block, kernel mode rounds to bf16 by ``mode`` ("rtne" or
    "rtz")."""
    if mode not in ("rtne", "rtz"):
        raise ValueError(mode)
    old = _BF16_ROUNDING[0]
    _BF16_ROUNDING[0] = mode
    try:
        yield
    finally:
        _BF16_ROUNDING[0] = old


def _bf(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (nearest even, or toward zero under bf16_rounding("rtz"))
    and return fp32."""
    if _BF16_ROUNDING[0] == "rtz":
        bits = x.to(torch.float32).contiguous().view(torch.int32) & -65536
        return bits.view(torch.float32)
    return x.to(torch.bfloat16).to(torch.float32)


# The bf16 rounding points of the reference's chunked path, by name:
#   stage 1 (kernels.py:108-113, 153, 169-176): q_hat, k_hat (the l2norm
#   outputs), Aqk (stored bf16), A (bf16(A_inv), the W/U operand), kb_beta
#   (bf16(k_hat * beta)), kb (bf16(kb_beta * 2^G)), vb (bf16(v * beta)), w, u;
#   stage 2 (kernels.py:261-291): hc (bf16(S)), v_new, qg (bf16(q_hat * 2^G)),
#   o, kg (bf16(k_hat * 2^(G_last - G))).
# `planted_mistake` leaves named points unrounded: the tests use it to show
# which of them the fixtures written by the reference's own kernels pin.
ROUNDING_POINTS = ("q_hat", "k_hat", "Aqk", "A", "kb_beta", "kb", "vb", "w", "u",
                   "hc", "v_new", "qg", "o", "kg")
_UNROUNDED: set = set()


@contextlib.contextmanager
def planted_mistake(*names: str):
    """Within the block, kernel mode skips the named bf16 rounding points
    (test use only: a planted mistake for mutation tests)."""
    bad = set(names) - set(ROUNDING_POINTS)
    if bad:
        raise ValueError(f"unknown rounding points {sorted(bad)}")
    _UNROUNDED.update(names)
    try:
        yield
    finally:
        _UNROUNDED.difference_update(names)


def _rb(name: str, x: torch.Tensor) -> torch.Tensor:
    """bf16 rounding at the named point (kernel mode)."""
    return x if name in _UNROUNDED else _bf(x)


def _chunks(x: torch.Tensor, NT: int) -> torch.Tensor:
    """[B, T, H, ...] -> [B, H, NT, 16, ...], zero padded past T."""
    B, T, H = x.shape[:3]
    x = x.movedim(2, 1)  # [B, H, T, ...]
    pad = NT * BT - T
    if pad:
        shape = list(x.shape)
        shape[2] = pad
        x = torch.cat([x, x.new_zeros(shape)], dim=2)
    return x.reshape(B, H, NT, BT, *x.shape[3:])


def _unchunk(x: torch.Tensor, T: int) -> torch.Tensor:
    """[B, H, NT, 16, D] -> [B, T, H, D]."""
    B, H, NT = x.shape[:3]
    return x.reshape(B, H, NT * BT, *x.shape[4:])[:, :, :T].movedim(1, 2).contiguous()


def k1_reference(
    q, k, v, g, beta, scale, *, A_log=None, dt_bias=None, lower_bound=-5.0,
    use_gate=True, use_l2norm=True, use_beta_sigmoid=True, mode="kernel", gate_log=False,
) -> dict:
    """Stage-1 intermediates, chunked as [B, HV, NT, 16, ...].

    Follows kernels.py:97-184.  Returns q_hat, k_hat, v, beta, G (fp32 log2
    cumsum), Aqk (stored bf16 in kernel mode), A_inv (fp32 and bf16), w, u,
    nvalid (valid rows per chunk).

    Beyond the reference: grouped value heads (v, g, beta, A_log, dt_bias
    with HV heads, value head hv using q/k head hv // (HV // H), the
    indexing of kernels.py:88), and ``gate_log``: without ``use_gate``, g is
    the per-token natural-log decay and G its chunk-local cumsum times
    RCP_LN2, the cumsum-then-scale order of the in-kernel gate.
    """
    exact = mode == "exact"
    dt = torch.float64 if exact else torch.float32
    H = q.shape[2]
    HV = v.shape[2]
    q = q.repeat_interleave(HV // H, dim=2)
    k = k.repeat_interleave(HV // H, dim=2)
    B, T, H, K = q.shape  # H is now the value-head count
    NT = -(-T // BT)
    rows = torch.arange(NT * BT).reshape(NT, BT)
    valid = (rows < T)  # [NT, 16]
    nvalid = torch.clamp(T - torch.arange(NT) * BT, max=BT)  # [NT]
    vmask = valid[None, None, :, :, None]

    qc = _chunks(q.to(dt), NT)
    kc = _chunks(k.to(dt), NT)
    vc = _chunks(v.to(dt), NT)
    gc = _chunks(g.to(dt), NT)
    bc = _chunks(beta.to(dt), NT)  # [B, H, NT, 16]; padded rows 0 (kernels.py:97)
    if use_beta_sigmoid:
        bc = torch.sigmoid(bc)  # kernels.py:98-99

    if use_l2norm:  # kernels.py:108-113: x * (1 / sqrt(sum x^2 + eps)), back to bf16
        qn = qc * (1.0 / torch.sqrt((qc * qc).sum(-1, keepdim=True) + EPS))
        kn = kc * (1.0 / torch.sqrt((kc * kc).sum(-1, keepdim=True) + EPS))
        if not exact:
            qn, kn = _rb("q_hat", qn), _rb("k_hat", kn)
    else:
        qn, kn = qc, kc

    if use_gate:  # kernels.py:115-124
        s = gc
        if dt_bias is not None:
            s = s + dt_bias.to(dt).view(1, H, 1, 1, K)
        ea = torch.exp(A_log.to(dt)).view(1, H, 1, 1, 1)
        gate = lower_bound * torch.sigmoid(ea * s)
        gate = torch.where(vmask, gate, torch.zeros((), dtype=dt))
        G = torch.cumsum(gate, dim=3) * RCP_LN2
    elif gate_log:
        G = torch.cumsum(torch.where(vmask, gc, torch.zeros((), dtype=dt)), dim=3) * RCP_LN2
    else:
        G = gc

    # kernels.py:133-136: recentre on the chunk-local row min(8, nvalid - 1)
    mid = torch.clamp(nvalid - 1, max=BT // 2)
    Gmid = G[:, :, torch.arange(NT), mid][:, :, :, None, :]  # [B, H, NT, 1, K]
    gm = G - Gmid
    zero = torch.zeros((), dtype=dt)
    gq = torch.where(vmask, torch.exp2(gm), zero)
    gk = torch.where(vmask, torch.exp2(-gm), zero)

    Ks = kn * gk  # kernels.py:141-143: fp32 ieee dots
    Aqk = ((qn * gq) @ Ks.transpose(-1, -2)) * scale
    Akk = ((kn * gq) @ Ks.transpose(-1, -2)) * bc[..., :, None]
    ii = torch.arange(BT)
    Aqk = torch.where(ii[:, None] >= ii[None, :], Aqk, zero)  # kernels.py:145-148
    Akk = torch.where(ii[:, None] > ii[None, :], Akk, zero)

    # forward substitution, kernels.py:160-167: X = -Akk; X[i] = -Akk[i,:i] + sum_j (-Akk[i,j]) X[j]
    X = -Akk
    for i in range(2, BT):
        a = torch.where(ii < i, -Akk[..., i, :], zero)
        a = a + (a[..., :, None] * X).sum(-2)
        X = X.clone()
        X[..., i, :] = a
    A_inv = X + torch.eye(BT, dtype=dt)

    if exact:
        A = A_inv
        kb = kn * bc[..., None] * torch.exp2(G)
        vb = vc * bc[..., None]
        w = A @ kb
        u = A @ vb
        Aqk_st = Aqk
    else:  # kernels.py:170-176: bf16 A, bf16 operands, fp32 accumulation, bf16 stores
        A = _rb("A", A_inv)
        kb = _rb("kb", _rb("kb_beta", kn * bc[..., None]) * torch.exp2(G))
        vb = _rb("vb", vc * bc[..., None])
        w = _rb("w", A @ kb)
        u = _rb("u", A @ vb)
        Aqk_st = _rb("Aqk", Aqk)

    return {
        "q_hat": qn, "k_hat": kn, "beta": bc, "G": G, "Aqk": Aqk_st, "Akk": Akk,
        "A_inv_f32": A_inv, "A_inv": A, "w": w, "u": u, "nvalid": nvalid, "T": T,
    }


def k2_reference(st: dict, scale, *, h0=None, state_v_first=True, mode="kernel", out_dtype=None):
    """Stage-2 recurrence over stage-1 intermediates, kernels.py:225-302.

    Returns (o [B, T, H, V], ht in the layout of h0 / state_v_first).
    """
    exact = mode == "exact"
    dt = torch.float64 if exact else torch.float32
    rb = (lambda name, x: x) if exact else _rb
    qn, kn, G = st["q_hat"], st["k_hat"], st["G"]
    w, u, Aqk, nvalid, T = st["w"], st["u"], st["Aqk"], st["nvalid"], st["T"]
    B, H, NT = qn.shape[:3]
    K = qn.shape[-1]
    V = u.shape[-1]
    if h0 is None:
        S = torch.zeros(B, H, V, K, dtype=dt)
    else:
        S = h0.to(dt)
        if not state_v_first:
            S = S.transpose(-1, -2)
        S = S.clone()
    o = torch.empty(B, H, NT, BT, V, dtype=dt)
    for c in range(NT):
        hc = rb("hc", S)
        hct = hc.transpose(-1, -2)
        Gc = G[:, :, c]
        vnew = u[:, :, c] - w[:, :, c] @ hct  # kernels.py:261-266
        vb = rb("v_new", vnew)
        qg = rb("qg", qn[:, :, c] * torch.exp2(Gc))  # kernels.py:269
        oc = (qg @ hct) * scale + Aqk[:, :, c] @ vb  # kernels.py:270-276
        o[:, :, c] = rb("o", oc)
        last = int(nvalid[c]) - 1  # kernels.py:282
        Gl = Gc[:, :, last]  # [B, H, K]
        kg = rb("kg", kn[:, :, c] * torch.exp2(Gl[:, :, None, :] - Gc))  # kernels.py:285-286
        S = S * torch.exp2(Gl)[:, :, None, :] + vb.transpose(-1, -2) @ kg  # kernels.py:288-290
    o = _unchunk(o, T)
    if out_dtype is not None:
        o = o.to(out_dtype)
    ht = S if state_v_first else S.transpose(-1, -2).contiguous()
    return o, ht


def chunked_reference(
    q, k, v, g, beta, scale=None, *, A_log=None, dt_bias=None, lower_bound=-5.0,
    initial_state=None, state_v_first=True, use_gate=True, use_l2norm=True,
    use_beta_sigmoid=True, mode="kernel", gate_log=False,
):
    """The reference's chunked forward on the CPU.

    Returns ``(o, ht, intermediates)``.  In kernel mode ``o`` is bf16-valued
    (returned as bf16) and ``ht`` fp32; intermediates are reshaped to the
    reference's debug layouts ([B, T, H, 16] / [B, T, H, 128]).
    """
    K = q.shape[-1]
    if scale is None:
        scale = K ** -0.5
    st = k1_reference(
        q, k, v, g, beta, scale, A_log=A_log, dt_bias=dt_bias, lower_bound=lower_bound,
        use_gate=use_gate, use_l2norm=use_l2norm, use_beta_sigmoid=use_beta_sigmoid, mode=mode,
        gate_log=gate_log,
    )
    o, ht = k2_reference(
        st, scale, h0=initial_state, state_v_first=state_v_first, mode=mode,
        out_dtype=None if mode == "exact" else torch.bfloat16,
    )
    T = st["T"]
    inter = {
        "Aqk": _unchunk(st["Aqk"], T),
        "A_inv": _unchunk(st["A_inv"], T),
        "w": _unchunk(st["w"], T),
        "u": _unchunk(st["u"], T),
        "g": _unchunk(st["G"], T),
    }
    return o, ht, inter


def recurrent_gold(
    q, k, v, g, beta, scale=None, *, A_log=None, dt_bias=None, lower_bound=-5.0,
    initial_state=None, state_v_first=True, use_gate=True, use_l2norm=True,
    use_beta_sigmoid=True, dtype=torch.float32, gate_log=False,
):
    """Token-by-token KDA recurrence (the fp32 gold of the reference's tests).

    Per token t, with S in R^{V x K}:
      S <- S * alpha_t[None, :]            alpha_t = exp(lb*sigmoid(exp(A_log)*(g_t+dt_bias)))
      v_new = beta_t * (v_t - S k^_t)
      S <- S + v_new k^_t^T
      o_t = scale * S q^_t
    Without the in-kernel gate, ``g`` is the chunk-local log2 cumsum and
    alpha_t = 2^(g_t - g_{t-1}) (g_{-1} = 0 at every chunk start); with
    ``gate_log`` it is instead the per-token natural-log decay,
    alpha_t = exp(g_t) (FLA's fused_recurrent_kda convention).
    Grouped value heads: v, g, beta, A_log, dt_bias and the states have HV
    heads and q, k have H; value head hv reads q/k head hv // (HV // H)
    (kernels.py:88).
    """
    B, T, H, K = q.shape
    HV = v.shape[2]
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    rep = HV // H
    qf = q.to(dtype).repeat_interleave(rep, dim=2).movedim(2, 1)  # [B, HV, T, K]
    kf = k.to(dtype).repeat_interleave(rep, dim=2).movedim(2, 1)
    vf = v.to(dtype).movedim(2, 1)
    gf = g.to(dtype).movedim(2, 1)
    bf = beta.to(dtype).movedim(2, 1)  # [B, HV, T]
    if use_l2norm:
        qf = qf / torch.sqrt((qf * qf).sum(-1, keepdim=True) + EPS)
        kf = kf / torch.sqrt((kf * kf).sum(-1, keepdim=True) + EPS)
    if use_beta_sigmoid:
        bf = torch.sigmoid(bf)
    if use_gate:
        s = gf if dt_bias is None else gf + dt_bias.to(dtype).view(1, HV, 1, K)
        ea = torch.exp(A_log.to(dtype)).view(1, HV, 1, 1)
        alpha = torch.exp(lower_bound * torch.sigmoid(ea * s))
    elif gate_log:
        alpha = torch.exp(gf)
    else:
        prev = torch.zeros_like(gf)
        prev[:, :, 1:] = gf[:, :, :-1]
        prev[:, :, ::BT] = 0
        alpha = torch.exp2(gf - prev)
    if initial_state is None:
        S = torch.zeros(B, HV, V, K, dtype=dtype)
    else:
        S = initial_state.to(dtype)
        if not state_v_first:
            S = S.transpose(-1, -2)
        S = S.clone()
    o = torch.empty(B, HV, T, V, dtype=dtype)
    for t in range(T):
        S = S * alpha[:, :, t, None, :]
        kt = kf[:, :, t]
        vnew = bf[:, :, t, None] * (vf[:, :, t] - (S @ kt[..., None])[..., 0])
        S = S + vnew[..., :, None] * kt[..., None, :]
        o[:, :, t] = scale * (S @ qf[:, :, t, :, None])[..., 0]
    ht = S if state_v_first else S.transpose(-1, -2).contiguous()
    return o.movedim(1, 2).contiguous(), ht


def per_sequence(fn, q, k, v, g, beta, cu_seqlens, *args, initial_state=None,
                 state_v_first=True, **kwargs):
    """Varlen by definition: sequence n (tokens cu_seqlens[n] to
    cu_seqlens[n+1] of the single batch row) runs on its own with state
    initial_state[n], and the outputs are concatenated along T (o) and
    stacked (final states).  ``fn`` is :func:`chunked_reference` or
    :func:`recurrent_gold`; an empty sequence passes its state through.
    Returns (o, ht)."""
    cu = [int(x) for x in cu_seqlens]
    HV = v.shape[2]
    K, V = q.shape[-1], v.shape[-1]
    outs, states = [], []
    for n in range(len(cu) - 1):
        a, b = cu[n], cu[n + 1]
        h0 = None if initial_state is None else initial_state[n:n + 1]
        if b == a:
            if h0 is None:
                shape = (1, HV, V, K) if state_v_first else (1, HV, K, V)
                states.append(torch.zeros(shape))
            else:
                states.append(h0.clone())
            continue
        res = fn(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], beta[:, a:b], *args,
                 initial_state=h0, state_v_first=state_v_first, **kwargs)
        outs.append(res[0])
        states.append(res[1])
    return torch.cat(outs, dim=1), torch.cat(states, dim=0)


def make_inputs(B, T, H, *, seed=42, g_std=1.0, h0_std=0.0, K=128, storage=torch.bfloat16,
                gate_dtype=None):
    """The BASELINE.json generators, on the CPU: seed, then in order
    q, k, v, g_raw, beta_raw ~N(0,1) (g_raw std ``g_std``) stored as
    ``storage``; A_log = log U(1,16); dt_bias ~N(0, 0.1); h0 ~N(0, h0_std)
    or None.  g and beta are stored as ``gate_dtype`` (default: storage)."""
    gate_dtype = storage if gate_dtype is None else gate_dtype
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=gen).to(storage)
    k = torch.randn(B, T, H, K, generator=gen).to(storage)
    v = torch.randn(B, T, H, K, generator=gen).to(storage)
    g = (torch.randn(B, T, H, K, generator=gen) * g_std).to(gate_dtype)
    beta = torch.randn(B, T, H, generator=gen).to(gate_dtype)
    A_log = torch.log(torch.rand(H, generator=gen) * 15.0 + 1.0)
    dt_bias = torch.randn(H * K, generator=gen) * 0.1
    h0 = None
    if h0_std > 0:
        h0 = torch.randn(B, H, K, K, generator=gen) * h0_std
    return dict(q=q, k=k, v=v, g=g, beta=beta, A_log=A_log, dt_bias=dt_bias, h0=h0)


def algorithmic_units(B, T, H, *, g_bytes=2, beta_bytes=2, h0=False, ht=True, K=128, V=128):
    """Algorithmic HBM bytes and matmul FLOPs of one forward.

    bytes: q, k, v, o (2 B each per element), g (g_bytes), beta (beta_bytes),
    states (4 B), A_log + dt_bias; FLOPs: the grams and W/U of stage 1 and the
    three state products plus Aqk @ v_new of stage 2 per chunk.
    """
    nth = B * T * H
    nch = B * H * math.ceil(T / BT)
    byts = nth * (3 * K * 2 + K * g_bytes + beta_bytes + V * 2)
    byts += B * H * K * V * 4 * (int(h0) + int(ht)) + H * (4 + 4 * K)
    flops_k1 = 4 * (2 * BT * BT * K)
    flops_k2 = 3 * (2 * BT * K * V) + 2 * BT * BT * V
    return byts, nch * (flops_k1 + flops_k2)

"""CPU oracle for the backward of the KDA BT=16 chunked forward.

TEST INFRASTRUCTURE ONLY.  Nothing on the product path imports this module:
it is used by ``tests/`` as the checker of the HIP backward.

The reference is forward-only (/root/reference/README.md:420); its roadmap
names the backward (/root/reference/docs/KDA_ANALYSIS.md:134-165, FLA's
``chunk_kda_bwd`` call graph: recompute w/u/h, dAv, the dh recurrence, the
WY/gate gradients and the reverse cumsum of dg).  The gradient of the op is
fixed by its mathematics, so two formulations serve as the oracle:

* :func:`autograd_grads` -- torch autograd through :func:`recurrent_gold`
  (the token recurrence) in fp64: the exact gradient of the op's
  definition, independent of any chunked algebra.  Pinned against central
  finite differences (``torch.autograd.gradcheck``) on tiny shapes.
* :func:`chunked_backward` -- the chunked (WY) backward written out by hand,
  per 16-token chunk, in the order the HIP kernels run it: the reverse state
  chain (dh, dv_new), then the per-chunk products and the intra-chunk
  gradients (solve, grams, gates, beta, l2norm).  In ``mode="exact"`` (fp64,
  no rounding) it must equal :func:`autograd_grads` to roundoff on every
  flag set, partial chunks and grouped value heads; in ``mode="kernel"`` it
  keeps the bf16 rounding points of the HIP path (the forward's, plus bf16
  h, v_new, dh and dv_new) so that the GPU intermediates can be compared
  tightly.

Notation (per chunk, rows i < n valid): state h = S^T [K, V]; E = 2^G;
v_new = u - w h; o = scale qg h + Aqk v_new; h' = E_l h + kg^T v_new, with
qg = q^ E, kg = k^ 2^(G_l - G), w = A kb, u = A vb, kb = beta k^ E,
vb = beta v, A = (I + L)^-1, L = beta_i tril_strict(kp km^T),
Aqk = scale tril(qp km^T), kp / qp / km the recentred k^ 2^(G - G_m),
q^ 2^(G - G_m), k^ 2^(G_m - G).
"""

from __future__ import annotations

import math

import torch

from kda_oracle import BT, EPS, RCP_LN2, _bf, _chunks, _unchunk, k1_reference, recurrent_gold

LN2 = math.log(2.0)


def autograd_grads(q, k, v, g, beta, do, scale=None, *, dht=None, A_log=None, dt_bias=None,
                   lower_bound=-5.0, initial_state=None, state_v_first=True, use_gate=True,
                   use_l2norm=True, use_beta_sigmoid=True, gate_log=False,
                   dtype=torch.float64):
    """Gradients of sum(o * do) + sum(ht * dht) through the token recurrence.

    Returns a dict with dq, dk, dv, dg, dbeta (shapes of the inputs), dA_log,
    ddt_bias (when used) and dh0 (when an initial state is given), all in
    ``dtype``, plus the forward's o and ht."""
    leaves = {}

    def leaf(name, x):
        if x is None:
            return None
        t = x.detach().to(dtype).clone().requires_grad_(True)
        leaves[name] = t
        return t

    qq, kk, vv, gg, bb = (leaf(n, x) for n, x in
                          (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta)))
    al = leaf("A_log", A_log) if use_gate else None
    db = leaf("dt_bias", dt_bias) if use_gate else None
    h0 = leaf("h0", initial_state)
    o, ht = recurrent_gold(qq, kk, vv, gg, bb, scale, A_log=al, dt_bias=db,
                           lower_bound=lower_bound, initial_state=h0,
                           state_v_first=state_v_first, use_gate=use_gate,
                           use_l2norm=use_l2norm, use_beta_sigmoid=use_beta_sigmoid,
                           dtype=dtype, gate_log=gate_log)
    loss = (o * do.to(dtype)).sum()
    if dht is not None:
        loss = loss + (ht * dht.to(dtype)).sum()
    names = list(leaves)
    grads = torch.autograd.grad(loss, [leaves[n] for n in names], allow_unused=True)
    out = {"d" + n: (torch.zeros_like(leaves[n]) if gr is None else gr)
           for n, gr in zip(names, grads)}
    out["o"] = o.detach()
    out["ht"] = ht.detach()
    return out


def _revcumsum(x: torch.Tensor, dim: int) -> torch.Tensor:
    return x.flip(dim).cumsum(dim).flip(dim)


def chunked_backward(q, k, v, g, beta, do, scale=None, *, dht=None, A_log=None, dt_bias=None,
                     lower_bound=-5.0, initial_state=None, state_v_first=True, use_gate=True,
                     use_l2norm=True, use_beta_sigmoid=True, gate_log=False, mode="exact"):
    """The chunked backward, by hand.  Returns the gradients (as
    :func:`autograd_grads`) and the per-chunk intermediates the HIP kernels
    exchange: ``h`` (state at each chunk start, [B, HV, NT, K, V]),
    ``v_new`` [B, HV, NT, 16, V], ``dh`` (gradient of the state after each
    chunk, [B, HV, NT, K, V]) and ``dv_new`` [B, HV, NT, 16, V].

    ``mode="kernel"``: fp32 with the forward's bf16 rounding points
    (kernels.py:97-302) and bf16 h, v_new, dh, dv_new, scale*qg, kg, w where
    they enter matrix products, as the HIP backward rounds them."""
    exact = mode == "exact"
    dt = torch.float64 if exact else torch.float32
    rb = (lambda x: x) if exact else _bf
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[-1]
    rep = HV // H
    if scale is None:
        scale = K ** -0.5
    NT = -(-T // BT)
    st = k1_reference(q, k, v, g, beta, scale, A_log=A_log, dt_bias=dt_bias,
                      lower_bound=lower_bound, use_gate=use_gate, use_l2norm=use_l2norm,
                      use_beta_sigmoid=use_beta_sigmoid, mode=mode, gate_log=gate_log)
    qn, kn, bc, G = st["q_hat"], st["k_hat"], st["beta"], st["G"]  # [B, HV, NT, 16, K]
    nvalid = st["nvalid"]
    ii = torch.arange(BT)
    valid = (torch.arange(NT)[:, None] * BT + ii[None, :]) < T  # [NT, 16]
    vmask = valid[None, None, :, :, None]
    zero = torch.zeros((), dtype=dt)
    E = torch.where(vmask, torch.exp2(G), zero)
    last = (nvalid - 1).clamp_min(0)
    Gl = G[:, :, torch.arange(NT), last]  # [B, HV, NT, K]
    El = torch.exp2(Gl)
    mid = torch.clamp(nvalid - 1, max=BT // 2)
    Gm = G[:, :, torch.arange(NT), mid][:, :, :, None, :]
    eq = torch.where(vmask, torch.exp2(G - Gm), zero)
    ek = torch.where(vmask, torch.exp2(Gm - G), zero)
    qp, kp, km = qn * eq, kn * eq, kn * ek
    qg = qn * E
    kgl = torch.where(vmask, torch.exp2(Gl[:, :, :, None, :] - G), zero)
    kg = kn * kgl
    vc = _chunks(v.to(dt), NT)
    A = st["A_inv"]  # bf16-valued in kernel mode, the operand of w/u
    Ainv = st["A_inv_f32"].to(dt)
    w, u, Aqk = st["w"], st["u"], st["Aqk"]
    kb = kn * bc[..., None] * E
    vb = vc * bc[..., None]
    if not exact:
        kb = _bf(_bf(kn * bc[..., None]) * E)
        vb = _bf(vb)
    doc = _chunks(do.to(dt), NT)  # [B, HV, NT, 16, V]

    # ---- forward recompute of h (state at chunk start) and v_new ---------
    if initial_state is None:
        h = torch.zeros(B, HV, K, V, dtype=dt)
    else:
        h0 = initial_state.to(dt)
        h = h0.transpose(-1, -2) if state_v_first else h0
        h = h.clone()
    hs, vns = [], []
    for c in range(NT):
        hc = rb(h)
        vn = rb(u[:, :, c] - w[:, :, c] @ hc)
        hs.append(hc)
        vns.append(vn)
        h = El[:, :, c, :, None] * h + rb(kg[:, :, c]).transpose(-1, -2) @ vn
    hall = torch.stack(hs, 2)
    vnall = torch.stack(vns, 2)

    # ---- reverse state chain: dv_new and dh per chunk --------------------
    if dht is None:
        dh = torch.zeros(B, HV, K, V, dtype=dt)
    else:
        d = dht.to(dt)
        dh = (d.transpose(-1, -2) if state_v_first else d).clone()
    dhs = [None] * NT
    dvns = [None] * NT
    qgs = rb(scale * qg)
    for c in range(NT - 1, -1, -1):
        dhb = rb(dh)
        dhs[c] = dhb  # gradient of the state after chunk c
        dvn = Aqk[:, :, c].transpose(-1, -2) @ doc[:, :, c] + rb(kg[:, :, c]) @ dhb
        dvns[c] = dvn
        dh = (El[:, :, c, :, None] * dh + qgs[:, :, c].transpose(-1, -2) @ doc[:, :, c]
              - rb(w[:, :, c]).transpose(-1, -2) @ rb(dvn))
    dh0 = dh
    dhall = torch.stack(dhs, 2)
    dvnall = torch.stack(dvns, 2)

    # ---- per-chunk products over V ---------------------------------------
    hT = hall.transpose(-1, -2)  # [.., V, K]
    dqg = scale * (doc @ hT)
    dw = -(rb(dvnall) @ hT)
    dkg = vnall @ dhall.transpose(-1, -2)
    dEl = (dhall * hall).sum(-1)  # [B, HV, NT, K]
    dAqk = doc @ vnall.transpose(-1, -2)
    du = rb(dvnall)  # the HIP path hands dv_new over in bf16

    # ---- intra-chunk ------------------------------------------------------
    tril_incl = (ii[:, None] >= ii[None, :])
    tril_strict = (ii[:, None] > ii[None, :])
    dA = dw @ kb.transpose(-1, -2) + du @ vb.transpose(-1, -2)
    dkb = A.transpose(-1, -2) @ dw
    dvb = A.transpose(-1, -2) @ du
    dL = -(Ainv.transpose(-1, -2) @ dA @ Ainv.transpose(-1, -2))
    dL = torch.where(tril_strict, dL, zero)
    Lraw = kp @ km.transpose(-1, -2)
    dbeta = (dL * Lraw).sum(-1)
    dLr = bc[..., :, None] * dL
    dkp = dLr @ km
    dkm = dLr.transpose(-1, -2) @ kp
    dAqm = torch.where(tril_incl, dAqk, zero) * scale
    dqp = dAqm @ km
    dkm = dkm + dAqm.transpose(-1, -2) @ qp

    dqn = dqg * E + dqp * eq
    dkn = dkb * bc[..., None] * E + dkg * kgl + dkp * eq + dkm * ek
    dbeta = dbeta + (dkb * kn * E).sum(-1) + (dvb * vc).sum(-1)
    dv_c = dvb * bc[..., None]
    dG = LN2 * (dkb * kb + dqg * qg - dkg * kg + dqp * qp + dkp * kp - dkm * km)
    dGl = LN2 * ((dkg * kg).sum(-2) + El * dEl)  # [B, HV, NT, K]
    onehot = (ii[None, :] == last[:, None]).to(dt)  # [NT, 16]
    dG = dG + onehot[None, None, :, :, None] * dGl[:, :, :, None, :]
    dG = torch.where(vmask, dG, zero)

    # ---- gates, beta, l2norm ---------------------------------------------
    gc = _chunks(g.to(dt), NT)
    if use_gate:
        dgate = RCP_LN2 * _revcumsum(dG, 3)
        s = gc if dt_bias is None else gc + dt_bias.to(dt).view(1, HV, 1, 1, K)
        ea = torch.exp(A_log.to(dt)).view(1, HV, 1, 1, 1)
        sg = torch.sigmoid(ea * s)
        dz = dgate * lower_bound * sg * (1 - sg)
        dgc = torch.where(vmask, dz * ea, zero)
        dA_log = (dgc * s).sum(dim=(0, 2, 3, 4))
        ddt_bias = dgc.sum(dim=(0, 2, 3)).reshape(HV * K)
    elif gate_log:
        dgc = RCP_LN2 * _revcumsum(dG, 3)
        dA_log = ddt_bias = None
    else:
        dgc = dG
        dA_log = ddt_bias = None
    braw = _chunks(beta.to(dt), NT)
    if use_beta_sigmoid:
        sb = torch.sigmoid(braw)
        dbeta = dbeta * sb * (1 - sb)

    def l2_bwd(x, dxn):
        xc = _chunks(x.to(dt), NT)
        if not use_l2norm:
            return dxn
        r = 1.0 / torch.sqrt((xc * xc).sum(-1, keepdim=True) + EPS)
        xn = xc * r
        return r * (dxn - xn * (xn * dxn).sum(-1, keepdim=True))

    # grouped value heads: sum the q/k gradients over each group
    dqn_h = dqn.reshape(B, H, rep, NT, BT, K).sum(2)
    dkn_h = dkn.reshape(B, H, rep, NT, BT, K).sum(2)
    dq = _unchunk(l2_bwd(q, dqn_h), T)
    dk = _unchunk(l2_bwd(k, dkn_h), T)
    out = {
        "dq": dq, "dk": dk, "dv": _unchunk(dv_c, T), "dg": _unchunk(dgc, T),
        "dbeta": _unchunk(dbeta[..., None], T)[..., 0],
        "h": hall, "v_new": vnall, "dh": dhall, "dv_new": dvnall,
    }
    if use_gate:
        out["dA_log"] = dA_log
        out["ddt_bias"] = ddt_bias
    if initial_state is not None:
        out["dh0"] = dh0.transpose(-1, -2) if state_v_first else dh0
    return out

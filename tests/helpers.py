"""Shared test helpers (tolerances, seeded parameters)."""

import torch


def rel_err(a, b):
    """max|a-b| / max|b| (the stricter per-tensor form of the bf16 bar)."""
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def max_abs(a, b):
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def polar_params(H, d, *, seed=0, prior=False, dtype=torch.float32, device="cpu"):
    """Polar parameters: the reference priors (model/reference.py:17-20) or N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    if prior:
        p = dict(v_null=torch.randn(H, d, generator=g) * 0.1,
                 null_base=torch.full((H,), 2.0), null_slope_raw=torch.full((H,), 0.5),
                 len_gain_raw=torch.full((H,), -1.0), mag_beta_raw=torch.full((H,), -1.5))
    else:
        p = {n: torch.randn(*s, generator=g) for n, s in
             (("v_null", (H, d)), ("null_base", (H,)), ("null_slope_raw", (H,)),
              ("len_gain_raw", (H,)), ("mag_beta_raw", (H,)))}
    return {n: t.to(device=device, dtype=dtype) for n, t in p.items()}


_CH = 64


def _to_chunks(x, NC):
    """(B, T, H, ...) -> (B*H, NC, 64, ...), zero-padded to NC * 64 tokens."""
    B, T, H = x.shape[:3]
    pad = NC * _CH - T
    if pad:
        x = torch.nn.functional.pad(x, (0, 0) * (x.dim() - 2) + (0, pad))
    return x.movedim(2, 1).reshape(B * H, NC, _CH, *x.shape[3:])


def _from_chunks(x, B, T):
    """(B*H, NC, 64, ...) -> (B, T, H, ...)."""
    BH, NC = x.shape[:2]
    return x.reshape(B, BH // B, NC * _CH, *x.shape[3:]).movedim(1, 2)[:, :T].contiguous()


def bwd16_prep_reference(q, k, v, g, beta, dO, tile_dtype, scale=1.0, l2norm=True):
    """fp32 torch restatement of ``gated_delta_bwd16_prep``: the raw q, k rows
    l2-normalised (x / max(|x|, 1e-12)) with q then times scale, and per 64-token chunk
    (zero padding past T) lg = cumsum(g), Ga = exp(lg), w = exp(lg_C - lg),
    E[p,s] = exp(lg_p - lg_s) (s <= p), A = E o K K^T (s < p),
    T = (I + diag(beta) A)^-1, Rq = E o Q K^T.  Returns a dict with the op's tiles (kr, kt,
    qr, qt, tm, tt, rt, vt, ot, got in tile_dtype, f fp32) and the fp32 chunk matrices the
    local restatement takes."""
    B, T, H, D = q.shape
    NC = (T + _CH - 1) // _CH
    BH = B * H
    dev = q.device
    qf, kf = q.float(), k.float()
    if l2norm:
        nq, nk = qf.norm(dim=-1), kf.norm(dim=-1)
        iq, ik = scale / nq.clamp_min(1e-12), 1.0 / nk.clamp_min(1e-12)
        uq2 = torch.where(nq > 1e-12, 1.0 / nq.square(), torch.zeros_like(nq))
        uk2 = torch.where(nk > 1e-12, 1.0 / nk.square(), torch.zeros_like(nk))
    else:
        iq, ik = torch.full_like(qf[..., 0], scale), torch.ones_like(kf[..., 0])
        uq2, uk2 = torch.zeros_like(iq), torch.zeros_like(ik)
    Q, K, V, dOc = (_to_chunks(t, NC) for t in (qf * iq[..., None], kf * ik[..., None], v.float(), dO.float()))
    qraw, kraw = _to_chunks(qf, NC), _to_chunks(kf, NC)
    gc, bc = _to_chunks(g.float(), NC), _to_chunks(beta.float(), NC)
    iq, ik, uq2, uk2 = (_to_chunks(x, NC) for x in (iq, ik, uq2, uk2))
    lg = gc.cumsum(-1)
    Ga = lg.exp()
    w = (lg[..., -1:] - lg).exp()
    GaC = Ga[..., -1]
    idx = torch.arange(_CH, device=dev)
    incl = idx[:, None] >= idx[None, :]
    strict = idx[:, None] > idx[None, :]
    E = (lg[..., :, None] - lg[..., None, :]).masked_fill(~incl, float("-inf")).exp()
    Kt = K.transpose(-1, -2)
    A = (E * (K @ Kt)).masked_fill(~strict, 0.0)
    eye = torch.eye(_CH, device=dev, dtype=torch.float32)
    Tm = torch.linalg.solve_triangular(eye + bc[..., :, None] * A, eye.expand(BH, NC, _CH, _CH),
                                       upper=False, unitriangular=True)
    Rq = E * (Q @ Kt)

    def tile(x):
        return x.to(tile_dtype).contiguous()
    f = torch.stack((Ga, w, bc, GaC[..., None].expand_as(Ga), lg, iq, ik, uq2, uk2), dim=-2).contiguous()
    out = dict(kr=tile(K), kt=tile(Kt), qr=tile(Q), qt=tile(Q.transpose(-1, -2)), tm=tile(Tm),
               tt=tile(Tm.transpose(-1, -2)), rt=tile(Rq.transpose(-1, -2)), vt=tile(V.transpose(-1, -2)),
               ot=tile(dOc.transpose(-1, -2)), got=tile((Ga[..., None] * dOc).transpose(-1, -2)), f=f)
    out.update(B=B, T=T, Q=Q, K=K, V=V, dOc=dOc, bc=bc, Ga=Ga, w=w, GaC=GaC, incl=incl, strict=strict,
               E=E, A=A, Tm=Tm, Rq=Rq, qraw=qraw, kraw=kraw, iq=iq, ik=ik, uq2=uq2, uk2=uk2)
    return out


CHAIN_TILES = ("kr", "kt", "qt", "tm", "tt", "rt", "vt", "ot", "got", "f")


def bwd16_chain_reference(kr, kt, qt, tm, tt, rt, vt, ot, got, f, s0, dst):
    """fp32 torch restatement of ``gated_delta_bwd16_chain`` on the same tiles (the
    kernel's products round their right operand -- the state, Y, U, dU, dY -- to 16 bits;
    this one does not).  Forward chain: U = T diag(beta)(V - diag(Ga) K S),
    S <- Ga_C S + K^T diag(w) U; backward chain: dU = diag(w) K dS + Rq^T dO,
    dY = T^T dU, dS <- Ga_C dS + Q^T (Ga dO) - K^T diag(Ga beta) dY.
    Returns (s_entry, ds_end, u, dy, ds0) as the op does, in fp32."""
    BH, NC, C, D = kr.shape
    F = lambda x: x.float()  # noqa: E731
    o = dict(device=kr.device, dtype=torch.float32)
    S = torch.zeros(BH, D, D, **o) if s0 is None else s0.float().clone()
    s_entry, ds_end = torch.empty(BH, NC, D, D, **o), torch.empty(BH, NC, D, D, **o)
    u, dy = torch.empty(BH, NC, C, D, **o), torch.empty(BH, NC, C, D, **o)
    for c in range(NC):
        Ga, w, b, GaC = f[:, c, 0], f[:, c, 1], f[:, c, 2], f[:, c, 3, :1, None]
        s_entry[:, c] = S
        U = F(tm[:, c]) @ (b[..., None] * (F(vt[:, c]).transpose(-1, -2) - Ga[..., None] * (F(kr[:, c]) @ S)))
        u[:, c] = U
        S = GaC * S + F(kt[:, c]) @ (w[..., None] * U)
    dS = torch.zeros(BH, D, D, **o) if dst is None else dst.float().clone()
    for c in reversed(range(NC)):
        Ga, w, b, GaC = f[:, c, 0], f[:, c, 1], f[:, c, 2], f[:, c, 3, :1, None]
        ds_end[:, c] = dS
        dU = w[..., None] * (F(kr[:, c]) @ dS) + F(rt[:, c]) @ F(ot[:, c]).transpose(-1, -2)
        dY = F(tt[:, c]) @ dU
        dy[:, c] = dY
        dS = GaC * dS + F(qt[:, c]) @ F(got[:, c]).transpose(-1, -2) - F(kt[:, c]) @ ((Ga * b)[..., None] * dY)
    return s_entry, ds_end, u, dy, dS


def bwd16_local_reference(p, s_entry, ds_end, u, dy):
    """fp32 torch restatement of ``gated_delta_bwd16_local``: every gradient local to a
    chunk from the prep's matrices ``p`` (``bwd16_prep_reference``) and the chain's
    outputs.  dV = diag(beta) dY; dL = -(dY U^T) strictly lower, dA = diag(beta) dL;
    dRq = dO U^T lower; dbeta = rowsum(dY o (V - diag(Ga) K S0)) + rowsum(dL o A);
    dK = (dA o E + (dA o E)^T) K + (dRq o E)^T Q - diag(Ga beta) dY S0^T + diag(w) U dS^T;
    dQ = (dRq o E) K + diag(Ga) dO S0^T; dlg = rowsum - colsum of dA o A and dRq o Rq
    + Ga o (rowsum(dO o Q S0) - beta o rowsum(dY o K S0)) - w o rowsum(K dS o U), plus
    sum(w o rowsum(K dS o U)) + Ga_C <dS, S0> at the chunk's last token; dg = the
    reverse cumulative sum of dlg within the chunk; dq, dk then taken through the l2 norm
    and scale to the raw rows.  Returns dq, dk, dv, dg, dbeta in (B, T, H, .) fp32."""
    Q, K, V, dOc, bc, Ga, w, GaC = (p[n] for n in ("Q", "K", "V", "dOc", "bc", "Ga", "w", "GaC"))
    E, A, Rq, incl, strict = (p[n] for n in ("E", "A", "Rq", "incl", "strict"))
    B, T = p["B"], p["T"]
    S0, dS, U, dY = (x.float() for x in (s_entry, ds_end, u, dy))
    KS, QS = K @ S0, Q @ S0
    Vres = V - Ga[..., None] * KS
    Ut = U.transpose(-1, -2)
    KdS = K @ dS
    dV = bc[..., None] * dY
    dL = -(dY @ Ut).masked_fill(~strict, 0.0)
    dA = bc[..., None] * dL
    db = (dY * Vres).sum(-1) + (dL * A).sum(-1)
    GA = dA * E
    dRq = (dOc @ Ut).masked_fill(~incl, 0.0)
    GR = dRq * E
    S0t = S0.transpose(-1, -2)
    dK = ((GA + GA.transpose(-1, -2)) @ K + GR.transpose(-1, -2) @ Q
          - (Ga * bc)[..., None] * (dY @ S0t) + w[..., None] * (U @ dS.transpose(-1, -2)))
    dQ = GR @ K + Ga[..., None] * (dOc @ S0t)
    # the l2 norm's backward to the raw rows: dx = i_x dX - i_x u_x2 x (x . dX)
    qraw, kraw, iq, ik, uq2, uk2 = (p[n] for n in ("qraw", "kraw", "iq", "ik", "uq2", "uk2"))
    dQ = iq[..., None] * dQ - (iq * uq2 * (qraw * dQ).sum(-1))[..., None] * qraw
    dK = ik[..., None] * dK - (ik * uk2 * (kraw * dK).sum(-1))[..., None] * kraw
    dAA, dRR = dA * A, dRq * Rq
    dw = (KdS * U).sum(-1)
    dlg = (dAA.sum(-1) - dAA.sum(-2) + dRR.sum(-1) - dRR.sum(-2)
           + Ga * ((dOc * QS).sum(-1) - bc * (dY * KS).sum(-1)) - w * dw)
    dlg[..., -1] += (w * dw).sum(-1) + GaC * (dS * S0).sum((-2, -1))
    dg = dlg.flip(-1).cumsum(-1).flip(-1)
    return (_from_chunks(dQ, B, T), _from_chunks(dK, B, T), _from_chunks(dV, B, T),
            _from_chunks(dg, B, T), _from_chunks(db, B, T))

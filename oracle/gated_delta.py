"""CPU oracle for the additive gated-delta (Titans / Gated-DeltaNet) memory
(test infrastructure only; see ``oracle/__init__``).

Recurrence per head (FLA convention, ``scripts/titans_proto.py:53-66``)::

    M   <- gamma_t * M                 decay first
    u_t  = beta_t * (v_t - M k_t)      predict on the decayed state
    M   <- M + u_t k_t^T               undecayed write
    r_t  = M q_t                       self-inclusive readout

Here ``M`` is (dv, dk) -- the "torch" layout.  The engine's state tables and the
FLA contract store the transpose, ``[K, V]`` = (dk, dv)
(``inference/models/atma.py:48-51``); functions below say which layout they use.
"""

import torch
import torch.nn.functional as F


def gated_delta_sequential(q, k, v, gamma, beta, S0=None):
    """Token-by-token definition.  ``scripts/titans_proto.py:53-76``.

    q,k: (B,H,N,dk); v: (B,H,N,dv); gamma,beta: (B,H,N); S0: (B,H,dv,dk) or None.
    Returns R (B,H,N,dv) and the final state (B,H,dv,dk)."""
    B, H, N, dk = q.shape
    dv = v.shape[-1]
    M = torch.zeros(B, H, dv, dk, dtype=q.dtype) if S0 is None else S0.clone()
    out = []
    for t in range(N):
        M = gamma[:, :, t, None, None] * M
        pred = (M @ k[:, :, t, :, None])[..., 0]                   # (B,H,dv)
        u = beta[:, :, t, None] * (v[:, :, t] - pred)
        M = M + u[..., :, None] * k[:, :, t, None, :]
        out.append((M @ q[:, :, t, :, None])[..., 0])
    return torch.stack(out, dim=2), M


def gated_delta_chunked(q, k, v, gamma, beta, chunk=64, S0=None):
    """Chunkwise-parallel UT form.  ``model/blocks.py:375-423``.

    Inside a chunk with inclusive decay products g_p = prod_{l<=p} gamma_l, the
    increments u solve the unit lower-triangular system
    ``(I + diag(beta) D) U = diag(beta)(V - diag(g) K M0^T)`` with
    ``D[p,s] = (g_p/g_s) k_s.k_p`` (s < p); the readout is
    ``R = diag(g) Q M0^T + Rq U`` with ``Rq[p,s] = (g_p/g_s) k_s.q_p`` (s <= p), and
    the state advances to ``g_C M0 + sum_s (g_C/g_s) u_s k_s^T``.

    Same shapes / layout as ``gated_delta_sequential``."""
    B, H, N, dk = q.shape
    dv = v.shape[-1]
    M = torch.zeros(B, H, dv, dk, dtype=q.dtype) if S0 is None else S0.clone()
    pieces = []
    for c0 in range(0, N, chunk):
        c1 = min(c0 + chunk, N)
        C = c1 - c0
        qc, kc, vc = q[:, :, c0:c1], k[:, :, c0:c1], v[:, :, c0:c1]
        bc = beta[:, :, c0:c1]
        lg = torch.cumsum(torch.log(gamma[:, :, c0:c1]), dim=-1)   # log g_p (inclusive)
        rel = lg[..., :, None] - lg[..., None, :]                  # log(g_p / g_s)
        p_idx = torch.arange(C)[:, None]
        s_idx = torch.arange(C)[None, :]
        below = (s_idx < p_idx)
        on_or_below = (s_idx <= p_idx)
        ratio_strict = torch.where(below, torch.exp(rel.clamp(max=0.0)), torch.zeros_like(rel))
        ratio_incl = torch.where(on_or_below, torch.exp(rel.clamp(max=0.0)), torch.zeros_like(rel))
        D = ratio_strict * (kc @ kc.transpose(-1, -2))             # [p, s] = k_p.k_s
        Rq = ratio_incl * (qc @ kc.transpose(-1, -2))              # [p, s] = q_p.k_s
        g = torch.exp(lg)
        carry_k = g[..., None] * (kc @ M.transpose(-1, -2))        # g_p M0 k_p   (C, dv)
        carry_q = g[..., None] * (qc @ M.transpose(-1, -2))        # g_p M0 q_p
        lower = bc[..., None] * D                                  # strictly lower part
        rhs = bc[..., None] * (vc - carry_k)
        U = torch.linalg.solve_triangular(lower, rhs, upper=False, unitriangular=True)
        pieces.append(carry_q + Rq @ U)
        tail = torch.exp(lg[..., -1:] - lg)                        # g_C / g_s
        M = torch.exp(lg[..., -1])[..., None, None] * M + (tail[..., None] * U).transpose(-1, -2) @ kc
    return torch.cat(pieces, dim=2), M


def gated_delta_chunked_backward(q, k, v, gl, beta, S0, dO, dST, chunk=64):
    """Chunked (WY / UT) backward of the recurrence, per sequence-head, in the ``[K, V]``
    layout (S (dk, dv)).  The algorithm FLA's autograd of ``chunk_gated_delta_rule``
    follows (the reference trains through it, ``model/blocks.py:44-84``), restated from
    the chunked forward of ``gated_delta_chunked`` by reverse-mode differentiation.

    q, k: (T, dk) (q already scaled / normalised, k normalised); v, dO: (T, dv); gl: (T,)
    log decay; beta: (T,); S0, dST: (dk, dv) (dST = dL/dS_final).  Inside a chunk with
    inclusive log decays lg, Ga = exp(lg), E[p,s] = exp(lg_p - lg_s), A = E o K K^T
    (strictly lower), T = (I + diag(beta) A)^-1, Rq = E o Q K^T (lower incl.) and
    w = exp(lg_C - lg), the forward is U = T diag(beta)(V - diag(Ga) K S0),
    O = diag(Ga) Q S0 + Rq U, S_end = Ga_C S0 + K^T diag(w) U.  Backward, with dS the
    gradient of S_end::

        dU = Rq^T dO + diag(w) K dS;   dY = T^T dU;   dV = diag(beta) dY
        dS0 = Ga_C dS + Q^T diag(Ga) dO - K^T diag(Ga beta) dY
        dL = -(dY U^T) (strictly lower);  dA = diag(beta) dL;  dRq = dO U^T (lower)
        dbeta = rowsum(dY o (V - diag(Ga) K S0)) + rowsum(dL o A)
        dK = (dA o E) K + (dA o E)^T K + (dRq o E)^T Q - diag(Ga beta) dY S0^T + diag(w) U dS^T
        dQ = (dRq o E) K + diag(Ga) dO S0^T
        dlg = rowsum - colsum of (dA o A) and of (dRq o Rq) + Ga o (rowsum(dO o Q S0)
              - beta o rowsum(dY o K S0)) - w o rowsum(K dS o U),
              dlg[C-1] += sum(w o rowsum(K dS o U)) + Ga_C <dS, S0>;  dgl = reverse cumsum

    Returns (dq, dk, dv, dgl, dbeta, dS0) in the inputs' dtype."""
    T = q.shape[0]
    dt = q.dtype
    S = S0.clone()
    entry = []
    for c0 in range(0, T, chunk):                      # entry states of the chunks
        c1 = min(c0 + chunk, T)
        Q, K, V, g, b = q[c0:c1], k[c0:c1], v[c0:c1], gl[c0:c1], beta[c0:c1]
        n = c1 - c0
        lg = torch.cumsum(g, 0)
        Ga = torch.exp(lg)
        E = torch.exp(lg[:, None] - lg[None, :])
        A = E * torch.tril(torch.ones(n, n, dtype=dt), -1) * (K @ K.T)
        Tm = torch.linalg.inv(torch.eye(n, dtype=dt) + b[:, None] * A)
        U = Tm @ (b[:, None] * (V - Ga[:, None] * (K @ S)))
        entry.append(S)
        S = Ga[-1] * S + K.T @ (torch.exp(lg[-1] - lg)[:, None] * U)
    dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    dgl, db = torch.zeros_like(gl), torch.zeros_like(beta)
    dS = dST.clone()
    starts = list(range(0, T, chunk))
    for ci in reversed(range(len(starts))):
        c0 = starts[ci]
        c1 = min(c0 + chunk, T)
        n = c1 - c0
        Q, K, V, g, b, dOc, S0c = q[c0:c1], k[c0:c1], v[c0:c1], gl[c0:c1], beta[c0:c1], dO[c0:c1], entry[ci]
        lg = torch.cumsum(g, 0)
        Ga = torch.exp(lg)
        E = torch.exp(lg[:, None] - lg[None, :])
        lower = torch.tril(torch.ones(n, n, dtype=dt), -1)
        incl = torch.tril(torch.ones(n, n, dtype=dt))
        A = E * lower * (K @ K.T)
        Tm = torch.linalg.inv(torch.eye(n, dtype=dt) + b[:, None] * A)
        KS, QS = K @ S0c, Q @ S0c
        Vres = V - Ga[:, None] * KS
        U = Tm @ (b[:, None] * Vres)
        Rq = E * incl * (Q @ K.T)
        w = torch.exp(lg[-1] - lg)
        KdS = K @ dS
        dU = Rq.T @ dOc + w[:, None] * KdS
        dY = Tm.T @ dU
        dS0 = Ga[-1] * dS + Q.T @ (Ga[:, None] * dOc) - K.T @ ((Ga * b)[:, None] * dY)
        dv[c0:c1] = b[:, None] * dY
        dL = -(dY @ U.T) * lower
        dA = b[:, None] * dL
        db[c0:c1] = (dY * Vres).sum(1) + (dL * A).sum(1)
        GA = dA * E
        dRq = (dOc @ U.T) * incl
        GR = dRq * E
        dk[c0:c1] = (GA @ K + GA.T @ K + GR.T @ Q - (Ga * b)[:, None] * (dY @ S0c.T)
                     + w[:, None] * (U @ dS.T))
        dq[c0:c1] = GR @ K + Ga[:, None] * (dOc @ S0c.T)
        dlg = (dA * A).sum(1) - (dA * A).sum(0) + (dRq * Rq).sum(1) - (dRq * Rq).sum(0)
        dlg = dlg + Ga * ((dOc * QS).sum(1) - b * (dY * KS).sum(1))
        dw = (KdS * U).sum(1)
        dlg = dlg - w * dw
        dlg[-1] = dlg[-1] + (w * dw).sum() + Ga[-1] * (dS * S0c).sum()
        dgl[c0:c1] = torch.flip(torch.cumsum(torch.flip(dlg, [0]), 0), [0])
        dS = dS0
    return dq, dk, dv, dgl, db, dS


def l2_normalize(x, eps=1e-12):
    """``F.normalize(x, dim=-1)``: x / max(|x|, eps) -- the unit-key normalisation of the
    memory branch (``model/blocks.py:481-482``, ``kernel/gated_delta_triton.py:58-60``)."""
    return x / x.norm(dim=-1, keepdim=True).clamp_min(eps)


def gated_delta_decode_step(q, k, v, gamma, beta, state_table, slots, eps=1e-12):
    """One batched decode step IN PLACE on a ``[K, V]`` (dk, dv) fp32 state table.

    Closed form of ``kernel/gated_delta_triton.py:1-20`` / the torch route of
    ``inference/models/atma.py:362-372``::

        qn, kn = q/|q|, k/|k|;  Sd = gamma*S;  pred_v = sum_k kn_k Sd[k,v]
        u = beta*(v - pred);    S' = Sd + kn u^T (stored);   r_v = sum_k qn_k S'[k,v]

    q,k,v: (B,H,d); gamma,beta: (B,H); state_table (max_seqs,H,dk,dv); slots (B,).
    Returns r (B,H,dv) fp32 (fp64 for fp64 inputs)."""
    wd = torch.float64 if q.dtype == torch.float64 else torch.float32
    qn = l2_normalize(q.to(wd), eps)
    kn = l2_normalize(k.to(wd), eps)
    idx = slots.long()
    S = state_table[idx].to(wd)                                    # (B,H,dk,dv)
    Sd = gamma.to(wd)[..., None, None] * S
    pred = (kn[..., None, :] @ Sd)[..., 0, :]                      # (B,H,dv)
    u = beta.to(wd)[..., None] * (v.to(wd) - pred)
    S_new = Sd + kn[..., :, None] * u[..., None, :]
    state_table[idx] = S_new.to(state_table.dtype)
    return (qn[..., None, :] @ S_new)[..., 0, :]


def chunk_gated_delta_rule(q, k, v, g, beta, scale=1.0, initial_state=None,
                           output_final_state=False, use_qk_l2norm_in_kernel=False, chunk=64):
    """The FLA ``chunk_gated_delta_rule`` contract exactly as the reference calls it
    (``model/blocks.py:44-49``, ``inference/models/atma.py:285-287,318-322``).

    q,k: (B,T,H,dk); v: (B,T,H,dv); g: (B,T,H) log-decay (log gamma); beta: (B,T,H);
    initial_state: (B,H,dk,dv) ``[K,V]`` fp32 or None.  q,k are L2-normalised when
    ``use_qk_l2norm_in_kernel`` (the reference's torch route uses ``F.normalize``), q is
    then multiplied by ``scale``.  Arithmetic in fp32 (fp64 stays fp64).
    Returns (o (B,T,H,dv) in q's dtype, final_state (B,H,dk,dv) fp32 or None)."""
    wd = torch.float64 if q.dtype == torch.float64 else torch.float32
    qf, kf, vf = (x.to(wd).transpose(1, 2) for x in (q, k, v))    # (B,H,T,d)
    if use_qk_l2norm_in_kernel:
        qf, kf = l2_normalize(qf), l2_normalize(kf)
    qf = qf * scale
    gamma = torch.exp(g.to(wd)).transpose(1, 2)
    bt = beta.to(wd).transpose(1, 2)
    S0 = None if initial_state is None else initial_state.to(wd).transpose(-1, -2)
    R, S = gated_delta_chunked(qf, kf, vf, gamma, bt, chunk=chunk, S0=S0)
    o = R.transpose(1, 2).to(q.dtype)
    final = S.transpose(-1, -2).to(torch.float32 if wd == torch.float32 else wd) if output_final_state else None
    return o, final


def prefill_flops(B, T, H, d, chunk=64):
    """Algorithmic gated-delta prefill FLOPs ``B*T*H*(6 d^2 + 4 C d)``: three d x d state
    products per token plus four causally-halved C x C x d intra-chunk products."""
    return float(B) * T * H * (6 * d * d + 4 * chunk * d)

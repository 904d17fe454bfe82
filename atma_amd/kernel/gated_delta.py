"""Gated-delta memory ops backed by libatma_hip.so.

* ``gated_delta_decode_step`` mirrors ``kernel/gated_delta_triton.py:78-117``.
* ``chunk_gated_delta_rule`` replaces the third-party
  ``fla.ops.gated_delta_rule.chunk_gated_delta_rule`` with the contract the
  reference uses (``model/blocks.py:44-49``, ``inference/models/atma.py:285-287``).

Convention (``scripts/titans_proto.py:53-66``): decay first, predict on the decayed
state, undecayed write, self-inclusive readout ``r_t = M_t q_t``; states are fp32
in the ``[K, V]`` = (dk, dv) layout.
"""

import torch

from .. import _ops  # noqa: F401  (registers torch.ops.atma_hip.*)


@torch.no_grad()
def gated_delta_decode_step(q, k, v, gamma, beta, state_table, slots, eps=1e-12, block_v=None):
    """One batched gated-delta step, IN PLACE on the slot-indexed state table.

    q: (B, H, d), k, v: (B, Hkv, d) current-token tensors with H % Hkv == 0: query
    head h reads key / value head h // (H // Hkv), so grouped KV heads need no
    expansion (Hkv == H is the reference's expanded call).
    gamma, beta: (B, H) retention / write strength.  state_table: (max_seqs, H, dk, dv)
    fp32 ``[K, V]``, updated in place.  slots: (B,) int64 rows of the table.
    ``block_v`` (a Triton tile knob) is accepted and ignored.
    Returns r (B, H, dv) fp32.  Graph capturable."""
    if q.dim() != 3 or k.dim() != 3 or k.shape[0] != q.shape[0] or k.shape[2] != q.shape[2] \
            or v.dim() != 3 or v.shape[:2] != k.shape[:2]:
        raise ValueError("q: (B, H, d) and k, v: (B, Hkv, d) required")
    B, H, dk = q.shape
    if k.shape[1] < 1 or H % k.shape[1]:
        raise ValueError(f"q heads ({H}) must be a multiple of k/v heads ({k.shape[1]})")
    if state_table.dim() != 4 or state_table.shape[1] != H or state_table.shape[2] != dk:
        raise ValueError(f"state_table {tuple(state_table.shape)} incompatible with q {tuple(q.shape)}")
    if v.shape[2] != state_table.shape[3]:
        raise ValueError("v's last dim must equal the state's dv")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share a dtype")
    gamma = gamma.to(torch.float32).reshape(B, H).contiguous()
    beta = beta.to(torch.float32).reshape(B, H).contiguous()
    slots = slots.to(device=q.device, dtype=torch.int64).reshape(B).contiguous()
    return torch.ops.atma_hip.gated_delta_decode_step(q, k, v, gamma, beta, state_table, slots,
                                                      float(eps))


def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None,
                           output_final_state=False, use_qk_l2norm_in_kernel=False,
                           cu_seqlens=None, head_first=False, gate_bias=None, start_signal=None):
    """Chunked gated-delta prefill with state carry (FLA contract).

    q: (B, T, H, dk); k: (B, T, Hkv, dk); v: (B, T, Hkv, dv) with H % Hkv == 0 (query
    head h reads key / value head h // (H // Hkv); Hkv == H is the expanded form FLA
    takes); g: (B, T, H) log-decay (log gamma); beta: (B, T, H); initial_state: (B, H, dk, dv) fp32 or None.  With
    ``use_qk_l2norm_in_kernel`` q and k are L2-normalised (x / max(|x|, 1e-12)) before
    the recurrence; q is then scaled by ``scale`` (default dk**-0.5, FLA's default;
    the reference passes 1.0).
    ``gate_bias=(g_bias, b_bias)`` (an extension, no FLA counterpart): ``g`` and ``beta``
    are the memory branch's raw gate logits, and the kernel applies
    ``g = logsigmoid(g + g_bias)``, ``beta = sigmoid(beta + b_bias)`` as it loads them,
    bit-identical to ``gated_delta_gates`` followed by the plain call, one launch fewer.
    ``start_signal`` (a :class:`StartSignal`, also an extension): armed by the caller, it
    is raised as the recurrence kernel starts, so another stream can hold work back until
    then (``StartSignal.wait``); results are unaffected.
    Returns (o (B, T, H, dv) in q's dtype, final_state (B, H, dk, dv) fp32 or None)."""
    if cu_seqlens is not None or head_first:
        raise NotImplementedError("cu_seqlens / head_first layouts are not supported")
    _check_args(q, k, v, g, beta, initial_state)
    if q.shape[1] > 0 and torch.is_grad_enabled() and \
            any(isinstance(t, torch.Tensor) and t.requires_grad for t in (q, k, v, g, beta, initial_state)):
        if gate_bias is not None:   # raw logits: the activations as differentiable torch ops
            g = torch.nn.functional.logsigmoid(g.float() + float(gate_bias[0]))
            beta = torch.sigmoid(beta.float() + float(gate_bias[1]))
        if start_signal is not None:  # nothing to overlap with: release the waiting stream now
            start_signal.flag.fill_(start_signal.epoch)
        return _chunk_gated_delta_train(q, k, v, g, beta, scale, initial_state, output_final_state,
                                        use_qk_l2norm_in_kernel)
    with torch.no_grad():
        return _chunk_gated_delta_infer(q, k, v, g, beta, scale, initial_state, output_final_state,
                                        use_qk_l2norm_in_kernel, gate_bias, start_signal)


def _check_args(q, k, v, g, beta, initial_state):
    """Shapes and dtypes of ``chunk_gated_delta_rule``'s operands, checked before any
    launch on both the inference and the autograd route (the kernels index g, beta and
    the state by these shapes without bounds checks)."""
    if q.dim() != 4 or k.dim() != 4 or k.shape[:2] != q.shape[:2] or k.shape[3] != q.shape[3] \
            or v.dim() != 4 or v.shape[:3] != k.shape[:3]:
        raise ValueError("q: (B, T, H, dk), k: (B, T, Hkv, dk) and v: (B, T, Hkv, dv) required")
    B, T, H, dk = q.shape
    if k.shape[2] < 1 or H % k.shape[2]:
        raise ValueError(f"q heads ({H}) must be a multiple of k/v heads ({k.shape[2]})")
    dv = v.shape[3]
    if tuple(g.shape) != (B, T, H) or tuple(beta.shape) != (B, T, H):
        raise ValueError("g and beta must be (B, T, H)")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share a dtype")
    if initial_state is not None and tuple(initial_state.shape) != (B, H, dk, dv):
        raise ValueError(f"initial_state must be (B, H, dk, dv) = {(B, H, dk, dv)}")


def _chunk_gated_delta_infer(q, k, v, g, beta, scale, initial_state, output_final_state,
                             use_qk_l2norm_in_kernel, gate_bias, start_signal):
    B, T, H, dk = q.shape
    dv = v.shape[3]
    if initial_state is not None:
        initial_state = initial_state.to(torch.float32).contiguous()
    if scale is None:
        scale = dk ** -0.5
    if start_signal is not None and (B == 0 or T == 0):
        start_signal.flag.fill_(start_signal.epoch)   # no recurrence launch: raise it here
    if T == 0:
        o = q.new_empty((B, 0, H, dv))
        if not output_final_state:
            return o, None
        final = (initial_state.clone() if initial_state is not None
                 else torch.zeros((B, H, dk, dv), device=q.device, dtype=torch.float32))
        return o, final
    g = g.to(torch.float32).contiguous()
    beta = beta.to(torch.float32).contiguous()
    gb, bb = (0.0, 0.0) if gate_bias is None else (float(gate_bias[0]), float(gate_bias[1]))
    outs = torch.ops.atma_hip.chunk_gated_delta_rule(q, k, v, g, beta, initial_state, float(scale),
                                                     bool(use_qk_l2norm_in_kernel),
                                                     bool(output_final_state),
                                                     None if start_signal is None else start_signal.flag,
                                                     0 if start_signal is None else start_signal.epoch,
                                                     gate_bias is not None, gb, bb)
    return outs[0], (outs[1] if output_final_state else None)


class _GatedDeltaFn(torch.autograd.Function):
    """The recurrence on prepared fp32 operands (q scaled and normalised, k normalised,
    log decay g, beta, [K, V] initial state): forward by the chunked prefill kernel,
    backward by ``gated_delta_bwd`` (state checkpoints every 64 tokens, sub-blocks
    recomputed in registers)."""

    @staticmethod
    def forward(ctx, qs, kn, v, g, beta, S0):
        o, S = torch.ops.atma_hip.gated_delta_fwd(qs, kn, v, g, beta, S0)
        ctx.save_for_backward(qs, kn, v, g, beta, S0)
        return o, S

    @staticmethod
    def backward(ctx, dO, dS):
        qs, kn, v, g, beta, S0 = ctx.saved_tensors
        dO = torch.zeros_like(v) if dO is None else dO.to(torch.float32).contiguous()
        dS = None if dS is None else dS.to(torch.float32).contiguous()
        dq, dk, dv, dg, db, ds0 = torch.ops.atma_hip.gated_delta_bwd(qs, kn, v, g, beta, S0, dO, dS)
        return dq, dk, dv, dg, db, (ds0 if S0 is not None else None)


_CH = 64  # chunk length of the chunked (WY) form


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


def _gated_delta_bwd16(qs, kn, v, g, beta, S0, dO, dST, tile_dtype):
    """Chunked (WY) backward of the recurrence for 16-bit training, the algorithm of the
    FLA autograd the reference trains through (``model/blocks.py:44-84``).  In a chunk with
    inclusive log decays lg, Ga = exp(lg), w = exp(lg_C - lg), E[p,s] = exp(lg_p - lg_s)
    (s <= p), A = E o K K^T (strictly lower), T = (I + diag(beta) A)^-1, Rq = E o Q K^T:
    U = T diag(beta)(V - diag(Ga) K S0), O = diag(Ga) Q S0 + Rq U,
    S_end = Ga_C S0 + K^T diag(w) U.  The state gradient dS runs backwards over the chunks:
    dU = Rq^T dO + diag(w) K dS, dY = T^T dU, dS <- Ga_C dS + Q^T diag(Ga) dO
    - K^T diag(Ga beta) dY.  That chain (and the forward one that recovers each chunk's
    S0) is ``gated_delta_bwd16_chain`` (16-bit MFMA, fp32 state); the per-chunk matrices
    it takes and every gradient local to a chunk are batched fp32 products here:
    dV = diag(beta) dY; dL = -(dY U^T) strictly lower, dA = diag(beta) dL;
    dRq = dO U^T lower; dbeta = rowsum(dY o (V - diag(Ga) K S0)) + rowsum(dL o A);
    dK = (dA o E + (dA o E)^T) K + (dRq o E)^T Q - diag(Ga beta) dY S0^T + diag(w) U dS^T;
    dQ = (dRq o E) K + diag(Ga) dO S0^T; dlg = rowsum - colsum of dA o A and dRq o Rq
    + Ga o (rowsum(dO o Q S0) - beta o rowsum(dY o K S0)) - w o rowsum(K dS o U), plus
    sum(w o rowsum(K dS o U)) + Ga_C <dS, S0> at the chunk's last token; dg = the
    reverse cumulative sum of dlg within the chunk.

    qs, kn, v, dO: (B, T, H, d) (q scaled and normalised, k normalised); g, beta (B, T, H);
    S0, dST (B, H, d, d) or None.  Returns dq, dk, dv, dg, dbeta (fp32, (B, T, H, .)) and
    dS0 (B, H, d, d)."""
    prep = _bwd16_prep(qs, kn, v, g, beta, dO, tile_dtype)
    B, H, D = qs.shape[0], qs.shape[2], qs.shape[3]
    s_entry, ds_end, dY, ds0 = torch.ops.atma_hip.gated_delta_bwd16_chain(
        *prep["tiles"], None if S0 is None else S0.float().reshape(B * H, D, D),
        None if dST is None else dST.float().reshape(B * H, D, D))
    return _bwd16_local(prep, s_entry, ds_end, dY) + (ds0.reshape(B, H, D, D),)


def _bwd16_prep(qs, kn, v, g, beta, dO, tile_dtype):
    """The per-chunk matrices of the chunked backward, and the operand tiles of
    ``gated_delta_bwd16_chain`` in ``tile_dtype`` (argument order of the op, up to f)."""
    B, T, H, D = qs.shape
    NC = (T + _CH - 1) // _CH
    BH = B * H
    dev = qs.device
    Q, K, V, dOc = (_to_chunks(t.float(), NC) for t in (qs, kn, v, dO))      # (BH, NC, C, D)
    gc, bc = _to_chunks(g.float(), NC), _to_chunks(beta.float(), NC)        # (BH, NC, C)
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
    f = torch.stack((Ga, w, bc, GaC[..., None].expand_as(Ga)), dim=-2).contiguous()
    tiles = (tile(K), tile(Kt), tile(Q.transpose(-1, -2)), tile(Tm), tile(Tm.transpose(-1, -2)),
             tile(Rq.transpose(-1, -2)), tile(V.transpose(-1, -2)), tile(dOc.transpose(-1, -2)),
             tile((Ga[..., None] * dOc).transpose(-1, -2)), f)
    return dict(B=B, T=T, Q=Q, K=K, V=V, dOc=dOc, bc=bc, Ga=Ga, w=w, GaC=GaC, incl=incl, strict=strict,
                E=E, A=A, Tm=Tm, Rq=Rq, tiles=tiles)


def _bwd16_local(p, s_entry, ds_end, dY):
    """Every gradient local to a chunk, from the chains' outputs (each chunk's entry
    state, the gradient of its exit state, dY).  Returns dq, dk, dv, dg, dbeta."""
    Q, K, V, dOc, bc, Ga, w, GaC = (p[n] for n in ("Q", "K", "V", "dOc", "bc", "Ga", "w", "GaC"))
    E, A, Tm, Rq, incl, strict = (p[n] for n in ("E", "A", "Tm", "Rq", "incl", "strict"))
    B, T = p["B"], p["T"]
    KS, QS = K @ s_entry, Q @ s_entry
    Vres = V - Ga[..., None] * KS
    U = Tm @ (bc[..., None] * Vres)
    Ut = U.transpose(-1, -2)
    KdS = K @ ds_end
    dV = bc[..., None] * dY
    dL = -(dY @ Ut).masked_fill(~strict, 0.0)
    dA = bc[..., None] * dL
    db = (dY * Vres).sum(-1) + (dL * A).sum(-1)
    GA = dA * E
    dRq = (dOc @ Ut).masked_fill(~incl, 0.0)
    GR = dRq * E
    S0t = s_entry.transpose(-1, -2)
    dK = ((GA + GA.transpose(-1, -2)) @ K + GR.transpose(-1, -2) @ Q
          - (Ga * bc)[..., None] * (dY @ S0t) + w[..., None] * (U @ ds_end.transpose(-1, -2)))
    dQ = GR @ K + Ga[..., None] * (dOc @ S0t)
    dAA, dRR = dA * A, dRq * Rq
    dw = (KdS * U).sum(-1)
    dlg = (dAA.sum(-1) - dAA.sum(-2) + dRR.sum(-1) - dRR.sum(-2)
           + Ga * ((dOc * QS).sum(-1) - bc * (dY * KS).sum(-1)) - w * dw)
    dlg[..., -1] += (w * dw).sum(-1) + GaC * (ds_end * s_entry).sum((-2, -1))
    dg = dlg.flip(-1).cumsum(-1).flip(-1)
    return (_from_chunks(dQ, B, T), _from_chunks(dK, B, T), _from_chunks(dV, B, T),
            _from_chunks(dg, B, T), _from_chunks(db, B, T))


class _GatedDelta16Fn(torch.autograd.Function):
    """The recurrence on prepared operands for 16-bit training (q scaled and normalised,
    k normalised, in fp32; v, log decay g, beta, fp32 [K, V] initial state): forward by
    the 16-bit chunked prefill kernel on the operands rounded to the input dtype,
    backward by the chunked (WY) form (``_gated_delta_bwd16``)."""

    @staticmethod
    def forward(ctx, qs, kn, v, g, beta, S0):
        td = v.dtype
        o, S = torch.ops.atma_hip.gated_delta_fwd(qs.to(td), kn.to(td), v, g, beta, S0)
        ctx.save_for_backward(qs, kn, v, g, beta, S0)
        return o, S

    @staticmethod
    def backward(ctx, dO, dS):
        qs, kn, v, g, beta, S0 = ctx.saved_tensors
        dO = torch.zeros(v.shape, device=v.device, dtype=torch.float32) if dO is None else dO
        dq, dk, dv, dg, db, ds0 = _gated_delta_bwd16(qs, kn, v, g, beta, S0, dO, dS, v.dtype)
        return dq, dk, dv.to(v.dtype), dg, db, (ds0 if S0 is not None else None)


def _chunk_gated_delta_train(q, k, v, g, beta, scale, initial_state, output_final_state, use_qk_l2norm):
    """Differentiable ``chunk_gated_delta_rule`` (the FLA autograd the reference trains
    through, ``model/blocks.py:44-84``).  The l2 norm, the scale and grouped-head expansion
    are torch ops (autograd differentiates them); the recurrence and its backward are HIP.
    fp32 inputs: fp32 arithmetic throughout (sequential backward).  16-bit inputs with
    dk = dv in {64, 128}: the 16-bit chunked forward and the chunked (WY) backward, 16-bit
    products with fp32 accumulation as FLA's kernels.  o is returned in q's dtype."""
    B, T, H, dk = q.shape
    if k.shape[2] != H:
        rep = H // k.shape[2]
        k, v = k.repeat_interleave(rep, dim=2), v.repeat_interleave(rep, dim=2)
    qf, kf = q.float(), k.float()
    if use_qk_l2norm:
        qf = torch.nn.functional.normalize(qf, dim=-1, eps=1e-12)
        kf = torch.nn.functional.normalize(kf, dim=-1, eps=1e-12)
    qs = qf * (dk ** -0.5 if scale is None else float(scale))
    S0 = None if initial_state is None else initial_state.float().contiguous()
    if q.dtype in (torch.bfloat16, torch.float16) and dk == v.shape[3] and dk in (64, 128):
        o, S = _GatedDelta16Fn.apply(qs.contiguous(), kf.contiguous(), v.contiguous(),
                                     g.float().contiguous(), beta.float().contiguous(), S0)
        return o, (S if output_final_state else None)
    o, S = _GatedDeltaFn.apply(qs.contiguous(), kf.contiguous(), v.float().contiguous(),
                               g.float().contiguous(), beta.float().contiguous(), S0)
    return o.to(q.dtype), (S if output_final_state else None)


def recurrence_pays_to_overlap(B, H, dv, dtype, device):
    """True when the recurrence kernel's grid (B*H workgroups per column slab: 32 columns
    for 16-bit inputs, 16 for fp32) takes at most a quarter of the CUs, so running Polar
    attention beside it (``StartSignal``) hides the recurrence's latency.  With more
    workgroups the two kernels compete for the same CUs and back to back is faster
    (measured: B = 8, T = 2,048, 256 workgroups: 0.219 ms back to back, 0.263 ms overlapped;
    B = 1, T = 65,536, 32 workgroups: 10.70 ms back to back, 8.90 ms overlapped)."""
    slab = 32 if dtype in (torch.bfloat16, torch.float16) else 16
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    return B * H * max(dv // slab, 1) <= cus // 4


class StartSignal:
    """Orders a launch on one stream after the start of the gated-delta recurrence on
    another.  The recurrence (one workgroup per CU, latency-bound) and Polar attention
    (which fills every CU) overlap only if the recurrence's workgroups are resident
    first; otherwise Polar's queue keeps every CU busy and the recurrence runs after it.

    Use: ``e = sig.arm()`` once per step; pass ``start_signal=sig`` to
    ``chunk_gated_delta_rule`` on the side stream; call ``sig.wait()`` on the main stream
    before the Polar launch.  The wait is a one-wave kernel with a time limit (a missed
    signal costs the overlap, never results).  Not for graph capture: the epoch is a
    launch argument, so a replayed graph would see an old epoch as already raised."""

    def __init__(self, device):
        self.flag = torch.zeros(1, dtype=torch.int32, device=device)
        self.epoch = 0

    def arm(self):
        self.epoch = self.epoch % 0x7FFFFFFE + 1
        return self.epoch

    def wait(self, timeout_us=20000):
        torch.ops.atma_hip.wait_start_flag(self.flag, self.epoch, int(timeout_us))


@torch.no_grad()
def gated_delta_gates(g_logit, b_logit, g_bias=0.0, b_bias=0.0, decay_as_prob=False):
    """The memory branch's gate activations in one launch (TitansMemory,
    ``model/blocks.py:426-490``): returns ``(logsigmoid(g_logit + g_bias),
    sigmoid(b_logit + b_bias))`` -- the log-decay and write strength
    ``chunk_gated_delta_rule`` takes -- or, with ``decay_as_prob``, the decode step's
    ``(sigmoid(g_logit + g_bias), sigmoid(b_logit + b_bias))``.  fp32 in and out."""
    g, beta = torch.ops.atma_hip.gated_delta_gates(g_logit.float(), b_logit.float(), float(g_bias),
                                                   float(b_bias), bool(decay_as_prob))
    return g, beta

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


class _GatedDelta16Fn(torch.autograd.Function):
    """The recurrence for 16-bit training on the raw q, k, v (H heads each), log decay g,
    beta and fp32 [K, V] initial state: forward by the 16-bit chunked prefill kernel (l2
    norm and scale applied in-kernel), backward by the chunked (WY) form
    (``gated_delta_bwd16``: a prep launch forming each chunk's matrices from the
    normalised rows, the chain launch carrying the state and its gradient across the
    chunks, and a launch forming every gradient local to a chunk, taken back through the
    l2 norm to the raw rows)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, S0, scale, l2norm):
        o, S = torch.ops.atma_hip.gated_delta_fwd(q, k, v, g, beta, S0, scale, l2norm)
        ctx.save_for_backward(q, k, v, g, beta, S0)
        ctx.scale, ctx.l2norm = scale, l2norm
        return o, S

    @staticmethod
    def backward(ctx, dO, dS):
        q, k, v, g, beta, S0 = ctx.saved_tensors
        dO = torch.zeros_like(v) if dO is None else dO.to(v.dtype)
        dq, dk, dv, dg, db, ds0 = torch.ops.atma_hip.gated_delta_bwd16(q, k, v, g, beta, S0, dO, dS, ctx.scale,
                                                                      ctx.l2norm)
        return dq, dk, dv, dg, db, (ds0 if S0 is not None else None), None, None


def _chunk_gated_delta_train(q, k, v, g, beta, scale, initial_state, output_final_state, use_qk_l2norm):
    """Differentiable ``chunk_gated_delta_rule`` (the FLA autograd the reference trains
    through, ``model/blocks.py:44-84``).  Grouped KV heads are expanded by a torch op
    (autograd sums their gradients).  16-bit inputs with dk = dv in {64, 128}: the raw rows
    go to the 16-bit chunked forward and the chunked (WY) backward, which apply the l2 norm
    and scale (and their backward) in-kernel, 16-bit products with fp32 accumulation as
    FLA's kernels.  Other inputs: the l2 norm and scale as torch ops, then the recurrence
    and its sequential backward in fp32.  o is returned in q's dtype."""
    B, T, H, dk = q.shape
    if k.shape[2] != H:
        rep = H // k.shape[2]
        k, v = k.repeat_interleave(rep, dim=2), v.repeat_interleave(rep, dim=2)
    S0 = None if initial_state is None else initial_state.float().contiguous()
    if q.dtype in (torch.bfloat16, torch.float16) and dk == v.shape[3] and dk in (64, 128):
        o, S = _GatedDelta16Fn.apply(q.contiguous(), k.contiguous(), v.contiguous(), g.float().contiguous(),
                                     beta.float().contiguous(), S0, float(dk ** -0.5 if scale is None else scale),
                                     bool(use_qk_l2norm))
        return o, (S if output_final_state else None)
    qf, kf = q.float(), k.float()
    if use_qk_l2norm:
        qf = torch.nn.functional.normalize(qf, dim=-1, eps=1e-12)
        kf = torch.nn.functional.normalize(kf, dim=-1, eps=1e-12)
    qs = qf * (dk ** -0.5 if scale is None else float(scale))
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

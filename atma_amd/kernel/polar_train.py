"""Autograd-aware Polar attention for training: ``polar_attention``
(``kernel/polar_triton.py:1158-1219``), backed by the HIP forward (with its saved
statistics) and the HIP backward loops (``atma_hip::polar_attention_bwd``).

The backward follows ``_polar_backward`` (``kernel/polar_triton.py:1033-1155``): a
per-query preamble (one HIP kernel, O(B*H*T*d)) turns the output cotangents into the
score-space cotangents (gs, gL, gQ2) and the null-sink / parameter partial sums, two HIP
kernels run the O(T^2) loops, and the parameter gradients are assembled from the sums.
The saved reference max M of the 16-bit forward may sit below the true running max; L,
Q2 and s are relative to the same M, so every formula holds for any such M (the outputs
are invariant to it).
"""

import torch

from .. import _ops  # noqa: F401  (registers torch.ops.atma_hip.*)
from .polar import _params, _window_arg


class PolarAttentionHip(torch.autograd.Function):
    """Forward: the HIP kernel with saved statistics.  Backward: preamble + HIP loops."""

    @staticmethod
    def forward(ctx, q, k, v, n_keys, v_null, null_base, null_slope_raw, len_gain_raw,
                mag_beta_raw, eps, is_causal, window, preserve_length):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        p = _params(q.device, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw)
        nk = n_keys.to(device=q.device, dtype=torch.float32).reshape(-1).contiguous()
        c, mag, M, L, Q2, S = torch.ops.atma_hip.polar_attention_fwd_train(
            q, k, v, nk, *p, float(eps), bool(is_causal), _window_arg(window), bool(preserve_length))
        ctx.save_for_backward(q, k, v, nk, *p, M, L, Q2, S)
        ctx.eps, ctx.is_causal, ctx.window, ctx.preserve_length = eps, is_causal, window, preserve_length
        ctx.param_dtypes = tuple(t.dtype for t in (v_null, null_base, null_slope_raw, len_gain_raw,
                                                   mag_beta_raw))
        return c, mag

    @staticmethod
    def backward(ctx, gc, gm):
        q, k, v, nk, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw, M, L, Q2, S = \
            ctx.saved_tensors
        B, H, Tq, d = q.shape
        win = _window_arg(ctx.window)
        # per-query preamble + parameter partial sums (one HIP kernel)
        gs, gL, gQ2, temp, part = torch.ops.atma_hip.polar_attention_bwd_prep(
            gc, gm, S, M, L, Q2, nk, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw,
            float(ctx.eps), win, bool(ctx.preserve_length), q.dtype)
        # the O(T^2) loops
        dq, dt, dkv = torch.ops.atma_hip.polar_attention_bwd(
            q, k, v, gs, gL, gQ2, M, temp, nk, bool(ctx.is_causal), win)
        dk, dv = dkv[0], dkv[1]
        # parameters (one HIP launch): temp = 1 + softplus(lg) log n,
        # nu = nb + softplus(ns) sqrt(log(n + 1)), mag = tanh(softplus(mb) log1p(m_eff));
        # d softplus = sigmoid.  The real keys' share of dL/dtemp is dt; the preamble summed
        # the sink's share and the rest per block.
        grad_v_null, g4 = torch.ops.atma_hip.polar_bwd_param_grads(
            part, dt, nk, len_gain_raw, null_slope_raw, mag_beta_raw, win, bool(ctx.preserve_length))
        grad_null_base, grad_null_slope, grad_len_gain, grad_mag_beta = g4[0], g4[1], g4[2], g4[3]

        pd = ctx.param_dtypes
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None,
                grad_v_null.to(pd[0]), grad_null_base.to(pd[1]), grad_null_slope.to(pd[2]),
                grad_len_gain.to(pd[3]), grad_mag_beta.to(pd[4]), None, None, None, None)


def polar_attention(q, k, v, n_keys, *, v_null, null_base, null_slope_raw, len_gain_raw,
                    mag_beta_raw, eps=1e-6, is_causal=True, input_precision="ieee", window=None,
                    preserve_length=False):
    """Autograd-aware Polar attention, the signature of ``polar_attention``
    (``kernel/polar_triton.py:1203-1219``).  q: (B, Hq, T, d); k, v: (B, Hkv, T, d) with
    Hq % Hkv == 0 (the reference's expanded form, or grouped heads whose gradients are
    summed in-kernel); n_keys: (Tq,).  ``window`` is the trainable causal band (the
    backward masks the same band); ``preserve_length`` keeps temp / null on the raw count.
    ``input_precision`` is accepted for signature compatibility (fp32 inputs always use
    full-fp32 MFMA products).  Returns (c (B, Hq, T, d), mag (B, Hq, T)) in q's dtype."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or k.shape != v.shape or k.shape[0] != q.shape[0] \
            or k.shape[3] != q.shape[3] or q.shape[1] % k.shape[1]:
        raise ValueError("q: (B, Hq, T, d) and k, v: (B, Hkv, T, d) with Hq % Hkv == 0 required")
    B, H, Tq, dk = q.shape
    if is_causal and Tq != k.shape[2]:
        raise ValueError(f"is_causal=True requires Tq == Tk; got Tq={Tq}, Tk={k.shape[2]}")
    if dk & (dk - 1):
        raise ValueError(f"head_dim (dk={dk}) must be a power of two.")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share a dtype")
    if input_precision not in ("ieee", "tf32", "tf32x3"):
        raise ValueError(f"unknown input_precision {input_precision!r}")
    return PolarAttentionHip.apply(q, k, v, n_keys, v_null, null_base, null_slope_raw, len_gain_raw,
                                   mag_beta_raw, eps, is_causal, window, preserve_length)


def polar_bwd_flops(B, Hq, T, d):
    """Matmul FLOPs the backward executes for a causal T x T problem: the dq loop
    recomputes S and forms dP and dQ, the dk / dv loop recomputes S and dP and forms
    dV and dK -- 7 products of 2 d FLOP per causal (query, key) pair."""
    return B * Hq * 7 * d * T * (T + 1)


__all__ = ["polar_attention", "PolarAttentionHip", "polar_bwd_flops"]

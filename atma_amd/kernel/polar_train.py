"""Autograd-aware Polar attention for training: ``polar_attention``
(``kernel/polar_triton.py:1158-1219``), backed by the HIP forward (with its saved
statistics) and the HIP backward loops (``atma_hip::polar_attention_bwd``).

The backward follows ``_polar_backward`` (``kernel/polar_triton.py:1033-1155``): a
per-query preamble turns the output cotangents into the score-space cotangents
(gs, gL, gQ2) and the null-sink / parameter terms (O(B*H*T*d), here in PyTorch), the
kernels run the two O(T^2) loops, and the parameter gradients are assembled from their
per-query sums.  The saved reference max M of the 16-bit forward may sit below the true
running max; L, Q2 and s are relative to the same M, so every formula below holds for
any such M (the outputs are invariant to it).
"""

import torch
import torch.nn.functional as F

from .. import _ops  # noqa: F401  (registers torch.ops.atma_hip.*)
from .polar import _params, _window_arg

_TINY = 1.0e-30   # the Q2 / Z floors of the forward (kernel/polar_triton.py:175-177)


def _calibration(n_keys, H, len_gain_raw, null_base, null_slope_raw, window, preserve_length):
    """temp (H, Tq), nu (H, Tq), log n (Tq,), sqrt(log(n + 1)) (Tq,) from the counts the
    forward's temp / null see (windowed unless preserve_length, clamped at 1)."""
    n = n_keys.float()
    if window is not None and not preserve_length:
        n = torch.minimum(n, torch.full_like(n, float(window)))
    n = n.clamp(min=1.0)
    logn = torch.log(n)
    root = torch.sqrt(torch.log(n + 1.0))
    temp = 1.0 + F.softplus(len_gain_raw.float()).view(H, 1) * logn.view(1, -1)
    nu = null_base.float().view(H, 1) + F.softplus(null_slope_raw.float()).view(H, 1) * root.view(1, -1)
    return temp, nu, logn, root


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
        eps = ctx.eps
        gc = gc.float() if gc is not None else torch.zeros(q.shape, device=q.device)
        gm = gm.float() if gm is not None else torch.zeros((B, H, Tq), device=q.device)
        temp, nu, logn, root = _calibration(nk, H, len_gain_raw, null_base, null_slope_raw,
                                            ctx.window, ctx.preserve_length)
        beta = F.softplus(mag_beta_raw.float()).view(1, H, 1)

        # the sink and the magnitude, recomputed from the saved statistics
        a_null = (temp * nu).unsqueeze(0)                   # (1, H, Tq)
        p_null = torch.exp(a_null - M)                      # (B, H, Tq)
        Z = L + p_null
        Zc, Q2c = Z.clamp_min(_TINY), Q2.clamp_min(_TINY)
        m_eff = (L * L / Q2c) * (L / Zc)                    # = L^3 / (Q2 Z)
        lm = torch.log1p(m_eff)
        mag = torch.tanh(beta * lm)

        # magnitude path: d mag / d m_eff, then m_eff's partials in L, Q2 and Z (= L + p_null)
        g_me = gm * beta * (1.0 - mag * mag) / (1.0 + m_eff)
        dme_dL = torch.where(L > 0, 3.0 * m_eff / L.clamp_min(_TINY), torch.zeros_like(L))
        dme_dQ2 = torch.where(Q2 > _TINY, -m_eff / Q2c, torch.zeros_like(Q2))
        dme_dZ = torch.where(Z > _TINY, -m_eff / Zc, torch.zeros_like(Z))
        gL = g_me * (dme_dL + dme_dZ)
        gQ2 = g_me * dme_dQ2

        # direction path: c = s / max(|s|, eps) -> gs = (gc - (gc.c) c) / max(|s|, eps)
        snorm = S.norm(dim=-1, keepdim=True).clamp_min(eps)
        cdir = S / snorm
        gs = (gc - (gc * cdir).sum(-1, keepdim=True) * cdir) / snorm
        # the sink enters s through p_null * v_null and Z through p_null
        g_pnull = (gs * v_null.float().view(1, H, 1, d)).sum(-1) + g_me * dme_dZ
        grad_v_null = (p_null.unsqueeze(-1) * gs).sum(dim=(0, 2))
        g_anull = g_pnull * p_null                          # d p_null / d a_null = p_null

        dq, dt, dk, dv = torch.ops.atma_hip.polar_attention_bwd(
            q, k, v, gs.to(q.dtype), gL, gQ2, M, temp.contiguous(), nk, bool(ctx.is_causal),
            _window_arg(ctx.window))

        # parameters: temp = 1 + softplus(lg) log n, nu = nb + softplus(ns) sqrt(log(n + 1)),
        # mag = tanh(softplus(mb) log1p(m_eff)); d softplus = sigmoid
        g_temp = dt + g_anull * nu                          # real keys + the sink's logit
        g_nu = g_anull * temp
        grad_len_gain = (g_temp * logn).sum(dim=(0, 2)) * torch.sigmoid(len_gain_raw.float())
        grad_null_base = g_nu.sum(dim=(0, 2))
        grad_null_slope = (g_nu * root).sum(dim=(0, 2)) * torch.sigmoid(null_slope_raw.float())
        grad_mag_beta = (gm * (1.0 - mag * mag) * lm).sum(dim=(0, 2)) * torch.sigmoid(mag_beta_raw.float())

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

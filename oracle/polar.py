"""CPU oracle for Polar attention (test infrastructure only; see ``oracle/__init__``).

Polar attention mixes a query's causal keys with ONE temperature-sharpened softmax
that also carries a single "null sink" logit.  It returns a unit direction ``c``
and a bounded magnitude ``mag`` in [0, 1).  Per query i with ``n_i`` valid keys
(reference docstring ``kernel/polar_triton.py:10-21``)::

    sigma_ij = q_i.k_j / sqrt(d)                        (j < n_i, others masked)
    temp_i   = 1 + softplus(len_gain_raw) * ln(max(n_i,1))
    null_i   = null_base + softplus(null_slope_raw) * sqrt(ln(max(n_i,1) + 1))
    w        = softmax([temp_i*sigma_i*, temp_i*null_i])
    s_i      = sum_j w_ij v_j + w_iN v_null,   c_i = s_i / max(|s_i|, eps)
    n_eff    = 1 / sum_j (w_ij / sum_j w_ij)^2        (participation ratio)
    m_eff    = n_eff * (1 - w_iN)
    mag_i    = tanh(softplus(mag_beta_raw) * log1p(m_eff))

Three CPU forms are given: the materialised reduction (``polar_reduce``), the
streaming form the GPU kernels follow (``polar_online``), and the paged decode
(``polar_decode_paged``), plus a row-sampled exact checker for very long T.
"""

import math

import torch
import torch.nn.functional as F

_PARAM_NAMES = ("v_null", "null_base", "null_slope_raw", "len_gain_raw", "mag_beta_raw")


def _work_dtype(dtype):
    """Half types are reduced in fp32; fp32/fp64 keep their precision
    (``model/blocks.py:167-168``)."""
    return torch.float32 if dtype in (torch.float16, torch.bfloat16) else dtype


def _expand_kv(x, hq):
    """GQA: repeat each KV head for its ``hq // hkv`` query heads, as the callers do
    before the kernel (``inference/models/atma.py:416-420``, ``model/reference.py:155-157``)."""
    hkv = x.shape[1]
    if hkv == hq:
        return x
    if hq % hkv:
        raise ValueError(f"query heads {hq} not a multiple of kv heads {hkv}")
    return x.repeat_interleave(hq // hkv, dim=1)


def polar_temp_null(n_keys, len_gain_raw, null_base, null_slope_raw):
    """Per-(head, query) temperature and null logit.  ``model/blocks.py:104-117``.

    n_keys (Tq,) is the valid-key count (the caller has already applied any window
    cap); the clamp to >= 1 applies to these two quantities only.
    Returns temp, null shaped (H, Tq)."""
    n = n_keys.clamp(min=1.0)
    log_n = torch.log(n)[None, :]
    temp = 1.0 + F.softplus(len_gain_raw)[:, None] * log_n
    null = null_base[:, None] + F.softplus(null_slope_raw)[:, None] * torch.sqrt(torch.log(n + 1.0))[None, :]
    return temp, null


def polar_reduce(sigma, v, n_keys, *, v_null, null_base, null_slope_raw, len_gain_raw,
                 mag_beta_raw, eps=1e-6):
    """Materialised Polar reduction.  ``model/blocks.py:120-164``.

    sigma: (B, H, Tq, Tk) raw scores with -inf at masked keys; v: (B, H, Tk, d)
    (KV heads expanded); n_keys: (Tq,) count used for temp/null.
    Returns c (B, H, Tq, d) and mag (B, H, Tq) in v's dtype."""
    out_dtype = v.dtype
    wd = _work_dtype(out_dtype)
    sigma, v = sigma.to(wd), v.to(wd)
    H, d = v.shape[1], v.shape[-1]
    temp, null = polar_temp_null(n_keys.to(wd), len_gain_raw.to(wd), null_base.to(wd),
                                 null_slope_raw.to(wd))
    temp4 = temp[None, :, :, None]
    dead = torch.isneginf(sigma)
    # scale the finite scores only, so masked entries stay exactly -inf
    real = torch.where(dead, torch.full_like(sigma, float("-inf")),
                       torch.where(dead, torch.zeros_like(sigma), sigma) * temp4)
    sink = (null * temp)[None, :, :, None].expand(sigma.shape[0], H, sigma.shape[2], 1)
    w = torch.softmax(torch.cat([real, sink], dim=-1), dim=-1)
    w_real, w_sink = w[..., :-1], w[..., -1]

    s = w_real @ v + w_sink[..., None] * v_null.to(wd).view(1, H, 1, d)
    c = s / s.norm(dim=-1, keepdim=True).clamp_min(eps)

    mass = w_real.sum(-1, keepdim=True).clamp_min(eps)
    n_eff = 1.0 / (w_real / mass).square().sum(-1).clamp_min(eps)
    m_eff = n_eff * (1.0 - w_sink)
    mag = torch.tanh(F.softplus(mag_beta_raw.to(wd)).view(1, H, 1) * torch.log1p(m_eff))
    return c.to(out_dtype), mag.to(out_dtype)


def _valid_mask(n_keys, Tk, window, device):
    """(Tq, Tk) bool: key j visible to query i iff j < n_i (and, with a window,
    j >= n_i - W).  ``kernel/polar_triton.py:129-133``."""
    j = torch.arange(Tk, device=device)[None, :]
    n = n_keys[:, None]
    ok = j < n
    if window is not None:
        ok = ok & (j >= n - window)
    return ok


def _count_for_calibration(n_keys, window):
    """temp/null see min(n, W) under a window (``kernel/polar_triton.py:85-96``)."""
    if window is None:
        return n_keys
    return torch.minimum(n_keys, torch.full_like(n_keys, float(window)))


def polar_dense(q, k, v, n_keys, *, params, eps=1e-6, window=None, preserve_length=False):
    """Materialised Polar attention for (B,Hq,Tq,d) q against (B,Hkv,Tk,d) k/v with
    an arbitrary per-query valid count ``n_keys`` (Tq,).  This is the CPU route of
    ``AtmaAttention._polar`` (``inference/models/atma.py:236-244``) -> ``polar_reduce``.
    ``preserve_length`` keeps temp/null on the raw count under a window
    (``kernel/polar_triton.py:1049-1053``).  Differentiable (autograd), which the
    backward tests use in fp64."""
    B, H, Tq, d = q.shape
    wd = _work_dtype(q.dtype)
    kx, vx = _expand_kv(k, H), _expand_kv(v, H)
    Tk = kx.shape[2]
    sigma = (q.to(wd) @ kx.to(wd).transpose(-1, -2)) / math.sqrt(d)
    ok = _valid_mask(n_keys.to(q.device), Tk, window, q.device)
    sigma = sigma.masked_fill(~ok[None, None], float("-inf"))
    cal = _count_for_calibration(n_keys, None if preserve_length else window)
    return polar_reduce(sigma, vx.to(q.dtype), cal, eps=eps, **{n: params[n] for n in _PARAM_NAMES})


def polar_online(q, k, v, n_keys, *, params, k_block=512, eps=1e-6, window=None,
                 q2_floor=1e-30, return_stats=False, preserve_length=False):
    """Streaming Polar forward: the formulation every GPU kernel implements.

    Follows ``model/blocks.py:181-250`` (running max M, L = sum p, Q2 = sum p^2
    rescaled by alpha^2, S = sum p v; the null sink folded once at the end), with the
    kernel's clamps (``kernel/polar_triton.py:151-178``): ``Q2`` floored at ``q2_floor``
    (1e-30, not eps) and ``mag`` through ``log1p``.  Masked logits use the finite
    sentinel -1e38 and contribute p = 0.

    q: (B,Hq,Tq,d); k,v: (B,Hkv,Tk,d) (GQA expanded here); n_keys: (Tq,).
    ``preserve_length`` keeps temp/null on the raw count under a window.  Differentiable
    (autograd): this streaming form is the oracle the backward is checked against, as the
    reference checks its backward against ``model/blocks.py:polar_attention_online``.
    Returns c, mag in q's dtype (and, with ``return_stats``, fp M, L, Q2, s)."""
    B, H, Tq, d = q.shape
    wd = _work_dtype(q.dtype)
    qd = q.to(wd)
    kx, vx = _expand_kv(k, H).to(wd), _expand_kv(v, H).to(wd)
    Tk = kx.shape[2]
    n_keys = n_keys.to(device=q.device, dtype=wd)
    temp, null = polar_temp_null(_count_for_calibration(n_keys, None if preserve_length else window),
                                 params["len_gain_raw"].to(wd), params["null_base"].to(wd),
                                 params["null_slope_raw"].to(wd))
    sentinel = -1e38
    M = torch.full((B, H, Tq), sentinel, dtype=wd)
    L = torch.zeros((B, H, Tq), dtype=wd)
    Q2 = torch.zeros((B, H, Tq), dtype=wd)
    S = torch.zeros((B, H, Tq, d), dtype=wd)
    scale = 1.0 / math.sqrt(d)
    for k0 in range(0, Tk, k_block):
        k1 = min(k0 + k_block, Tk)
        a = (qd @ kx[:, :, k0:k1].transpose(-1, -2)) * scale * temp[None, :, :, None]
        ok = _valid_mask(n_keys, Tk, window, q.device)[:, k0:k1][None, None]
        a = torch.where(ok, a, torch.full_like(a, sentinel))
        M_new = torch.maximum(M, a.amax(-1))
        alpha = torch.exp(M - M_new)
        p = torch.where(ok, torch.exp(a - M_new[..., None]), torch.zeros_like(a))
        L = L * alpha + p.sum(-1)
        Q2 = Q2 * alpha * alpha + (p * p).sum(-1)
        S = S * alpha[..., None] + p @ vx[:, :, k0:k1]
        M = M_new
    # fold the null sink once
    a_n = (temp * null)[None].expand(B, H, Tq)
    M_new = torch.maximum(M, a_n)
    alpha = torch.exp(M - M_new)
    L, Q2, S, M = L * alpha, Q2 * alpha * alpha, S * alpha[..., None], M_new
    p_n = torch.exp(a_n - M)
    Z = L + p_n
    s = S + p_n[..., None] * params["v_null"].to(wd).view(1, H, 1, d)
    c = s / s.norm(dim=-1, keepdim=True).clamp_min(eps)
    n_eff = L * L / Q2.clamp_min(q2_floor)
    m_eff = n_eff * (L / Z.clamp_min(eps))
    beta = F.softplus(params["mag_beta_raw"].to(wd)).view(1, H, 1)
    mag = torch.tanh(beta * torch.log1p(m_eff))
    if return_stats:
        return c.to(q.dtype), mag.to(q.dtype), (M, L, Q2, s)
    return c.to(q.dtype), mag.to(q.dtype)


def polar_rows(q, k, v, n_keys, rows, *, params, eps=1e-6, window=None, k_block=4096):
    """Exact Polar output for a subset of query rows (long-T checker).

    Row i only sees keys j < n_i, so each sampled row costs O(n_i d) and T = 262,144
    is checkable without a T^2 tensor.  Same math as ``polar_online``.
    rows: 1-D LongTensor of query indices.  Returns c (B,H,len(rows),d), mag (B,H,len(rows))."""
    rows = torch.as_tensor(rows, dtype=torch.long)
    nk = n_keys[rows]
    hi = int(nk.max().item()) if rows.numel() else 0
    hi = max(hi, 1)
    return polar_online(q[:, :, rows], k[:, :, :hi], v[:, :, :hi], nk, params=params,
                        k_block=k_block, eps=eps, window=window)


def gather_paged_kv(cache, block_tables, context_lens):
    """Logical (B, max_ctx, Hkv, d) view of a paged cache by explicit index math:
    position p of sequence b lives in page ``block_tables[b, p // page]`` at row
    ``p % page`` (``kernel/polar_triton.py:747-756``).  Positions >= context_len are
    never read (they are zero-filled)."""
    page = cache.shape[1]
    B = block_tables.shape[0]
    ctx = [int(x) for x in context_lens.tolist()]
    width = max(ctx) if ctx else 0
    out = torch.zeros((B, width) + tuple(cache.shape[2:]), dtype=cache.dtype)
    for b, n in enumerate(ctx):
        pos = torch.arange(n)
        phys = block_tables[b].long()[pos // page]
        out[b, :n] = cache[phys, pos % page]
    return out


def polar_decode_paged(q, k_cache, v_cache, block_tables, context_lens, *, params, eps=1e-6,
                       window=None, q2_floor=1e-30):
    """Paged decode oracle: one query per sequence against its cached context.

    The CPU route of the reference decode (``inference/models/atma.py:586-612``)
    gathers each sequence's pages and reduces densely with ``n_keys = ctx`` (under a
    window: the last ``min(ctx, W)`` keys, with that count for temp/null).  Here the
    per-sequence reduction is ``polar_online`` with one key block, which is the
    formulation the decode kernel implements (``kernel/polar_triton.py:682-792``).

    q: (B, Hq, d); caches: (pages, page_size, Hkv, d); block_tables (B, max_pages)
    int; context_lens (B,) int.  Returns c (B, Hq, d), mag (B, Hq) in q's dtype."""
    B, H, d = q.shape
    kg = gather_paged_kv(k_cache, block_tables, context_lens)
    vg = gather_paged_kv(v_cache, block_tables, context_lens)
    cs, ms = [], []
    for b in range(B):
        n = int(context_lens[b])
        lo = 0 if window is None else max(0, n - window)
        kb = kg[b, lo:n].permute(1, 0, 2)[None]            # (1, Hkv, n-lo, d)
        vb = vg[b, lo:n].permute(1, 0, 2)[None]
        nk = torch.tensor([float(n - lo)], dtype=torch.float64 if q.dtype == torch.float64 else torch.float32)
        c, m = polar_online(q[b][None, :, None], kb, vb, nk, params=params,
                            k_block=max(n - lo, 1), eps=eps, q2_floor=q2_floor)
        cs.append(c[0, :, 0])
        ms.append(m[0, :, 0])
    return torch.stack(cs), torch.stack(ms)


def prefill_flops(B, Hq, T, d):
    """Algorithmic Polar prefill FLOPs: 4d per causal (query, key) pair, i.e.
    ``B*Hq*2*d*T*(T+1)`` (the per-token term of ``scripts/roofline_inference.py:49``)."""
    return float(B) * Hq * 2 * d * T * (T + 1)

"""Polar attention ops with the reference's ``kernel/polar_triton.py`` signatures,
backed by the HIP kernels of libatma_hip.so (``atma_hip::polar_attention_*``).

Polar attention (reference docstring ``kernel/polar_triton.py:10-21``): one
temperature-sharpened softmax over the causal keys plus a null-sink logit gives a
unit direction ``c`` and a bounded magnitude ``mag``.
"""

import torch

from .. import _lib, _ops  # noqa: F401  (_ops registers torch.ops.atma_hip.*)


def _params(device, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw):
    f = lambda t: t.detach().to(device=device, dtype=torch.float32).contiguous()  # noqa: E731
    return (f(v_null), f(null_base), f(null_slope_raw), f(len_gain_raw), f(mag_beta_raw))


def _window_arg(window):
    if window is None:
        return 0
    w = int(window)
    if w <= 0:
        raise ValueError(f"window must be a positive int or None (got {window})")
    return w


@torch.no_grad()
def polar_attention_fwd(q, k, v, n_keys, *, v_null, null_base, null_slope_raw, len_gain_raw,
                        mag_beta_raw, eps=1e-6, is_causal=True, input_precision="ieee",
                        window=None):
    """Forward-only Polar attention.  Mirrors ``polar_attention_fwd``
    (``kernel/polar_triton.py:594-609``, launch checks ``:505-530``).

    q: (B, Hq, Tq, d).  k, v: (B, Hkv, Tk, d) with Hq % Hkv == 0 -- the reference's
    expanded form (Hkv == Hq) or the unexpanded GQA form (resolved in-kernel).
    n_keys: (Tq,) valid key count per query.  ``is_causal`` requires Tq == Tk.
    ``input_precision`` is accepted for signature compatibility: fp32 inputs always
    use full-fp32 MFMA products.  ``window``: causal sliding window (None = full).
    Returns (c (B, Hq, Tq, d), mag (B, Hq, Tq)) in q's dtype."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be (B, H, T, d)")
    B, Hq, Tq, dk = q.shape
    Tk = k.shape[2]
    if is_causal and Tq != Tk:
        raise ValueError(
            f"is_causal=True requires Tq == Tk (standard causal self-attention); got Tq={Tq}, "
            f"Tk={Tk}. Use is_causal=False with an explicit n_keys for decode / offset-prefill "
            f"layouts.")
    if dk & (dk - 1) != 0:
        raise ValueError(f"head_dim (dk={dk}) must be a power of two.")
    if k.shape != v.shape or k.shape[0] != B or k.shape[3] != dk:
        raise ValueError(f"k/v shape {tuple(k.shape)}/{tuple(v.shape)} incompatible with q {tuple(q.shape)}")
    if Hq % k.shape[1]:
        raise ValueError(f"query heads ({Hq}) must be a multiple of kv heads ({k.shape[1]})")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share a dtype")
    if input_precision not in ("ieee", "tf32", "tf32x3"):
        raise ValueError(f"unknown input_precision {input_precision!r}")
    n_keys = n_keys.to(device=q.device, dtype=torch.float32).reshape(-1).contiguous()
    if n_keys.numel() != Tq:
        raise ValueError(f"n_keys must have Tq={Tq} entries (got {n_keys.numel()})")
    p = _params(q.device, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw)
    c, mag = torch.ops.atma_hip.polar_attention_fwd(q, k, v, n_keys, *p, float(eps), bool(is_causal),
                                                    _window_arg(window))
    return c, mag


@torch.no_grad()
def polar_attention_packed_fwd(q, k, v, tile_seq_starts, tile_q_starts, tile_seq_lens, *, v_null,
                               null_base, null_slope_raw, len_gain_raw, mag_beta_raw, eps=1e-6,
                               input_precision="ieee", window=None):
    """Grouped fresh-prefill Polar attention for packed variable-length requests.
    Mirrors ``polar_attention_packed_fwd`` (``kernel/polar_triton.py:613-669``).

    q: (total_tokens, Hq, d); k, v: (total_tokens, Hkv, d) with Hq % Hkv == 0 -- the
    reference's expanded form (Hkv == Hq) or unexpanded GQA heads.  ``tile_*``: one
    entry per 128-row query tile, (first packed token of the tile's sequence, the tile's
    first query position in it, the sequence length), as the serving context builds
    them (``inference/engine/model_runner.py:390-404``).  Every sequence is a fresh
    causal prompt.  Returns (c (total_tokens, Hq, d), mag (total_tokens, Hq)) in q's dtype."""
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3 or k.shape != v.shape \
            or k.shape[0] != q.shape[0] or k.shape[2] != q.shape[2] or q.shape[1] % k.shape[1]:
        raise ValueError("q, k, and v must have identical [tokens, heads, dim] shapes "
                         "(k, v may carry fewer heads dividing q's)")
    total, heads, dk = q.shape
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("packed Polar route is enabled only for 16-bit inference")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share a dtype")
    if dk & (dk - 1):
        raise ValueError(f"head_dim (dk={dk}) must be a power of two")
    if not (tile_seq_starts.numel() == tile_q_starts.numel() == tile_seq_lens.numel()):
        raise ValueError("packed Polar tile-map tensors must have equal lengths")
    if input_precision not in ("ieee", "tf32", "tf32x3"):
        raise ValueError(f"unknown input_precision {input_precision!r}")
    maps = [t.to(device=q.device, dtype=torch.int32).reshape(-1).contiguous()
            for t in (tile_seq_starts, tile_q_starts, tile_seq_lens)]
    p = _params(q.device, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw)
    c, mag = torch.ops.atma_hip.polar_attention_packed_fwd(q, k, v, *maps, *p, float(eps),
                                                           _window_arg(window))
    return c, mag


@torch.no_grad()
def polar_attention_decode(q, k_cache, v_cache, block_tables, context_lens, *, v_null, null_base,
                           null_slope_raw, len_gain_raw, mag_beta_raw, eps=1e-6, block_n=None,
                           num_warps=None, num_stages=None, window=None):
    """Paged Polar decode.  Mirrors ``polar_attention_decode``
    (``kernel/polar_triton.py:796-858``).

    q: (B, Hq, d) current-token queries (KV heads NOT expanded, GQA in-kernel).
    k_cache, v_cache: (num_pages, page_size, Hkv, d) contiguous.  block_tables:
    (B, max_pages) int32 logical->physical page map.  context_lens: (B,) int32 keys
    per sequence, including the current token.  ``block_n`` / ``num_warps`` /
    ``num_stages`` are Triton tuning knobs, accepted and ignored.
    Returns (c (B, Hq, d), mag (B, Hq)) in q's dtype.  Graph capturable."""
    if q.dim() != 3 or k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("q must be (B, H, d) and k_cache/v_cache (pages, page_size, Hkv, d)")
    if q.shape[2] != k_cache.shape[3] or q.shape[1] % k_cache.shape[2]:
        raise ValueError(f"q {tuple(q.shape)} incompatible with cache {tuple(k_cache.shape)}")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise ValueError("q and the caches must share a dtype")
    if block_tables.dim() != 2 or block_tables.shape[0] != q.shape[0]:
        raise ValueError("block_tables must be (B, max_pages)")
    if block_tables.dtype != torch.int32:
        block_tables = block_tables.to(torch.int32)
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    context_lens = context_lens.to(device=q.device, dtype=torch.int32).contiguous()
    p = _params(q.device, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw)
    c, mag = torch.ops.atma_hip.polar_attention_decode(q, k_cache, v_cache, block_tables,
                                                       context_lens, *p, float(eps),
                                                       _window_arg(window))
    return c, mag


def global_decode_step_supported(q, k_cache, block_tables):
    """True when ``global_decode_step`` runs fused for these shapes: 16-bit caches whose
    pages hold whole 32-key units, head_dim 64 / 128, GQA groups of at most 16."""
    B, Hq, d = q.shape
    return global_decode_step_supported_shape(B, Hq, k_cache.shape[2], block_tables.shape[1], k_cache.shape[1], d,
                                              q.dtype)


def global_decode_step_supported_shape(B, Hq, Hkv, max_pages, page_size, d, dtype):
    """``global_decode_step_supported`` from the sizes alone."""
    return bool(_lib.load().atma_global_decode_step_supported(B, Hq, Hkv, max_pages, page_size, d,
                                                              _lib.dtype_code(dtype)))


def global_decode_step(q, k_new, v_new, k_cache, v_cache, slot_mapping, block_tables, context_lens,
                       gamma, beta, state_table, slots, *, v_null, null_base, null_slope_raw,
                       len_gain_raw, mag_beta_raw, eps=1e-6, mem_eps=1e-12, window=None):
    """The global layer's decode mixer (``inference/models/atma.py:546-618``): the calls
    ``store_kvcache(k_new, v_new, caches, slot_mapping)``, ``polar_attention_decode(q,
    caches, ...)`` and ``gated_delta_decode_step(q, k_new, v_new, gamma, beta, state_table,
    slots)`` in that order, fused into two launches where the shapes allow it (the newest
    key joins the attention from k_new / v_new, the cache row is written after the split
    pass; equal to the three calls when slot_mapping[b] is the slot of position
    context_lens[b] - 1, as the engine builds it), else the three calls.

    q: (B, Hq, d); k_new, v_new: (B, Hkv, d); caches (num_pages, page_size, Hkv, d)
    contiguous, written in place; state_table (max_seqs, Hq, d, d) fp32, advanced in place.
    Returns (c, mag, r)."""
    from .gated_delta import gated_delta_decode_step
    from ..layers.attention import store_kvcache
    if q.dim() != 3 or k_new.dim() != 3 or v_new.shape != k_new.shape or k_cache.dim() != 4 \
            or k_cache.shape != v_cache.shape or k_new.shape[1:] != k_cache.shape[2:]:
        raise ValueError("q (B, Hq, d), k_new / v_new (B, Hkv, d) and caches (pages, page_size, Hkv, d)")
    if q.shape[2] != k_cache.shape[3] or q.shape[1] % k_cache.shape[2]:
        raise ValueError(f"q {tuple(q.shape)} incompatible with cache {tuple(k_cache.shape)}")
    if not global_decode_step_supported(q, k_cache, block_tables) or k_new.dtype != q.dtype \
            or v_new.dtype != q.dtype or k_cache.dtype != q.dtype:
        store_kvcache(k_new, v_new, k_cache, v_cache, slot_mapping)
        c, mag = polar_attention_decode(q, k_cache, v_cache, block_tables, context_lens, v_null=v_null,
                                        null_base=null_base, null_slope_raw=null_slope_raw,
                                        len_gain_raw=len_gain_raw, mag_beta_raw=mag_beta_raw, eps=eps,
                                        window=window)
        r = gated_delta_decode_step(q, k_new, v_new, gamma, beta, state_table, slots, eps=mem_eps)
        return c, mag, r
    B, H, d = q.shape
    if state_table.dim() != 4 or state_table.shape[1:] != (H, d, d):
        raise ValueError(f"state_table {tuple(state_table.shape)} incompatible with q {tuple(q.shape)}")
    if block_tables.dtype != torch.int32 or block_tables.stride(1) != 1:
        block_tables = block_tables.to(torch.int32).contiguous()
    context_lens = context_lens.to(device=q.device, dtype=torch.int32).contiguous()
    slot_mapping = slot_mapping.to(device=q.device, dtype=torch.int32).contiguous()
    gamma = gamma.to(torch.float32).reshape(B, H).contiguous()
    beta = beta.to(torch.float32).reshape(B, H).contiguous()
    slots = slots.to(device=q.device, dtype=torch.int64).reshape(B).contiguous()
    p = _params(q.device, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw)
    c, mag, r = torch.ops.atma_hip.global_decode_step(
        q, k_new, v_new, k_cache, v_cache, slot_mapping, block_tables, context_lens, *p, gamma, beta,
        state_table, slots, float(eps), float(mem_eps), _window_arg(window))
    return c, mag, r

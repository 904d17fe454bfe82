"""torch.library custom ops ``atma_hip::*`` over the C ABI of libatma_hip.so.

Each op launches on torch's current stream of the input's device, allocates its
outputs / workspace through torch's caching allocator (so it is safe under
CUDA-graph capture), and never synchronises the host.  Ops that write into
caller-owned tensors declare them in ``mutates_args``.  There is no CPU
implementation: a CPU tensor raises, and a missing library raises
``HipLibraryMissing``.
"""

from typing import List, Optional

import torch
from torch import Tensor

from . import _lib


def _need_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("atma_hip ops run on the GPU only (got a CPU tensor); "
                               "this build has no CPU fallback")


def _rows16(t: Tensor) -> Tensor:
    """Return t with unit innermost stride and 16-byte aligned rows/base."""
    es = t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()


# --------------------------------------------------------------------------- Polar fwd
@torch.library.custom_op("atma_hip::polar_attention_fwd", mutates_args=())
def polar_attention_fwd_op(q: Tensor, k: Tensor, v: Tensor, n_keys: Tensor, v_null: Tensor,
                           null_base: Tensor, null_slope_raw: Tensor, len_gain_raw: Tensor,
                           mag_beta_raw: Tensor, eps: float, is_causal: bool,
                           window: int) -> List[Tensor]:
    _need_cuda(q, k, v, n_keys, v_null)
    lib = _lib.load()
    q, k, v = _rows16(q), _rows16(k), _rows16(v)
    B, Hq, Tq, d = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    c = torch.empty((B, Hq, Tq, d), device=q.device, dtype=q.dtype)
    mag = torch.empty((B, Hq, Tq), device=q.device, dtype=q.dtype)
    rc = lib.atma_polar_attention_fwd(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        n_keys.data_ptr(), v_null.data_ptr(), null_base.data_ptr(), null_slope_raw.data_ptr(),
        len_gain_raw.data_ptr(), mag_beta_raw.data_ptr(), c.data_ptr(), mag.data_ptr(),
        None, None, None, None, B, Hq, Hkv, Tq, Tk, d, _lib.dtype_code(q.dtype),
        1 if is_causal else 0, window, 0, eps, _lib.stream_handle(q.device))
    _lib.check(rc, "polar_attention_fwd")
    return [c, mag]


@polar_attention_fwd_op.register_fake
def _(q, k, v, n_keys, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw, eps,
      is_causal, window):
    B, Hq, Tq, d = q.shape
    return [q.new_empty((B, Hq, Tq, d)), q.new_empty((B, Hq, Tq))]


# --------------------------------------------------------------------------- Polar training pair
@torch.library.custom_op("atma_hip::polar_attention_fwd_train", mutates_args=())
def polar_attention_fwd_train_op(q: Tensor, k: Tensor, v: Tensor, n_keys: Tensor, v_null: Tensor,
                                 null_base: Tensor, null_slope_raw: Tensor, len_gain_raw: Tensor,
                                 mag_beta_raw: Tensor, eps: float, is_causal: bool, window: int,
                                 preserve_length: bool) -> List[Tensor]:
    """Forward that also returns the saved statistics (M, L, Q2, s) of the backward."""
    _need_cuda(q, k, v, n_keys, v_null)
    lib = _lib.load()
    q, k, v = _rows16(q), _rows16(k), _rows16(v)
    B, Hq, Tq, d = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    c = torch.empty((B, Hq, Tq, d), device=q.device, dtype=q.dtype)
    mag = torch.empty((B, Hq, Tq), device=q.device, dtype=q.dtype)
    M, L, Q2 = (torch.empty((B, Hq, Tq), device=q.device, dtype=torch.float32) for _ in range(3))
    S = torch.empty((B, Hq, Tq, d), device=q.device, dtype=torch.float32)
    rc = lib.atma_polar_attention_fwd(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        n_keys.data_ptr(), v_null.data_ptr(), null_base.data_ptr(), null_slope_raw.data_ptr(),
        len_gain_raw.data_ptr(), mag_beta_raw.data_ptr(), c.data_ptr(), mag.data_ptr(),
        M.data_ptr(), L.data_ptr(), Q2.data_ptr(), S.data_ptr(), B, Hq, Hkv, Tq, Tk, d,
        _lib.dtype_code(q.dtype), 1 if is_causal else 0, window, 1 if preserve_length else 0, eps,
        _lib.stream_handle(q.device))
    _lib.check(rc, "polar_attention_fwd")
    return [c, mag, M, L, Q2, S]


@polar_attention_fwd_train_op.register_fake
def _(q, k, v, n_keys, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw, eps,
      is_causal, window, preserve_length):
    B, Hq, Tq, d = q.shape
    f = dict(dtype=torch.float32)
    return [q.new_empty((B, Hq, Tq, d)), q.new_empty((B, Hq, Tq)), q.new_empty((B, Hq, Tq), **f),
            q.new_empty((B, Hq, Tq), **f), q.new_empty((B, Hq, Tq), **f), q.new_empty((B, Hq, Tq, d), **f)]


@torch.library.custom_op("atma_hip::polar_attention_bwd_prep", mutates_args=())
def polar_attention_bwd_prep_op(gc: Optional[Tensor], gm: Optional[Tensor], S: Tensor, M: Tensor,
                                L: Tensor, Q2: Tensor, n_keys: Tensor, v_null: Tensor,
                                null_base: Tensor, null_slope_raw: Tensor, len_gain_raw: Tensor,
                                mag_beta_raw: Tensor, eps: float, window: int, preserve_length: bool,
                                dtype: torch.dtype) -> List[Tensor]:
    """The backward's per-query preamble: returns gs (dtype), gL, gQ2, temp (H, T) and the
    per-block parameter partial sums (B * ceil(T / 16), H, d + 4), all fp32 but gs."""
    _need_cuda(S, M, L, Q2, n_keys, v_null)
    lib = _lib.load()
    B, H, T, d = S.shape
    f = dict(device=S.device, dtype=torch.float32)
    gc = None if gc is None else _rows16(gc.to(dtype).contiguous())
    gm = None if gm is None else gm.to(dtype).contiguous()
    S, v_null = _rows16(S.contiguous()), _rows16(v_null.contiguous())
    gs = torch.empty((B, H, T, d), device=S.device, dtype=dtype)
    gL = torch.empty((B, H, T), **f)
    gQ2 = torch.empty((B, H, T), **f)
    temp = torch.empty((H, T), **f)
    part = torch.empty((B * ((T + 15) // 16), H, d + 4), **f)
    rc = lib.atma_polar_attention_bwd_prep(
        _lib.ptr(gc), _lib.ptr(gm), S.data_ptr(), M.data_ptr(), L.data_ptr(), Q2.data_ptr(),
        n_keys.data_ptr(), v_null.data_ptr(), null_base.data_ptr(), null_slope_raw.data_ptr(),
        len_gain_raw.data_ptr(), mag_beta_raw.data_ptr(), gs.data_ptr(), gL.data_ptr(), gQ2.data_ptr(),
        temp.data_ptr(), part.data_ptr(), B, H, T, d, _lib.dtype_code(dtype), window,
        1 if preserve_length else 0, eps, _lib.stream_handle(S.device))
    _lib.check(rc, "polar_attention_bwd_prep")
    return [gs, gL, gQ2, temp, part]


@polar_attention_bwd_prep_op.register_fake
def _(gc, gm, S, M, L, Q2, n_keys, v_null, null_base, null_slope_raw, len_gain_raw, mag_beta_raw, eps,
      window, preserve_length, dtype):
    B, H, T, d = S.shape
    return [S.new_empty((B, H, T, d), dtype=dtype), S.new_empty((B, H, T)), S.new_empty((B, H, T)),
            S.new_empty((H, T)), S.new_empty((B * ((T + 15) // 16), H, d + 4))]


@torch.library.custom_op("atma_hip::polar_attention_bwd", mutates_args=())
def polar_attention_bwd_op(q: Tensor, k: Tensor, v: Tensor, gs: Tensor, gL: Tensor, gQ2: Tensor,
                           M: Tensor, temp: Tensor, n_keys: Tensor, is_causal: bool,
                           window: int) -> List[Tensor]:
    """The O(T^2) part of the backward: returns dq in q's dtype, dt in fp32 and dkv
    (2, B, Hkv, Tk, d) in q's dtype (dk = dkv[0], dv = dkv[1]: one group-sum launch writes
    both)."""
    _need_cuda(q, k, v, gs, gL, gQ2, M, temp, n_keys)
    lib = _lib.load()
    q, k, v, gs = _rows16(q), _rows16(k), _rows16(v), _rows16(gs)
    B, Hq, Tq, d = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    f = dict(device=q.device, dtype=torch.float32)
    new = torch.empty if Tk > 0 else torch.zeros   # with no keys nothing is written
    dq = new((B, Hq, Tq, d), device=q.device, dtype=q.dtype)
    dt = new((B, Hq, Tq), **f)
    share = torch.bfloat16 if q.dtype == torch.bfloat16 else torch.float32   # fp16: fp32 shares
    dkv = new((2, B, Hq, Tk, d), device=q.device, dtype=share)   # each query head's share; the group sum follows
    dk, dv = dkv[0], dkv[1]   # the kernel's two outputs
    gL, gQ2, M, temp = (t.to(torch.float32).contiguous() for t in (gL, gQ2, M, temp))
    rc = lib.atma_polar_attention_bwd(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        gs.data_ptr(), gs.stride(0), gs.stride(1), gs.stride(2),
        gL.data_ptr(), gQ2.data_ptr(), M.data_ptr(), temp.data_ptr(), n_keys.data_ptr(),
        dq.data_ptr(), dt.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, Hq, Hkv, Tq, Tk, d,
        _lib.dtype_code(q.dtype), 1 if is_causal else 0, window, _lib.stream_handle(q.device))
    _lib.check(rc, "polar_attention_bwd")
    # dk / dv: the group's shares summed (fixed order) into k's dtype
    if Hkv != Hq or q.dtype != torch.float32:   # dk and dv in one launch
        dkv = _group_sum(lib, dkv, 2 * B * Hkv, Tk * d, Hq // Hkv, q.dtype).view(2, B, Hkv, Tk, d)
    return [dq, dt, dkv]


def _group_sum(lib, part, n_groups, elems, G, dtype):
    """out[g0] = sum of part's G consecutive (elems,) slices g0 * G .. g0 * G + G - 1, in dtype."""
    out = torch.empty(n_groups * elems, device=part.device, dtype=dtype)
    rc = lib.atma_polar_bwd_group_sum(part.data_ptr(), _lib.dtype_code(part.dtype), out.data_ptr(), n_groups, G,
                                      elems, _lib.dtype_code(dtype), _lib.stream_handle(part.device))
    _lib.check(rc, "polar_bwd_group_sum")
    return out.view(part.shape) if G == 1 else out


@torch.library.custom_op("atma_hip::polar_bwd_param_grads", mutates_args=())
def polar_bwd_param_grads_op(part: Tensor, dt: Tensor, n_keys: Tensor, len_gain_raw: Tensor,
                             null_slope_raw: Tensor, mag_beta_raw: Tensor, window: int,
                             preserve_length: bool) -> List[Tensor]:
    """The Polar parameters' gradients from the preamble's block sums (B * ceil(T / 16), H,
    d + 4) and dt (B, H, T): returns [g_v_null (H, d), g (4, H) = null_base, null_slope_raw,
    len_gain_raw, mag_beta_raw], fp32."""
    _need_cuda(part, dt, n_keys, len_gain_raw, null_slope_raw, mag_beta_raw)
    lib = _lib.load()
    B, H, T = dt.shape
    d = part.shape[-1] - 4
    if part.dim() != 3 or part.shape[0] != B * ((T + 15) // 16) or part.shape[1] != H:
        raise ValueError("polar_bwd_param_grads: part must be (B * ceil(T / 16), H, d + 4)")
    f = dict(device=dt.device, dtype=torch.float32)
    part, dt, n_keys = part.contiguous(), dt.contiguous(), n_keys.to(torch.float32).contiguous()
    lg, ns, mb = (t.to(torch.float32).contiguous() for t in (len_gain_raw, null_slope_raw, mag_beta_raw))
    gv = torch.empty((H, d), **f)
    g4 = torch.empty((4, H), **f)
    ws_bytes = lib.atma_polar_bwd_param_grads_workspace_bytes(H, d)
    ws = torch.empty((ws_bytes // 4,), **f)
    rc = lib.atma_polar_bwd_param_grads(part.data_ptr(), dt.data_ptr(), n_keys.data_ptr(), lg.data_ptr(),
                                        ns.data_ptr(), mb.data_ptr(), gv.data_ptr(), g4.data_ptr(), B, H, T, d,
                                        window, 1 if preserve_length else 0, ws.data_ptr(), ws_bytes,
                                        _lib.stream_handle(dt.device))
    _lib.check(rc, "polar_bwd_param_grads")
    return [gv, g4]


@polar_bwd_param_grads_op.register_fake
def _(part, dt, n_keys, len_gain_raw, null_slope_raw, mag_beta_raw, window, preserve_length):
    B, H, T = dt.shape
    return [dt.new_empty((H, part.shape[-1] - 4)), dt.new_empty((4, H))]


@polar_attention_bwd_op.register_fake
def _(q, k, v, gs, gL, gQ2, M, temp, n_keys, is_causal, window):
    B, Hq, Tq, d = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    return [q.new_empty((B, Hq, Tq, d)), q.new_empty((B, Hq, Tq), dtype=torch.float32),
            q.new_empty((2, B, Hkv, Tk, d))]


# --------------------------------------------------------------------------- Polar packed fwd
@torch.library.custom_op("atma_hip::polar_attention_packed_fwd", mutates_args=())
def polar_attention_packed_fwd_op(q: Tensor, k: Tensor, v: Tensor, tile_seq_starts: Tensor,
                                  tile_q_starts: Tensor, tile_seq_lens: Tensor, v_null: Tensor,
                                  null_base: Tensor, null_slope_raw: Tensor, len_gain_raw: Tensor,
                                  mag_beta_raw: Tensor, eps: float, window: int) -> List[Tensor]:
    _need_cuda(q, k, v, tile_seq_starts, tile_q_starts, tile_seq_lens, v_null)
    lib = _lib.load()
    q, k, v = _rows16(q), _rows16(k), _rows16(v)
    total, Hq, d = q.shape
    c = torch.empty((total, Hq, d), device=q.device, dtype=q.dtype)
    mag = torch.empty((total, Hq), device=q.device, dtype=q.dtype)
    rc = lib.atma_polar_attention_packed_fwd(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1), tile_seq_starts.data_ptr(), tile_q_starts.data_ptr(),
        tile_seq_lens.data_ptr(), tile_seq_starts.numel(), v_null.data_ptr(), null_base.data_ptr(),
        null_slope_raw.data_ptr(), len_gain_raw.data_ptr(), mag_beta_raw.data_ptr(),
        c.data_ptr(), c.stride(0), c.stride(1), mag.data_ptr(), mag.stride(0), mag.stride(1),
        total, Hq, k.shape[1], d, _lib.dtype_code(q.dtype), window, eps,
        _lib.stream_handle(q.device))
    _lib.check(rc, "polar_attention_packed_fwd")
    return [c, mag]


@polar_attention_packed_fwd_op.register_fake
def _(q, k, v, tile_seq_starts, tile_q_starts, tile_seq_lens, v_null, null_base, null_slope_raw,
      len_gain_raw, mag_beta_raw, eps, window):
    total, Hq, d = q.shape
    return [q.new_empty((total, Hq, d)), q.new_empty((total, Hq))]


# --------------------------------------------------------------------------- Polar decode
@torch.library.custom_op("atma_hip::polar_attention_decode", mutates_args=())
def polar_attention_decode_op(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_tables: Tensor,
                              context_lens: Tensor, v_null: Tensor, null_base: Tensor,
                              null_slope_raw: Tensor, len_gain_raw: Tensor, mag_beta_raw: Tensor,
                              eps: float, window: int) -> List[Tensor]:
    _need_cuda(q, k_cache, v_cache, block_tables, context_lens)
    lib = _lib.load()
    q = _rows16(q)
    if not k_cache.is_contiguous() or not v_cache.is_contiguous():
        raise ValueError("k_cache / v_cache must be contiguous (num_pages, page_size, Hkv, d)")
    B, Hq, d = q.shape
    num_pages, page, Hkv, _ = k_cache.shape
    max_pages = block_tables.shape[1]
    c = torch.empty((B, Hq, d), device=q.device, dtype=q.dtype)
    mag = torch.empty((B, Hq), device=q.device, dtype=q.dtype)
    ws_bytes = lib.atma_polar_decode_workspace_bytes(B, Hq, Hkv, max_pages, page, d, _lib.dtype_code(q.dtype))
    ws = torch.empty((max(ws_bytes, 4) // 4,), device=q.device, dtype=torch.float32)
    rc = lib.atma_polar_attention_decode(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
        num_pages, page, Hkv, block_tables.data_ptr(), block_tables.stride(0), max_pages,
        context_lens.data_ptr(), v_null.data_ptr(), null_base.data_ptr(), null_slope_raw.data_ptr(),
        len_gain_raw.data_ptr(), mag_beta_raw.data_ptr(), c.data_ptr(), mag.data_ptr(), B, Hq, d,
        _lib.dtype_code(q.dtype), window, eps, ws.data_ptr(), ws.numel() * 4,
        _lib.stream_handle(q.device))
    _lib.check(rc, "polar_attention_decode")
    return [c, mag]


@polar_attention_decode_op.register_fake
def _(q, k_cache, v_cache, block_tables, context_lens, v_null, null_base, null_slope_raw,
      len_gain_raw, mag_beta_raw, eps, window):
    B, Hq, d = q.shape
    return [q.new_empty((B, Hq, d)), q.new_empty((B, Hq))]


# --------------------------------------------------------------------------- gated delta step
@torch.library.custom_op("atma_hip::gated_delta_decode_step", mutates_args=("state_table",))
def gated_delta_decode_step_op(q: Tensor, k: Tensor, v: Tensor, gamma: Tensor, beta: Tensor,
                               state_table: Tensor, slots: Tensor, eps: float) -> Tensor:
    _need_cuda(q, k, v, gamma, beta, state_table, slots)
    lib = _lib.load()
    if not state_table.is_contiguous() or state_table.dtype != torch.float32:
        raise ValueError("state_table must be a contiguous float32 (max_seqs, H, dk, dv) tensor")
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    B, H, dk = q.shape
    dv = state_table.shape[3]
    r = torch.empty((B, H, dv), device=q.device, dtype=torch.float32)
    rc = lib.atma_gated_delta_decode_step(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1), gamma.data_ptr(), beta.data_ptr(),
        state_table.data_ptr(), state_table.shape[0], slots.data_ptr(), r.data_ptr(), B, H,
        k.shape[1], dk, dv, _lib.dtype_code(q.dtype), eps, _lib.stream_handle(q.device))
    _lib.check(rc, "gated_delta_decode_step")
    return r


@gated_delta_decode_step_op.register_fake
def _(q, k, v, gamma, beta, state_table, slots, eps):
    B, H, _ = q.shape
    return q.new_empty((B, H, state_table.shape[3]), dtype=torch.float32)


# --------------------------------------------------------------------------- fused decode step
@torch.library.custom_op("atma_hip::global_decode_step",
                         mutates_args=("k_cache", "v_cache", "state_table"))
def global_decode_step_op(q: Tensor, k_new: Tensor, v_new: Tensor, k_cache: Tensor, v_cache: Tensor,
                          slot_mapping: Tensor, block_tables: Tensor, context_lens: Tensor,
                          v_null: Tensor, null_base: Tensor, null_slope_raw: Tensor,
                          len_gain_raw: Tensor, mag_beta_raw: Tensor, gamma: Tensor, beta: Tensor,
                          state_table: Tensor, slots: Tensor, eps: float, mem_eps: float,
                          window: int) -> List[Tensor]:
    _need_cuda(q, k_new, v_new, k_cache, v_cache, slot_mapping, block_tables, context_lens, gamma,
               beta, state_table, slots)
    lib = _lib.load()
    q, k_new, v_new = _rows16(q), _rows16(k_new), _rows16(v_new)
    if not k_cache.is_contiguous() or not v_cache.is_contiguous():
        raise ValueError("k_cache / v_cache must be contiguous (num_pages, page_size, Hkv, d)")
    if not state_table.is_contiguous() or state_table.dtype != torch.float32:
        raise ValueError("state_table must be a contiguous float32 (max_seqs, H, dk, dv) tensor")
    B, Hq, d = q.shape
    num_pages, page, Hkv, _ = k_cache.shape
    max_pages = block_tables.shape[1]
    code = _lib.dtype_code(q.dtype)
    c = torch.empty((B, Hq, d), device=q.device, dtype=q.dtype)
    mag = torch.empty((B, Hq), device=q.device, dtype=q.dtype)
    r = torch.empty((B, Hq, d), device=q.device, dtype=torch.float32)
    ws_bytes = lib.atma_polar_decode_workspace_bytes(B, Hq, Hkv, max_pages, page, d, code)
    ws = torch.empty((max(ws_bytes, 4) // 4,), device=q.device, dtype=torch.float32)
    rc = lib.atma_global_decode_step(
        q.data_ptr(), q.stride(0), q.stride(1), k_new.data_ptr(), k_new.stride(0), k_new.stride(1),
        v_new.data_ptr(), v_new.stride(0), v_new.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
        num_pages, page, Hkv, slot_mapping.data_ptr(), block_tables.data_ptr(), block_tables.stride(0),
        max_pages, context_lens.data_ptr(), v_null.data_ptr(), null_base.data_ptr(),
        null_slope_raw.data_ptr(), len_gain_raw.data_ptr(), mag_beta_raw.data_ptr(), c.data_ptr(),
        mag.data_ptr(), gamma.data_ptr(), beta.data_ptr(), state_table.data_ptr(), state_table.shape[0],
        slots.data_ptr(), r.data_ptr(), B, Hq, d, code, window, eps, mem_eps, ws.data_ptr(),
        ws.numel() * 4, _lib.stream_handle(q.device))
    _lib.check(rc, "global_decode_step")
    return [c, mag, r]


@global_decode_step_op.register_fake
def _(q, k_new, v_new, k_cache, v_cache, slot_mapping, block_tables, context_lens, v_null, null_base,
      null_slope_raw, len_gain_raw, mag_beta_raw, gamma, beta, state_table, slots, eps, mem_eps, window):
    B, Hq, d = q.shape
    return [q.new_empty((B, Hq, d)), q.new_empty((B, Hq)), q.new_empty((B, Hq, d), dtype=torch.float32)]


# --------------------------------------------------------------------------- conv decode step
@torch.library.custom_op("atma_hip::causal_conv1d_decode_step", mutates_args=("state_table",))
def causal_conv1d_decode_step_op(x: Tensor, weight: Tensor, slots: Tensor, state_table: Tensor,
                                 residual: bool) -> Tensor:
    _need_cuda(x, weight, slots, state_table)
    lib = _lib.load()
    x = x if x.stride(-1) == 1 else x.contiguous()
    B, D = x.shape
    K = weight.shape[1]
    out = torch.empty((B, D), device=x.device, dtype=x.dtype)
    st = state_table.stride() if state_table.dim() == 3 else (0, 0, 0)   # unused when K == 1
    rows = state_table.shape[0] if state_table.dim() == 3 else 0
    rc = lib.atma_causal_conv1d_decode_step(
        x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), weight.stride(1),
        slots.data_ptr(), state_table.data_ptr(), st[0], st[1], st[2], rows, out.data_ptr(),
        out.stride(0), B, D, K, 1 if residual else 0, _lib.dtype_code(x.dtype),
        _lib.stream_handle(x.device))
    _lib.check(rc, "causal_conv1d_decode_step")
    return out


@causal_conv1d_decode_step_op.register_fake
def _(x, weight, slots, state_table, residual):
    return torch.empty_like(x)


# --------------------------------------------------------------------------- gated delta backward
@torch.library.custom_op("atma_hip::gated_delta_bwd", mutates_args=())
def gated_delta_bwd_op(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                       initial_state: Optional[Tensor], d_out: Tensor,
                       d_final_state: Optional[Tensor]) -> List[Tensor]:
    """fp32 contiguous (B, T, H, .) inputs; returns dq, dk, dv, dg, dbeta, d_initial_state."""
    _need_cuda(q, k, v, g, beta, d_out)
    lib = _lib.load()
    B, T, H, dk = q.shape
    dv = v.shape[3]
    JB = dv // 16
    f = dict(device=q.device, dtype=torch.float32)
    dq_part = torch.empty((JB, B, T, H, dk), **f)
    dk_part = torch.empty((JB, B, T, H, dk), **f)
    dg_part = torch.empty((JB, B, T, H), **f)
    db_part = torch.empty((JB, B, T, H), **f)
    dv_out = torch.empty((B, T, H, dv), **f)
    ds0 = torch.empty((B, H, dk, dv), **f)
    ws_bytes = lib.atma_gated_delta_bwd_workspace_bytes(B, T, H, dk, dv)
    ws = torch.empty((max(ws_bytes, 4) // 4,), **f)
    rc = lib.atma_gated_delta_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                                  _lib.ptr(initial_state), d_out.data_ptr(), _lib.ptr(d_final_state),
                                  dq_part.data_ptr(), dk_part.data_ptr(), dv_out.data_ptr(), dg_part.data_ptr(),
                                  db_part.data_ptr(), ds0.data_ptr(), B, T, H, dk, dv, ws.data_ptr(),
                                  ws.numel() * 4, _lib.stream_handle(q.device))
    _lib.check(rc, "gated_delta_bwd")
    return [dq_part.sum(0), dk_part.sum(0), dv_out, dg_part.sum(0), db_part.sum(0), ds0]


@gated_delta_bwd_op.register_fake
def _(q, k, v, g, beta, initial_state, d_out, d_final_state):
    B, T, H, dk = q.shape
    dv = v.shape[3]
    return [q.new_empty(q.shape), q.new_empty(q.shape), v.new_empty(v.shape), g.new_empty(g.shape),
            g.new_empty(g.shape), q.new_empty((B, H, dk, dv))]


def _bwd16_check(q, k, v, d_out, g, beta):
    _need_cuda(q, k, v, d_out, g, beta)
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape or d_out.shape != q.shape:
        raise ValueError("gated_delta_bwd16: q, k, v, d_out must all be (B, T, H, d)")
    B, T, H, d = q.shape
    if tuple(g.shape) != (B, T, H) or tuple(beta.shape) != (B, T, H):
        raise ValueError("gated_delta_bwd16: g and beta must be (B, T, H)")
    if g.dtype != torch.float32 or beta.dtype != torch.float32:
        raise ValueError("gated_delta_bwd16: g and beta must be fp32")
    if q.dtype not in (torch.bfloat16, torch.float16) or any(t.dtype != q.dtype for t in (k, v, d_out)):
        raise ValueError("gated_delta_bwd16: q, k, v, d_out must share a 16-bit dtype")
    return [t.contiguous() for t in (q, k, v, d_out, g, beta)]


def _bwd16_prep(q, k, v, d_out, g, beta, scale, l2norm):
    lib = _lib.load()
    B, T, H, d = q.shape
    NC = (T + 63) // 64
    BH = B * H
    t16 = dict(device=q.device, dtype=v.dtype)
    kr, qr = (torch.empty((BH, NC, 64, d), **t16) for _ in range(2))
    kt, qt, vt, ot, got = (torch.empty((BH, NC, d, 64), **t16) for _ in range(5))
    tm, tt, rt = (torch.empty((BH, NC, 64, 64), **t16) for _ in range(3))
    f = torch.empty((BH, NC, 9, 64), device=q.device, dtype=torch.float32)
    rc = lib.atma_gated_delta_bwd16_prep(q.data_ptr(), k.data_ptr(), v.data_ptr(), d_out.data_ptr(), g.data_ptr(),
                                         beta.data_ptr(), kr.data_ptr(), kt.data_ptr(), qr.data_ptr(), qt.data_ptr(),
                                         tm.data_ptr(), tt.data_ptr(), rt.data_ptr(), vt.data_ptr(), ot.data_ptr(),
                                         got.data_ptr(), f.data_ptr(), B, T, H, d, float(scale), 1 if l2norm else 0,
                                         _lib.dtype_code(v.dtype), _lib.stream_handle(q.device))
    _lib.check(rc, "gated_delta_bwd16_prep")
    return [kr, kt, qr, qt, tm, tt, rt, vt, ot, got, f]


def _bwd16_chain(kr, kt, qt, tm, tt, rt, vt, ot, got, f, s0, dst):
    lib = _lib.load()
    BH, NC, C, d = kr.shape
    t16 = dict(device=kr.device, dtype=kr.dtype)
    s_entry, ds_end = (torch.empty((BH, NC, d, d), **t16) for _ in range(2))
    u = torch.empty((BH, NC, C, d), **t16)
    dy = torch.empty((BH, NC, C, d), device=kr.device, dtype=torch.float32)
    ds0 = torch.empty((BH, d, d), device=kr.device, dtype=torch.float32)
    rc = lib.atma_gated_delta_bwd16_chain(kr.data_ptr(), kt.data_ptr(), qt.data_ptr(), tm.data_ptr(), tt.data_ptr(),
                                          rt.data_ptr(), vt.data_ptr(), ot.data_ptr(), got.data_ptr(), f.data_ptr(),
                                          _lib.ptr(s0), _lib.ptr(dst), s_entry.data_ptr(), ds_end.data_ptr(),
                                          u.data_ptr(), dy.data_ptr(), ds0.data_ptr(), BH, NC, d,
                                          _lib.dtype_code(kr.dtype), _lib.stream_handle(kr.device))
    _lib.check(rc, "gated_delta_bwd16_chain")
    return [s_entry, ds_end, u, dy, ds0]


def _bwd16_local(kr, kt, qr, qt, q, k, v, d_out, f, s_entry, ds_end, u, dy):
    lib = _lib.load()
    B, T, H, d = q.shape
    t16 = dict(device=q.device, dtype=q.dtype)
    dq, dk, dv = (torch.empty((B, T, H, d), **t16) for _ in range(3))
    dg, db = (torch.empty((B, T, H), device=q.device, dtype=torch.float32) for _ in range(2))
    rc = lib.atma_gated_delta_bwd16_local(kr.data_ptr(), kt.data_ptr(), qr.data_ptr(), qt.data_ptr(), q.data_ptr(),
                                          k.data_ptr(), v.data_ptr(), d_out.data_ptr(), f.data_ptr(),
                                          s_entry.data_ptr(), ds_end.data_ptr(), u.data_ptr(), dy.data_ptr(),
                                          dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dg.data_ptr(), db.data_ptr(),
                                          B, T, H, d, _lib.dtype_code(q.dtype), _lib.stream_handle(q.device))
    _lib.check(rc, "gated_delta_bwd16_local")
    return [dq, dk, dv, dg, db]


def _bwd16_states(initial_state, d_final_state, B, H, d):
    out = []
    for x in (initial_state, d_final_state):
        if x is not None and tuple(x.shape) != (B, H, d, d):
            raise ValueError("gated_delta_bwd16: states must be (B, H, d, d)")
        out.append(None if x is None else x.to(torch.float32).contiguous().reshape(B * H, d, d))
    return out


@torch.library.custom_op("atma_hip::gated_delta_bwd16", mutates_args=())
def gated_delta_bwd16_op(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                         initial_state: Optional[Tensor], d_out: Tensor, d_final_state: Optional[Tensor],
                         scale: float, l2norm: bool) -> List[Tensor]:
    """Chunked (WY) backward for 16-bit training of ``chunk_gated_delta_rule`` with raw
    q, k, v, d_out (B, T, H, d) of one 16-bit dtype (l2norm: q and k l2-normalised in the
    recurrence, q then times scale); g (log decay), beta (B, T, H) fp32; initial_state,
    d_final_state (B, H, d, d) fp32 or None.  Returns dq, dk, dv (16-bit), dg, dbeta,
    d_initial_state (fp32).  Three launches: prep, chain, local."""
    q, k, v, d_out, g, beta = _bwd16_check(q, k, v, d_out, g, beta)
    B, T, H, d = q.shape
    s0, dst = _bwd16_states(initial_state, d_final_state, B, H, d)
    if T == 0:
        ds0 = torch.zeros((B, H, d, d), device=q.device, dtype=torch.float32) if dst is None else \
            dst.reshape(B, H, d, d).clone()
        return [torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v), torch.zeros_like(g),
                torch.zeros_like(beta), ds0]
    kr, kt, qr, qt, tm, tt, rt, vt, ot, got, f = _bwd16_prep(q, k, v, d_out, g, beta, scale, l2norm)
    s_entry, ds_end, u, dy, ds0 = _bwd16_chain(kr, kt, qt, tm, tt, rt, vt, ot, got, f, s0, dst)
    dq, dk, dv, dg, db = _bwd16_local(kr, kt, qr, qt, q, k, v, d_out, f, s_entry, ds_end, u, dy)
    return [dq, dk, dv, dg, db, ds0.reshape(B, H, d, d)]


@gated_delta_bwd16_op.register_fake
def _(q, k, v, g, beta, initial_state, d_out, d_final_state, scale, l2norm):
    B, T, H, d = q.shape
    return [q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape), g.new_empty(g.shape),
            g.new_empty(g.shape), g.new_empty((B, H, d, d))]


def gated_delta_bwd16_stages(q, k, v, g, beta, initial_state, d_out, d_final_state, scale, l2norm):
    """The three launches of ``gated_delta_bwd16`` with every intermediate returned (for
    tests): dict of the prep's tiles (kr, kt, qr, qt, tm, tt, rt, vt, ot, got, f; chunk-head
    tensors shaped (B*H, NC, ...)), the chain's outputs (s_entry, ds_end, u, dy, ds0) and
    the local gradients (dq, dk, dv, dg, db)."""
    q, k, v, d_out, g, beta = _bwd16_check(q, k, v, d_out, g, beta)
    B, T, H, d = q.shape
    s0, dst = _bwd16_states(initial_state, d_final_state, B, H, d)
    names = ["kr", "kt", "qr", "qt", "tm", "tt", "rt", "vt", "ot", "got", "f"]
    out = dict(zip(names, _bwd16_prep(q, k, v, d_out, g, beta, scale, l2norm)))
    chain = _bwd16_chain(*(out[n] for n in ("kr", "kt", "qt", "tm", "tt", "rt", "vt", "ot", "got", "f")), s0, dst)
    out.update(zip(["s_entry", "ds_end", "u", "dy", "ds0"], chain))
    loc = _bwd16_local(out["kr"], out["kt"], out["qr"], out["qt"], q, k, v, d_out, out["f"], out["s_entry"],
                       out["ds_end"], out["u"], out["dy"])
    out.update(zip(["dq", "dk", "dv", "dg", "db"], loc))
    return out


# --------------------------------------------------------------------------- inference fusions
@torch.library.custom_op("atma_hip::squared_relu_gate", mutates_args=())
def squared_relu_gate_op(x: Tensor, gate: Tensor) -> Tensor:
    _need_cuda(x, gate)
    lib = _lib.load()
    rows, width = x.shape
    out = torch.empty((rows, width), device=x.device, dtype=x.dtype)
    rc = lib.atma_squared_relu_gate(x.data_ptr(), x.stride(0), x.stride(1), gate.data_ptr(), gate.stride(0),
                                    gate.stride(1), out.data_ptr(), rows, width, _lib.dtype_code(x.dtype),
                                    _lib.stream_handle(x.device))
    _lib.check(rc, "squared_relu_gate")
    return out


@squared_relu_gate_op.register_fake
def _(x, gate):
    return x.new_empty(x.shape)


@torch.library.custom_op("atma_hip::softcap_logits", mutates_args=())
def softcap_logits_op(logits: Tensor) -> Tensor:
    _need_cuda(logits)
    lib = _lib.load()
    logits = logits.contiguous()
    out = torch.empty_like(logits)
    rc = lib.atma_softcap_logits(logits.data_ptr(), out.data_ptr(), logits.numel(),
                                 _lib.dtype_code(logits.dtype), _lib.stream_handle(logits.device))
    _lib.check(rc, "softcap_logits")
    return out


@softcap_logits_op.register_fake
def _(logits):
    return torch.empty_like(logits)


@torch.library.custom_op("atma_hip::linear_tokens", mutates_args=())
def linear_tokens_op(x: Tensor, weight: Tensor, bias: Optional[Tensor]) -> Tensor:
    """y = x weight^T (+ bias) for a few token rows (x (M, K), M <= 32): the decode
    projection of the served model, weights streamed once (``atma_linear_tokens``)."""
    _need_cuda(x, weight)
    lib = _lib.load()
    M, K = x.shape
    N = weight.shape[0]
    if x.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError("linear_tokens: x and weight need unit inner stride")
    out = torch.empty((M, N), device=x.device, dtype=x.dtype)
    b = bias.contiguous() if bias is not None else None
    rc = lib.atma_linear_tokens(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                                None if b is None else b.data_ptr(), out.data_ptr(), out.stride(0),
                                M, N, K, _lib.dtype_code(x.dtype), _lib.stream_handle(x.device))
    _lib.check(rc, "linear_tokens")
    return out


@linear_tokens_op.register_fake
def _(x, weight, bias):
    return x.new_empty((x.shape[0], weight.shape[0]))


@torch.library.custom_op("atma_hip::softcap_argmax", mutates_args=())
def softcap_argmax_op(logits: Tensor) -> List[Tensor]:
    _need_cuda(logits)
    rows, V = logits.shape
    out = torch.empty((rows, V), device=logits.device, dtype=logits.dtype)
    ids = torch.empty((rows,), device=logits.device, dtype=torch.int64)
    rc = _lib.load().atma_softcap_argmax(logits.data_ptr(), logits.stride(0), out.data_ptr(), out.stride(0),
                                         ids.data_ptr(), rows, V, _lib.dtype_code(logits.dtype),
                                         _lib.stream_handle(logits.device))
    _lib.check(rc, "softcap_argmax")
    return [out, ids]


@softcap_argmax_op.register_fake
def _(logits):
    return [logits.new_empty(logits.shape), logits.new_empty((logits.shape[0],), dtype=torch.int64)]


@torch.library.custom_op("atma_hip::packed_causal_conv1d", mutates_args=("state_table",))
def packed_causal_conv1d_op(x: Tensor, weight: Tensor, state_table: Tensor, token_seq_starts: Tensor,
                            token_seq_ends: Tensor, token_seq_slots: Tensor) -> Tensor:
    _need_cuda(x, weight, state_table, token_seq_starts, token_seq_ends, token_seq_slots)
    lib = _lib.load()
    total, channels = x.shape
    K = weight.shape[1]
    out = torch.empty((total, channels), device=x.device, dtype=x.dtype)
    ss = state_table.stride()
    rc = lib.atma_packed_causal_conv1d(
        x.data_ptr(), x.stride(0), x.stride(1), weight.data_ptr(), weight.stride(0), weight.stride(1),
        out.data_ptr(), state_table.data_ptr(), ss[0], ss[1], ss[2], state_table.shape[0],
        token_seq_starts.data_ptr(), token_seq_ends.data_ptr(), token_seq_slots.data_ptr(), total, channels, K,
        _lib.dtype_code(x.dtype), _lib.dtype_code(state_table.dtype), _lib.stream_handle(x.device))
    _lib.check(rc, "packed_causal_conv1d")
    return out


@packed_causal_conv1d_op.register_fake
def _(x, weight, state_table, token_seq_starts, token_seq_ends, token_seq_slots):
    return x.new_empty(x.shape)


# --------------------------------------------------------------------------- memory gates
@torch.library.custom_op("atma_hip::gated_delta_gates", mutates_args=())
def gated_delta_gates_op(zg: Tensor, zb: Tensor, g_bias: float, b_bias: float,
                         decay_as_prob: bool) -> List[Tensor]:
    _need_cuda(zg, zb)
    if zg.dtype != torch.float32 or zb.dtype != torch.float32 or zg.shape != zb.shape:
        raise ValueError("gate logits: two float32 tensors of the same shape")
    lib = _lib.load()
    zg, zb = zg.contiguous(), zb.contiguous()
    g, beta = torch.empty_like(zg), torch.empty_like(zb)
    rc = lib.atma_gated_delta_gates(zg.data_ptr(), zb.data_ptr(), g_bias, b_bias, g.data_ptr(),
                                    beta.data_ptr(), zg.numel(), 1 if decay_as_prob else 0,
                                    _lib.stream_handle(zg.device))
    _lib.check(rc, "gated_delta_gates")
    return [g, beta]


@gated_delta_gates_op.register_fake
def _(zg, zb, g_bias, b_bias, decay_as_prob):
    return [torch.empty_like(zg), torch.empty_like(zb)]


# --------------------------------------------------------------------------- chunked gated delta
def _chunk_gated_delta(q, k, v, g, beta, initial_state, scale, use_qk_l2norm, want_final, start_flag,
                       start_epoch, gate_logits, g_bias, b_bias):
    _need_cuda(q, k, v, g, beta, initial_state)
    lib = _lib.load()
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    B, T, H, dk = q.shape
    dv = v.shape[3]
    o = torch.empty((B, T, H, dv), device=q.device, dtype=q.dtype)
    final = torch.empty((B, H, dk, dv), device=q.device, dtype=torch.float32) if want_final else None
    chunk = 64
    ws_bytes = lib.atma_chunk_gated_delta_workspace_bytes(B, T, H, dk, dv, chunk,
                                                          _lib.dtype_code(q.dtype))
    ws = torch.empty((max(ws_bytes, 4) // 4,), device=q.device, dtype=torch.float32)
    rc = lib.atma_chunk_gated_delta_rule(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        g.data_ptr(), beta.data_ptr(), _lib.ptr(initial_state), _lib.ptr(final), o.data_ptr(),
        B, T, H, k.shape[2], dk, dv, _lib.dtype_code(q.dtype), scale, 1 if use_qk_l2norm else 0,
        1 if gate_logits else 0, g_bias, b_bias, chunk,
        ws.data_ptr(), ws.numel() * 4, _lib.ptr(start_flag), start_epoch, _lib.stream_handle(q.device))
    _lib.check(rc, "chunk_gated_delta_rule")
    return [o, final] if want_final else [o]


@torch.library.custom_op("atma_hip::chunk_gated_delta_rule", mutates_args=("start_flag",))
def chunk_gated_delta_rule_op(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                              initial_state: Optional[Tensor], scale: float, use_qk_l2norm: bool,
                              want_final: bool, start_flag: Optional[Tensor], start_epoch: int,
                              gate_logits: bool = False, g_bias: float = 0.0,
                              b_bias: float = 0.0) -> List[Tensor]:
    """Inference prefill; ``start_flag`` (mutated) is raised as the recurrence starts."""
    return _chunk_gated_delta(q, k, v, g, beta, initial_state, scale, use_qk_l2norm, want_final,
                              start_flag, start_epoch, gate_logits, g_bias, b_bias)


@torch.library.custom_op("atma_hip::gated_delta_fwd", mutates_args=())
def gated_delta_fwd_op(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                       initial_state: Optional[Tensor], scale: float = 1.0,
                       l2norm: bool = False) -> List[Tensor]:
    """The recurrence forward of the autograd routes (log decay, beta; q and k as given,
    l2-normalised in-kernel with ``l2norm``, q then times ``scale``): the prefill kernels
    with no start flag, so it mutates nothing and functionalises under torch.compile.
    Returns [o, final state]."""
    return _chunk_gated_delta(q, k, v, g, beta, initial_state, scale, l2norm, True, None, 0, False, 0.0, 0.0)


@gated_delta_fwd_op.register_fake
def _(q, k, v, g, beta, initial_state, scale=1.0, l2norm=False):
    B, T, H, dk = q.shape
    dv = v.shape[3]
    return [q.new_empty((B, T, H, dv)), q.new_empty((B, H, dk, dv), dtype=torch.float32)]


@chunk_gated_delta_rule_op.register_fake
def _(q, k, v, g, beta, initial_state, scale, use_qk_l2norm, want_final, start_flag, start_epoch,
      gate_logits=False, g_bias=0.0, b_bias=0.0):
    B, T, H, dk = q.shape
    dv = v.shape[3]
    o = q.new_empty((B, T, H, dv))
    return [o, q.new_empty((B, H, dk, dv), dtype=torch.float32)] if want_final else [o]


@torch.library.custom_op("atma_hip::wait_start_flag", mutates_args=("flag",))
def wait_start_flag_op(flag: Tensor, epoch: int, timeout_us: int) -> None:
    _need_cuda(flag)
    if flag.dtype != torch.int32 or flag.numel() < 1:
        raise ValueError("wait_start_flag: flag must be an int32 device tensor")
    rc = _lib.load().atma_wait_start_flag(flag.data_ptr(), epoch, timeout_us,
                                          _lib.stream_handle(flag.device))
    _lib.check(rc, "wait_start_flag")


@wait_start_flag_op.register_fake
def _(flag, epoch, timeout_us):
    return None


# --------------------------------------------------------------------------- paged KV write
@torch.library.custom_op("atma_hip::store_kvcache", mutates_args=("k_cache", "v_cache"))
def store_kvcache_op(key: Tensor, value: Tensor, k_cache: Tensor, v_cache: Tensor,
                     slot_mapping: Tensor) -> None:
    _need_cuda(key, value, k_cache, v_cache, slot_mapping)
    lib = _lib.load()
    N, hkv, d = key.shape
    row = hkv * d
    rc = lib.atma_store_kvcache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), k_cache.data_ptr(),
        v_cache.data_ptr(), slot_mapping.data_ptr(), N, row, k_cache.numel() // row,
        _lib.dtype_code(key.dtype), _lib.stream_handle(key.device))
    _lib.check(rc, "store_kvcache")


@store_kvcache_op.register_fake
def _(key, value, k_cache, v_cache, slot_mapping):
    return None

"""C-ABI checks that need no GPU: the library loads, exports every symbol declared in
include/atma_hip.h with the Python binding's signature table, and its host-side
argument validation rejects bad requests before any launch."""

import ctypes
import re

import pytest
import torch

from atma_amd import _lib


def _declared():
    text = _lib.HEADER.read_text()
    body = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(atma_\w+)\s*\(", body)))


def test_header_and_binding_agree():
    assert _declared() == sorted(_lib.SIGNATURES), "include/atma_hip.h and _lib.SIGNATURES differ"


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libatma_hip.so missing: run `python -m atma_amd._build` (the driver's build())")
    return _lib.load()


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.atma_abi_version() == 2


def test_validation_rejects_without_launch(lib):
    null = None
    # is_causal with Tq != Tk
    rc = lib.atma_polar_attention_fwd(null, 0, 0, 0, null, 0, 0, 0, null, 0, 0, 0, null, null, null,
                                      null, null, null, null, null, null, null, null, null,
                                      1, 8, 2, 16, 32, 128, 1, 1, 0, 0, 1e-6, null)
    assert rc == 1 and b"Tq == Tk" in lib.atma_last_error()
    # unsupported head dim
    rc = lib.atma_polar_attention_fwd(null, 0, 0, 0, null, 0, 0, 0, null, 0, 0, 0, null, null, null,
                                      null, null, null, null, null, null, null, null, null,
                                      1, 8, 2, 16, 16, 96, 1, 0, 0, 0, 1e-6, null)
    assert rc == 2
    # GQA group not dividing
    rc = lib.atma_polar_attention_decode(null, 0, 0, null, null, 4, 256, 3, null, 0, 2, null, null,
                                         null, null, null, null, null, null, 2, 8, 128, 1, 0, 1e-6,
                                         null, 0, null)
    assert rc == 1
    # decode workspace too small
    # span split (fp32): one (m, L, Q2, pad, acc[d]) fp32 record per (sequence, query head, span)
    need = lib.atma_polar_decode_workspace_bytes(2, 8, 2, 4, 256, 128, 0)
    rec = 2 * 8 * (128 + 4) * 4
    assert need > 0 and need % rec == 0
    assert lib.atma_polar_decode_workspace_bytes(2, 8, 2, 128, 256, 128, 0) >= need
    assert lib.atma_polar_decode_workspace_bytes(2, 8, 2, 0, 256, 128, 0) == 0
    # balanced split (16-bit, pages of 32-key multiples): (waves + B * Hkv) records of G rows;
    # waves = 4 * min(512, ceil(units / 4)) with units = B * Hkv * ceil(max_pages * page / 32)
    # after a header of whole 256-byte blocks holding the B + 1 prefix entries
    row = (128 + 4) * 4
    assert lib.atma_polar_decode_workspace_bytes(2, 8, 2, 4, 256, 128, 1) == 256 + (128 + 4) * 4 * row
    assert lib.atma_polar_decode_workspace_bytes(64, 8, 2, 128, 256, 128, 1) == 512 + (2048 + 128) * 4 * row
    # a page size that is not a multiple of 32 keys takes the span split
    assert lib.atma_polar_decode_workspace_bytes(2, 8, 2, 4, 16, 128, 1) == \
        lib.atma_polar_decode_workspace_bytes(2, 8, 2, 4, 16, 128, 0)
    buf = ctypes.create_string_buffer(16)
    rc = lib.atma_polar_attention_decode(buf, 8, 8, buf, buf, 4, 256, 2, buf, 4, 4, buf, buf, buf,
                                         buf, buf, buf, buf, buf, 2, 8, 128, 1, 0, 1e-6, buf, 16, null)
    assert rc == 3
    # chunked gated delta: chunk must be 64; dk == dv
    assert lib.atma_chunk_gated_delta_rule(null, 0, 0, 0, null, 0, 0, 0, null, 0, 0, 0, null, null,
                                           null, null, null, 1, 64, 2, 2, 128, 128, 1, 1.0, 1, 0,
                                           0.0, 0.0, 32,
                                           null, 0, null, 0, null) == 2
    # start-flag wait: null flag, timeout out of range
    assert lib.atma_wait_start_flag(null, 1, 1000, null) == 1
    buf4 = ctypes.create_string_buffer(4)
    assert lib.atma_wait_start_flag(buf4, 1, 0, null) == 1
    assert lib.atma_chunk_gated_delta_workspace_bytes(1, 65, 2, 128, 128, 64, 0) == 2 * 2 * (5 * 64 * 128 + 4) * 4
    # 16-bit path: one 13 KiB record per (sequence, head, chunk): T diag(beta) and Rq as six
    # 16 x 32 16-bit MFMA fragments each, then 4 x 64 fp32 per-token factors
    rec16 = 6 * 1024 + 6 * 1024 + 4 * 64 * 4
    assert lib.atma_chunk_gated_delta_workspace_bytes(1, 65, 2, 128, 128, 64, 1) == 2 * 2 * rec16
    assert lib.atma_chunk_gated_delta_workspace_bytes(3, 64, 4, 64, 64, 64, 2) == 3 * 4 * 1 * rec16
    # a long sequence with few heads splits the recurrence into segments (here 5 of 205
    # chunks: 8 heads x 8 summary workgroups per segment on 256 compute units), adding the
    # segments' [B | M] summaries (d x 2d fp32) and entry states (d x d fp32)
    assert lib.atma_chunk_gated_delta_workspace_bytes(1, 65536, 8, 128, 128, 64, 1) == \
        8 * 1024 * rec16 + 8 * 5 * 128 * 3 * 128 * 4
    # gated delta step: unsupported dims
    assert lib.atma_gated_delta_decode_step(null, 0, 0, null, 0, 0, null, 0, 0, null, null, null, 1,
                                            null, null, 1, 1, 1, 96, 96, 1, 1e-12, null) == 2
    # packed Polar prefill: 16-bit only; no tiles is a no-op
    assert lib.atma_polar_attention_packed_fwd(null, 0, 0, null, 0, 0, null, 0, 0, null, null, null, 1,
                                               null, null, null, null, null, null, 0, 0, null, 0, 0,
                                               10, 8, 2, 128, 0, 0, 1e-6, null) == 2
    assert lib.atma_polar_attention_packed_fwd(null, 0, 0, null, 0, 0, null, 0, 0, null, null, null, 0,
                                               null, null, null, null, null, null, 0, 0, null, 0, 0,
                                               10, 8, 2, 128, 1, 0, 1e-6, null) == 0
    # conv decode step: K out of range; zero rows are a no-op
    assert lib.atma_causal_conv1d_decode_step(null, 0, null, 0, 0, null, null, 0, 0, 0, 1, null, 0,
                                              1, 8, 17, 0, 1, null) == 1
    assert lib.atma_causal_conv1d_decode_step(null, 0, null, 0, 0, null, null, 0, 0, 0, 1, null, 0,
                                              0, 8, 4, 0, 1, null) == 0
    # Polar backward: causal needs Tq == Tk; head dim 96 unsupported; grouping; empty is a no-op
    bwd0 = [null, 0, 0, 0] * 4 + [null] * 9
    assert lib.atma_polar_attention_bwd(*bwd0, 1, 8, 2, 16, 32, 128, 1, 1, 0, null) == 1
    assert b"Tq == Tk" in lib.atma_last_error()
    assert lib.atma_polar_attention_bwd(*bwd0, 1, 8, 2, 16, 16, 96, 1, 1, 0, null) == 2
    assert lib.atma_polar_attention_bwd(*bwd0, 1, 8, 3, 16, 16, 128, 1, 1, 0, null) == 1
    assert lib.atma_polar_attention_bwd(*bwd0, 1, 8, 2, 0, 0, 128, 1, 1, 0, null) == 0
    # backward preamble: head dim 96 unsupported; no rows is a no-op; null statistics
    prep0 = [null] * 17
    assert lib.atma_polar_attention_bwd_prep(*prep0, 2, 8, 16, 96, 1, 0, 0, 1e-6, null) == 2
    assert lib.atma_polar_attention_bwd_prep(*prep0, 2, 8, 0, 128, 1, 0, 0, 1e-6, null) == 0
    assert lib.atma_polar_attention_bwd_prep(*prep0, 2, 8, 16, 128, 1, 0, 0, 1e-6, null) == 1
    # backward group sum: elems must be a multiple of 4; nothing to do is a no-op
    assert lib.atma_polar_bwd_group_sum(null, 0, null, 2, 4, 6, 1, null) == 1
    assert lib.atma_polar_bwd_group_sum(null, 0, null, 0, 4, 8, 1, null) == 0
    # store_kvcache: unknown dtype
    assert lib.atma_store_kvcache(null, 0, null, 0, null, null, null, 1, 256, 8, 9, null) == 1
    # zero-size requests are no-ops
    assert lib.atma_store_kvcache(null, 0, null, 0, null, null, null, 0, 256, 8, 1, null) == 0


def test_fusion_entry_points_validate_without_launch(lib):
    """The served path's projections and fusions reject bad requests before any launch
    (ATMA_ERR_INVALID = 1, ATMA_ERR_UNSUPPORTED = 2) and treat empty requests as no-ops."""
    null, BF16, F32 = None, 1, 0
    buf = ctypes.create_string_buffer(64)
    ptr = ctypes.cast(buf, ctypes.c_void_p)
    ptrs = (ctypes.c_void_p * 9)(*([ptr.value] * 9))
    lds = (ctypes.c_int64 * 9)(*([1024] * 9))
    ns = (ctypes.c_int64 * 9)(*([64] * 9))
    # residual + RMSNorm: D outside [8, 4096] or not a multiple of 8; both y and parts; 16-bit only
    assert lib.atma_residual_rms_norm(null, 0, null, 0, null, 0, null, 0, null, 0, null, 0, null, 0,
                                      null, null, 0, 4, 8192, 1e-6, BF16, null) == 1
    assert lib.atma_residual_rms_norm(ptr, 64, buf, 1, null, 0, null, 0, null, 0, null, 0, null, 0,
                                      ptr, ptr, 64, 4, 64, 1e-6, BF16, null) == 1
    assert lib.atma_residual_rms_norm(null, 0, null, 0, null, 0, null, 0, null, 0, null, 0, null, 0,
                                      null, null, 0, 4, 64, 1e-6, F32, null) == 2
    assert lib.atma_residual_rms_norm(null, 0, null, 0, null, 0, null, 0, null, 0, null, 0, null, 0,
                                      null, null, 0, 0, 64, 1e-6, BF16, null) == 0
    # token-row projections: at most 32 rows, K of 256 .. 2048, 1 to 8 weight segments
    assert lib.atma_linear_tokens_multi(ptr, 1024, 33, 1024, 1, ptrs, lds, ptrs, ptrs, lds, ns, BF16, null) == 2
    assert lib.atma_linear_tokens_multi(ptr, 1024, 4, 1000, 1, ptrs, lds, ptrs, ptrs, lds, ns, BF16, null) == 2
    assert lib.atma_linear_tokens_multi(ptr, 1024, 4, 1024, 9, ptrs, lds, ptrs, ptrs, lds, ns, BF16, null) == 1
    assert lib.atma_linear_tokens_multi(null, 1024, 4, 1024, 1, ptrs, lds, ptrs, ptrs, lds, ns, BF16, null) == 1
    assert lib.atma_linear_tokens_gated(ptr, 1024, ptr, 1024, null, ptr, 1024, 4, 40, 1024, BF16, null) == 2
    # gated MLP projection over many rows: H and K multiples of 128; no rows is a no-op
    assert lib.atma_linear_gated(ptr, 1024, ptr, 1024, null, ptr, 4096, 64, 4000, 1024, BF16, null) == 2
    assert lib.atma_linear_gated(ptr, 1024, ptr, 1024, null, ptr, 4096, 64, 4096, 1000, BF16, null) == 2
    assert lib.atma_linear_gated(ptr, 1024, ptr, 1024, null, ptr, 4096, 64, 4096, 1024, F32, null) == 2
    assert lib.atma_linear_gated(null, 1024, ptr, 1024, null, ptr, 4096, 64, 4096, 1024, BF16, null) == 1
    assert lib.atma_linear_gated(null, 0, null, 0, null, null, 0, 0, 4096, 1024, BF16, null) == 0
    # in_proj + conv step: H a multiple of 16, 1 .. 16 taps, a state table when taps > 1
    assert lib.atma_linear_tokens_conv(ptr, 1024, ptr, 1024, null, ptr, 3, ptr, ptr, 2048, 4, ptr, 1024,
                                       4, 40, 1024, BF16, null) == 2
    assert lib.atma_linear_tokens_conv(ptr, 1024, ptr, 1024, null, ptr, 17, ptr, ptr, 2048, 4, ptr, 1024,
                                       4, 1024, 1024, BF16, null) == 2
    assert lib.atma_linear_tokens_conv(ptr, 1024, ptr, 1024, null, ptr, 3, null, null, 2048, 4, ptr, 1024,
                                       4, 1024, 1024, BF16, null) == 1
    assert lib.atma_linear_tokens_conv(ptr, 1024, ptr, 1024, null, ptr, 3, ptr, ptr, 1000, 4, ptr, 1024,
                                       4, 1024, 1024, BF16, null) == 1
    assert lib.atma_linear_tokens_chunks(ptr, 4096, 4, 1024, 9, ptrs, lds, 64, buf, BF16, null) == 2
    assert lib.atma_linear_tokens_chunks(ptr, 2048, 4, 1024, 4, ptrs, lds, 64, buf, BF16, null) == 1
    # LFM2 conv step: kernel size 1 .. 16; no rows is a no-op
    assert lib.atma_lfm2_conv_step(null, 0, null, 17, null, null, 0, 0, null, 0, 1, 8, BF16, null) == 1
    assert lib.atma_lfm2_conv_step(null, 24, null, 3, null, null, 0, 0, null, 8, 0, 8, BF16, null) == 0
    # global decode inputs: head dim 64 or 128; heads in groups
    assert lib.atma_global_decode_prep(null, 0, 0, 0, 0, 0, null, null, null, 4, null, 0, null, 0, null, 0,
                                       0, null, null, null, null, null, null, 1e-6, 0.0, 0.0,
                                       1, 8, 2, 96, BF16, null) == 1
    assert lib.atma_global_decode_prep(null, 0, 0, 0, 0, 0, null, null, null, 4, null, 0, null, 0, null, 0,
                                       0, null, null, null, null, null, null, 1e-6, 0.0, 0.0,
                                       1, 8, 3, 128, BF16, null) == 1
    # per-head RMSNorm: head dim 64 or 128; overlapping heads
    assert lib.atma_head_rms_norm(null, 0, 0, null, 4, 8, 96, 1e-6, BF16, null) == 1
    assert lib.atma_head_rms_norm(ptr, 256, 128, ptr, 4, 8, 128, 1e-6, BF16, null) == 1
    assert lib.atma_head_rms_norm(null, 0, 0, null, 0, 8, 128, 1e-6, BF16, null) == 0
    # gated projection inputs: rows a multiple of T; r of another 16-bit dtype
    assert lib.atma_global_gate(null, 0, 0, 0, 3, null, 0, 0, null, 0, F32, null, 0, null, 0, null, 0,
                                4, 8, 128, 1e-6, BF16, null) == 1
    assert lib.atma_global_gate(ptr, 0, 0, 0, 4, ptr, 0, 0, ptr, 0, 2, ptr, 0, ptr, 0, ptr, 0,
                                4, 8, 128, 1e-6, BF16, null) == 1
    assert lib.atma_global_decode_gate(null, null, null, 0, 0, null, 0, 1e-6, 1, 8, 96, BF16, null) == 1
    # packed LFM2 prefill conv: kernel sizes 3 and 4 only; D a multiple of 8
    assert lib.atma_lfm2_conv_packed(null, 0, null, 5, null, 0, null, 0, 0, null, null, null, 4, 64,
                                     BF16, null) == 2
    assert lib.atma_lfm2_conv_packed(null, 0, null, 3, null, 0, null, 0, 0, null, null, null, 4, 60,
                                     BF16, null) == 1
    assert lib.atma_lfm2_conv_packed(null, 0, null, 3, null, 0, null, 0, 0, null, null, null, 0, 64,
                                     BF16, null) == 0
    # softcap + greedy pick: 16-bit logits; rows shorter than V
    assert lib.atma_softcap_argmax(null, 0, null, 0, null, 2, 100, F32, null) == 2
    assert lib.atma_softcap_argmax(null, 50, null, 100, null, 2, 100, BF16, null) == 1
    assert lib.atma_softcap_argmax(null, 100, null, 100, null, 0, 100, BF16, null) == 0


def test_python_wrappers_validate_like_the_reference():
    from atma_amd.kernel import polar_attention_fwd
    p = dict(v_null=torch.zeros(2, 128), null_base=torch.zeros(2), null_slope_raw=torch.zeros(2),
             len_gain_raw=torch.zeros(2), mag_beta_raw=torch.zeros(2))
    q = torch.zeros(1, 2, 4, 128)
    k = torch.zeros(1, 2, 6, 128)
    with pytest.raises(ValueError, match="Tq == Tk"):
        polar_attention_fwd(q, k, k, torch.arange(1, 5.0), is_causal=True, **p)
    q3 = torch.zeros(1, 2, 4, 96)
    with pytest.raises(ValueError, match="power of two"):
        polar_attention_fwd(q3, q3, q3, torch.arange(1, 5.0), **p)


def test_gated_delta_wrappers_check_head_grouping():
    """Grouped KV heads must divide the query heads; shapes are checked before any
    device work, so CPU tensors reach the check."""
    from atma_amd.kernel import chunk_gated_delta_rule, gated_delta_decode_step
    q, k = torch.zeros(1, 5, 6, 64), torch.zeros(1, 5, 4, 64)
    g = torch.zeros(1, 5, 6)
    with pytest.raises(ValueError, match="multiple of k/v heads"):
        chunk_gated_delta_rule(q, k, k, g, g)
    with pytest.raises(ValueError, match="required"):
        chunk_gated_delta_rule(q, k[:, :4], k, g, g)
    table = torch.zeros(2, 6, 64, 64)
    with pytest.raises(ValueError, match="multiple of k/v heads"):
        gated_delta_decode_step(q[:, 0], k[:, 0], k[:, 0], g[:, 0], g[:, 0], table, torch.zeros(1))


@pytest.mark.parametrize("bad", ["g", "beta", "initial_state", "raw_g"])
def test_gated_delta_autograd_route_checks_shapes_first(bad):
    """Inputs that require grad take the autograd route; a mis-shaped g, beta or initial
    state must raise ValueError there too, before any launch (CPU tensors reach the check)."""
    from atma_amd.kernel import chunk_gated_delta_rule
    B, T, H, d = 1, 5, 4, 64
    q = torch.zeros(B, T, H, d, requires_grad=True)
    k = torch.zeros(B, T, 2, d, requires_grad=True)
    g, beta = torch.zeros(B, T, H, requires_grad=True), torch.zeros(B, T, H, requires_grad=True)
    S0 = torch.zeros(B, H, d, d, requires_grad=True)
    kw = {}
    if bad == "g":
        g = torch.zeros(B, T + 1, H, requires_grad=True)
    elif bad == "beta":
        beta = torch.zeros(B, T, H - 1, requires_grad=True)
    elif bad == "initial_state":
        S0 = torch.zeros(B, H, d, d // 2, requires_grad=True)
    else:
        g, kw = torch.zeros(B, T, 1, requires_grad=True), {"gate_bias": (3.9, 0.0)}
    with pytest.raises(ValueError):
        chunk_gated_delta_rule(q, k, k, g, beta, initial_state=S0, **kw)


def test_packed_wrapper_validates_like_the_reference():
    """kernel/polar_triton.py:625-635: 16-bit only, [tokens, heads, dim] shapes, equal-length
    tile maps, power-of-two head dim -- all checked before any device work."""
    from atma_amd.kernel import polar_attention_packed_fwd
    p = dict(v_null=torch.zeros(2, 128), null_base=torch.zeros(2), null_slope_raw=torch.zeros(2),
             len_gain_raw=torch.zeros(2), mag_beta_raw=torch.zeros(2))
    t = torch.zeros(3, dtype=torch.int32)
    q = torch.zeros(10, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="16-bit"):
        polar_attention_packed_fwd(q.float(), q.float(), q.float(), t, t, t, **p)
    with pytest.raises(ValueError, match="equal lengths"):
        polar_attention_packed_fwd(q, q, q, t, t, t[:2], **p)
    with pytest.raises(ValueError, match="tokens, heads, dim"):
        polar_attention_packed_fwd(q, q[:5], q[:5], t, t, t, **p)
    q96 = torch.zeros(10, 2, 96, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="power of two"):
        polar_attention_packed_fwd(q96, q96, q96, t, t, t, **p)


def test_cpu_tensors_fail_loudly():
    from atma_amd.kernel import polar_attention_fwd
    p = dict(v_null=torch.zeros(2, 128), null_base=torch.zeros(2), null_slope_raw=torch.zeros(2),
             len_gain_raw=torch.zeros(2), mag_beta_raw=torch.zeros(2))
    q = torch.zeros(1, 2, 4, 128)
    with pytest.raises(RuntimeError, match="GPU only"):
        polar_attention_fwd(q, q, q, torch.arange(1, 5.0), **p)


def test_noalloc_decode_rejects_requests_above_its_scratch(lib):
    """The no-allocation decode refuses, before touching any device, a launch whose split
    records exceed its fixed scratch array."""
    cap = lib.atma_polar_decode_noalloc_max_bytes()
    assert cap == 32 << 20
    B, Hq, page, d = 4096, 8, 256, 128
    max_pages = 256
    assert lib.atma_polar_decode_workspace_bytes(B, Hq, 2, max_pages, page, d, 0) > cap
    null = None
    rc = lib.atma_polar_attention_decode_noalloc(null, 0, 0, null, null, 16, page, 2, null, 0, max_pages,
                                                 null, null, null, null, null, null, null, null, B, Hq, d,
                                                 0, 0, 1e-6, null)
    assert rc == 3 and b"scratch maximum" in lib.atma_last_error()

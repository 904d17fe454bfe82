"""Per-head glue of the global layer, the LFM2 prefill conv and the MLP's gated first
projection over many rows, backed by libatma_hip.so (C ABI ``atma_head_rms_norm``,
``atma_global_gate``, ``atma_lfm2_conv_packed``, ``atma_linear_gated``).

No reference counterparts: each is one launch for a chain of the reference's eager ops on
the served path (``model/reference.py:31-48,131-139``, ``model/blocks.py:470-490``,
``inference/models/atma.py:227-252,625-673``), rounding where that chain rounds.
Inference only (no autograd), 16-bit tensors on the GPU, graph capturable.
"""

import torch

from .. import _lib

_DT = (torch.bfloat16, torch.float16)


def _gpu16(*ts):
    for t in ts:
        if t is not None and (not t.is_cuda or t.dtype not in _DT):
            raise ValueError("layer fusions take 16-bit GPU tensors")


@torch.no_grad()
def head_rms_norm(x, eps):
    """``F.rms_norm(x, (d,), eps=eps)`` over the last dim of a (..., H, d) view with unit inner
    stride whose leading dims flatten to rows (e.g. the q half of every head of the q|gate
    projection, read in place).  d 64 or 128.  Returns a contiguous (..., H, d) tensor."""
    _gpu16(x)
    H, d = x.shape[-2:]
    if d not in (64, 128) or x.stride(-1) != 1:
        raise ValueError(f"head_rms_norm: heads of 64 or 128 with unit inner stride, got {tuple(x.shape)}")
    xr = x.view(-1, H, d) if x.dim() > 2 else x.view(1, H, d)
    out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    rc = _lib.load().atma_head_rms_norm(xr.data_ptr(), xr.stride(0), xr.stride(1), out.data_ptr(), xr.shape[0], H, d,
                                        float(eps), _lib.dtype_code(x.dtype), _lib.stream_handle(x.device))
    _lib.check(rc, "head_rms_norm")
    return out


@torch.no_grad()
def global_gate(c, gate, r, mem_gate, mem_eps):
    """The global layer's two gated projection inputs, rows m = b T + t:
    ``xa = (c * sigmoid(gate)).reshape(rows, H d)`` and
    ``xm = (rms_norm(r).to(dtype) * sigmoid(mem_gate.view(rows, H, d))).reshape(rows, H d)``.
    c: (B, T, H, d) view (Polar's head-major output transposed, or (1, tokens, H, d));
    gate: (rows, H, d) view; r: (rows, H, d) fp32 or c's dtype (heads contiguous) or None; mem_gate:
    (rows, H d).  Returns (xa, xm or None)."""
    _gpu16(c, gate, mem_gate)
    B, T, H, d = c.shape
    rows = B * T
    if gate.shape != (rows, H, d) or gate.stride(2) != 1 or c.stride(3) != 1 or gate.dtype != c.dtype:
        raise ValueError("global_gate: gate (rows, H, d) and c (B, T, H, d) with unit inner strides")
    xa = torch.empty((rows, H * d), device=c.device, dtype=c.dtype)
    xm = None
    if r is not None:
        if r.dtype not in (torch.float32, c.dtype) or r.shape != (rows, H, d) or r.stride(2) != 1 or r.stride(1) != d:
            raise ValueError("global_gate: r must be fp32 or c's dtype, (rows, H, d) with contiguous heads")
        if mem_gate.shape != (rows, H * d) or mem_gate.stride(1) != 1 or mem_gate.dtype != c.dtype:
            raise ValueError("global_gate: mem_gate must be (rows, H d)")
        xm = torch.empty_like(xa)
    rc = _lib.load().atma_global_gate(
        c.data_ptr(), c.stride(0), c.stride(1), c.stride(2), T, gate.data_ptr(), gate.stride(0), gate.stride(1),
        _lib.ptr(r), 0 if r is None else r.stride(0), _lib.dtype_code(torch.float32 if r is None else r.dtype),
        _lib.ptr(mem_gate if r is not None else None),
        0 if r is None else mem_gate.stride(0), xa.data_ptr(), xa.stride(0), _lib.ptr(xm),
        0 if xm is None else xm.stride(0), rows, H, d, float(mem_eps), _lib.dtype_code(c.dtype),
        _lib.stream_handle(c.device))
    _lib.check(rc, "global_gate")
    return xa, xm


@torch.no_grad()
def lfm2_conv_packed(bcx, weight, state_table, token_seq_starts, token_seq_ends, token_seq_slots):
    """With ``b, c, x = bcx.chunk(3, -1)``: ``c * packed_causal_conv1d(b * x, weight, ...)`` in one
    launch over packed fresh sequences, each sequence's last K - 1 values of ``b * x`` written to
    its row of ``state_table`` (slots, D, K - 1).  bcx (tokens, 3 D) 16-bit; weight (D, K), K 3 or 4."""
    _gpu16(bcx, weight)
    total, D3 = bcx.shape
    D = D3 // 3
    K = weight.shape[1]
    if D3 != 3 * D or weight.shape[0] != D or not weight.is_contiguous() or bcx.stride(1) != 1:
        raise ValueError("lfm2_conv_packed: bcx (tokens, 3 D) and contiguous weight (D, K)")
    if state_table.shape[1:] != (D, K - 1) or not state_table.is_contiguous() or state_table.dtype != bcx.dtype:
        raise ValueError(f"lfm2_conv_packed: state_table must be contiguous (slots, {D}, {K - 1})")
    maps = [t.to(device=bcx.device, dtype=torch.int32).reshape(-1).contiguous()
            for t in (token_seq_starts, token_seq_ends, token_seq_slots)]
    if any(m.numel() != total for m in maps):
        raise ValueError("token maps must have one entry per token")
    out = torch.empty((total, D), device=bcx.device, dtype=bcx.dtype)
    rc = _lib.load().atma_lfm2_conv_packed(bcx.data_ptr(), bcx.stride(0), weight.data_ptr(), K, out.data_ptr(),
                                           out.stride(0), state_table.data_ptr(), state_table.stride(0),
                                           state_table.shape[0], *[m.data_ptr() for m in maps], total, D,
                                           _lib.dtype_code(bcx.dtype), _lib.stream_handle(bcx.device))
    _lib.check(rc, "lfm2_conv_packed")
    return out


def linear_gated_supported(rows, in_features, out_features, dtype):
    """Shapes ``linear_gated`` serves: 16-bit, K a multiple of 128, 2H rows with H a multiple
    of 128, at least 4,096 rows (fewer rows take the weight-streaming decode kernels)."""
    return (dtype in _DT and rows >= 4096 and in_features >= 128 and in_features % 128 == 0
            and out_features % 256 == 0 and out_features >= 256)


@torch.no_grad()
def linear_gated(x, weight, bias=None):
    """The MLP's first projection with its activation for many rows: ``a, gate =
    F.linear(x, weight, bias).chunk(2, -1)`` then ``squared_relu_gate(a, gate)`` in one kernel
    that never writes the 2H-wide projection.  x (M, K) with unit inner stride; weight (2H, K);
    bias (2H,) or None.  Equal to that chain up to the products' summation order (each
    projection value is one fp32 sum rounded once, as the vendor GEMM's)."""
    _gpu16(x, weight)
    if x.dim() != 2 or x.stride(1) != 1 or weight.dim() != 2 or weight.stride(1) != 1:
        raise ValueError("linear_gated: x (M, K) and weight (2H, K) with unit inner strides")
    M, K = x.shape
    H = weight.shape[0] // 2
    if weight.shape != (2 * H, K) or weight.dtype != x.dtype or (bias is not None and (
            bias.shape != (2 * H,) or bias.dtype != x.dtype)):
        raise ValueError(f"linear_gated: weight (2H, {K}) and bias (2H,) in x's dtype")
    b = None if bias is None else bias.contiguous()
    y = torch.empty((M, H), device=x.device, dtype=x.dtype)
    rc = _lib.load().atma_linear_gated(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), _lib.ptr(b),
                                       y.data_ptr(), y.stride(0), M, H, K, _lib.dtype_code(x.dtype),
                                       _lib.stream_handle(x.device))
    _lib.check(rc, "linear_gated")
    return y

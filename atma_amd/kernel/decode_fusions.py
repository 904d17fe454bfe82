"""Launch-count fusions of the served model's decode step, backed by libatma_hip.so.

A decode step pushes one token per sequence through every block; at 32 sequences each
kernel moves a few hundred KB, and a launch costs more than its memory traffic.  These
entry points replace chains of small launches with one each (C ABI
``atma_linear_tokens_multi``, ``atma_linear_tokens_gated``, ``atma_linear_tokens_conv``,
``atma_linear_tokens_chunks``,
``atma_residual_rms_norm``,
``atma_lfm2_conv_step``, ``atma_global_decode_prep``, ``atma_global_decode_gate``).
None has a reference counterpart: they are the engine's own compositions of the
reference's decode arithmetic (``inference/models/atma.py:546-713``), with its eager
roundings where the chain rounds in between.

Inference only: no autograd, 16-bit tensors on the GPU (the conv step also fp32),
graph capturable (no host synchronisation, no allocation beyond the outputs).
"""

import ctypes

import torch

from .. import _lib

_DT = (torch.bfloat16, torch.float16)


def _addr(ctype, values):
    arr = (ctype * len(values))(*values)
    return arr, ctypes.addressof(arr)


def _rows(t, what):
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{what} must be a 2-D tensor with unit inner stride, got {tuple(t.shape)} "
                         f"strides {t.stride()}")
    return t


def _contig_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("decode fusions run on the GPU (HIP) only")


class PartialSums:
    """A projection output not yet summed: a 16-bit ``base`` (M, N) or fp32 ``parts``
    (P, M, N) from ``linear_tokens_chunks``, plus ``biases`` (each (N,)) and an optional
    low-rank term ``mu_x @ mu_w.T`` (mu_x (M, k), mu_w (N, k), k 4, 8 or 16).
    ``residual_rms_norm`` adds it to the residual stream in the same launch (fp32, one
    rounding); ``materialize`` is the same sum in torch."""

    __slots__ = ("parts", "base", "biases", "mu_x", "mu_w", "dtype")

    def __init__(self, parts, biases=(), mu_x=None, mu_w=None, dtype=torch.bfloat16, base=None):
        if (parts is None) == (base is None):
            raise ValueError("PartialSums takes exactly one of parts / base")
        self.parts, self.base, self.biases, self.mu_x, self.mu_w = parts, base, tuple(biases), mu_x, mu_w
        self.dtype = dtype

    @property
    def shape(self):
        return self.parts.shape[1:] if self.parts is not None else self.base.shape

    def materialize(self):
        s = self.parts.sum(0) if self.parts is not None else self.base.float()
        for b in self.biases:
            s = s + b.float()
        if self.mu_x is not None:
            s = s + self.mu_x.float() @ self.mu_w.float().t()
        return s.to(self.dtype)


# --------------------------------------------------------------------------- projections
def linear_tokens_multi_supported(rows, in_features, out_features_list, dtype):
    return (dtype in _DT and 1 <= rows <= 32 and in_features in (256, 512, 1024, 2048)
            and 1 <= len(out_features_list) <= 8 and all(n >= 4 and n % 4 == 0 for n in out_features_list))


@torch.no_grad()
def linear_tokens_multi(x, weights, biases):
    """``torch.cat([F.linear(x, w, b) for w, b in zip(weights, biases)], -1)`` in one
    launch, without concatenating the weights: x (M, K), M <= 32, K in {256, 512, 1024,
    2048}; up to 8 weights (N_s, K) with N_s % 4 == 0; biases entries may be None."""
    _rows(x, "x")
    M, K = x.shape
    ns = [w.shape[0] for w in weights]
    if not linear_tokens_multi_supported(M, K, ns, x.dtype):
        raise ValueError(f"linear_tokens_multi: unsupported x {tuple(x.shape)} {x.dtype}, outputs {ns}")
    for w, b in zip(weights, biases):
        _rows(w, "weight")
        if w.shape[1] != K or w.dtype != x.dtype or (b is not None and (b.dtype != x.dtype or not b.is_contiguous())):
            raise ValueError("linear_tokens_multi: weights (N, K) and biases (N,) in x's dtype")
    _contig_cuda(x, *weights)
    y = torch.empty((M, sum(ns)), device=x.device, dtype=x.dtype)
    offs = [0]
    for n in ns[:-1]:
        offs.append(offs[-1] + n)
    esz = y.element_size()
    _w, pw = _addr(ctypes.c_void_p, [w.data_ptr() for w in weights])
    _lw, plw = _addr(ctypes.c_int64, [w.stride(0) for w in weights])
    _b, pb = _addr(ctypes.c_void_p, [None if b is None else b.data_ptr() for b in biases])
    _y, py = _addr(ctypes.c_void_p, [y.data_ptr() + o * esz for o in offs])
    _ly, ply = _addr(ctypes.c_int64, [y.stride(0)] * len(ns))
    _n, pn = _addr(ctypes.c_int64, ns)
    rc = _lib.load().atma_linear_tokens_multi(x.data_ptr(), x.stride(0), M, K, len(ns), pw, plw, pb, py, ply, pn,
                                              _lib.dtype_code(x.dtype), _lib.stream_handle(x.device))
    _lib.check(rc, "linear_tokens_multi")
    return y


def chunk_width(in_features):
    """The chunk width ``linear_tokens_chunks`` uses for a projection of in_features
    inputs: 1024 (four waves per workgroup) where that leaves at least four chunks, else
    256; None when in_features is no multiple of it or needs more than 8 chunks."""
    ck = 1024 if in_features >= 4096 else 256
    return ck if in_features % ck == 0 and in_features // ck <= 8 else None


@torch.no_grad()
def linear_tokens_gated(x, weight, bias=None):
    """The MLP's first projection with its activation: ``a, gate = F.linear(x, weight,
    bias).chunk(2, -1)`` then ``squared_relu_gate(a, gate)`` in one launch, the 2H-wide
    projection never written.  x (M, K), M <= 32, K in {256, 512, 1024, 2048}; weight
    (2H, K), H % 16 == 0.  Returns (M, H) in x's dtype, equal to that chain wherever the
    projections round alike."""
    _rows(x, "x")
    _rows(weight, "weight")
    M, K = x.shape
    H = weight.shape[0] // 2
    if x.dtype not in _DT or not 1 <= M <= 32 or K not in (256, 512, 1024, 2048) or weight.shape != (2 * H, K) \
            or H % 16 or weight.dtype != x.dtype or (bias is not None and (bias.shape != (2 * H,) or bias.dtype != x.dtype)):
        raise ValueError(f"linear_tokens_gated: unsupported x {tuple(x.shape)} {x.dtype}, weight {tuple(weight.shape)}")
    _contig_cuda(x, weight)
    b = None if bias is None else bias.contiguous()
    y = torch.empty((M, H), device=x.device, dtype=x.dtype)
    rc = _lib.load().atma_linear_tokens_gated(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                                              _lib.ptr(b), y.data_ptr(), y.stride(0), M, H, K,
                                              _lib.dtype_code(x.dtype), _lib.stream_handle(x.device))
    _lib.check(rc, "linear_tokens_gated")
    return y


def linear_tokens_conv_supported(x, weight, taps):
    M, K = x.shape if x.dim() == 2 else (0, 0)
    H = taps.shape[0]
    return (x.dtype in _DT and 1 <= M <= 32 and K in (256, 512, 1024, 2048) and H % 16 == 0 and H >= 16
            and weight.shape == (3 * H, K) and 2 <= taps.shape[1] <= 4)


@torch.no_grad()
def linear_tokens_conv(x, weight, bias, taps, slots, state_table):
    """The LFM2 block's in_proj and decode mixer in one launch: ``lfm2_conv_step(F.linear(x,
    weight, bias), taps, slots, state_table)``, bit for bit, the 3H-wide projection never
    written.  x (M, K), M <= 32, K in {256, 512, 1024, 2048}; weight (3H, K) -- b, c, x
    rows; bias (3H,) or None; taps (H, Kt) contiguous, 2 <= Kt <= 4; state_table (max_seqs,
    H, Kt - 1) contiguous, rows ``slots`` advanced in place.  Returns (M, H) in x's dtype."""
    _rows(x, "x")
    _rows(weight, "weight")
    M, K = x.shape
    H, Kt = taps.shape
    if not linear_tokens_conv_supported(x, weight, taps) or weight.dtype != x.dtype or taps.dtype != x.dtype \
            or not taps.is_contiguous() or (bias is not None and (bias.shape != (3 * H,) or bias.dtype != x.dtype)):
        raise ValueError(f"linear_tokens_conv: unsupported x {tuple(x.shape)} {x.dtype}, weight "
                         f"{tuple(weight.shape)}, taps {tuple(taps.shape)}")
    if state_table.shape[1:] != (H, Kt - 1) or state_table.dtype != x.dtype or not state_table.is_contiguous():
        raise ValueError(f"linear_tokens_conv: state_table must be contiguous (max_seqs, {H}, {Kt - 1}) in x's dtype")
    _contig_cuda(x, weight, taps, state_table)
    b = None if bias is None else bias.contiguous()
    slots = slots.to(device=x.device, dtype=torch.int64).reshape(M).contiguous()
    y = torch.empty((M, H), device=x.device, dtype=x.dtype)
    rc = _lib.load().atma_linear_tokens_conv(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                                             _lib.ptr(b), taps.data_ptr(), Kt, slots.data_ptr(),
                                             state_table.data_ptr(), state_table.stride(0), state_table.shape[0],
                                             y.data_ptr(), y.stride(0), M, H, K, _lib.dtype_code(x.dtype),
                                             _lib.stream_handle(x.device))
    _lib.check(rc, "linear_tokens_conv")
    return y


@torch.no_grad()
def linear_tokens_chunks(x, weights, chunk_k):
    """fp32 partial products ``parts[c] = X_c @ weights[c].T`` (C, M, N) where X_c is
    columns [c chunk_k, (c + 1) chunk_k) of x.  weights[c]: (N, chunk_k) with unit inner
    stride (slices of one weight matrix are fine).  No bias: the consumer adds it."""
    _rows(x, "x")
    M = x.shape[0]
    C = len(weights)
    N = weights[0].shape[0]
    if x.dtype not in _DT or not 1 <= M <= 32 or chunk_k not in (256, 512, 1024) or not 1 <= C <= 8 \
            or N % 4 or x.shape[1] < C * chunk_k:
        raise ValueError(f"linear_tokens_chunks: unsupported x {tuple(x.shape)} {x.dtype}, {C} chunks of "
                         f"{chunk_k} -> {N}")
    for w in weights:
        _rows(w, "weight")
        if w.shape != (N, chunk_k) or w.dtype != x.dtype:
            raise ValueError("linear_tokens_chunks: every chunk weight must be (N, chunk_k) in x's dtype")
    _contig_cuda(x, *weights)
    parts = torch.empty((C, M, N), device=x.device, dtype=torch.float32)
    _w, pw = _addr(ctypes.c_void_p, [w.data_ptr() for w in weights])
    _lw, plw = _addr(ctypes.c_int64, [w.stride(0) for w in weights])
    rc = _lib.load().atma_linear_tokens_chunks(x.data_ptr(), x.stride(0), M, chunk_k, C, pw, plw, N,
                                               parts.data_ptr(), _lib.dtype_code(x.dtype),
                                               _lib.stream_handle(x.device))
    _lib.check(rc, "linear_tokens_chunks")
    return parts


# --------------------------------------------------------------------------- residual stream
def residual_rms_norm_supported(x):
    D = x.shape[-1]
    return x.is_cuda and x.dtype in _DT and D % 8 == 0 and 8 <= D <= 4096


@torch.no_grad()
def residual_rms_norm(branch, residual, weight, eps):
    """The pre-norm block's ``s = residual + branch; return rms_norm(s) * weight, s`` in
    one launch (each sum rounded to the stream's dtype as the eager add rounds it).
    ``branch``: (M, D) tensor or ``PartialSums`` (summed in fp32 with its biases and
    low-rank term, rounded once); ``residual`` None starts the stream with the branch.
    Returns (normed (M, D), stream (M, D))."""
    ps = branch if isinstance(branch, PartialSums) else None
    parts = ps.parts if ps is not None else None
    y = branch if ps is None else ps.base
    dtype = branch.dtype
    if y is not None:
        _rows(y, "branch")
    M, D = (parts.shape[1], parts.shape[2]) if parts is not None else y.shape
    if dtype not in _DT or D % 8 or not 8 <= D <= 4096 or weight.shape != (D,) or weight.dtype != dtype:
        raise ValueError(f"residual_rms_norm: unsupported rows of {D} {dtype}")
    if residual is not None:
        _rows(residual, "residual")
        if residual.shape != (M, D) or residual.dtype != dtype:
            raise ValueError("residual_rms_norm: residual must match the branch")
    out = torch.empty((M, D), device=weight.device, dtype=dtype)
    new_res = branch if (residual is None and ps is None) else torch.empty_like(out)
    if parts is not None and (not parts.is_contiguous() or parts.dtype != torch.float32):
        raise ValueError("residual_rms_norm: parts must be contiguous fp32 (P, M, D)")
    biases = [b.contiguous() for b in ps.biases] if ps is not None else []
    _b, pb = _addr(ctypes.c_void_p, [b.data_ptr() for b in biases] or [None])
    mu_x = ps.mu_x if ps is not None else None
    mu_w = None
    if mu_x is not None:
        _rows(mu_x, "mu_x")
        mu_w = ps.mu_w.contiguous()
    rc = _lib.load().atma_residual_rms_norm(
        _lib.ptr(y), 0 if y is None else y.stride(0), _lib.ptr(parts), 0 if parts is None else parts.shape[0],
        pb, len(biases), _lib.ptr(mu_x), 0 if mu_x is None else mu_x.stride(0), _lib.ptr(mu_w),
        0 if mu_x is None else mu_x.shape[1], _lib.ptr(residual), 0 if residual is None else residual.stride(0),
        None if new_res is branch else new_res.data_ptr(), new_res.stride(0), weight.data_ptr(),
        out.data_ptr(), out.stride(0), M, D, float(eps), _lib.dtype_code(dtype), _lib.stream_handle(weight.device))
    _lib.check(rc, "residual_rms_norm")
    return out, new_res


# --------------------------------------------------------------------------- mixers
@torch.no_grad()
def lfm2_conv_step(bcx, weight, slots, state_table):
    """The LFM2 block's decode mixer input to out_proj: with ``b, c, x = bcx.chunk(3, -1)``,
    ``c * conv(b * x)`` for one token per sequence, the depthwise conv's last K - 1 inputs
    per sequence in ``state_table`` (max_seqs, D, K - 1), advanced in place (rows
    ``slots``).  bcx (B, 3 D); weight (D, K)."""
    _rows(bcx, "bcx")
    B, D3 = bcx.shape
    D = D3 // 3
    K = weight.shape[1]
    if D3 != 3 * D or weight.shape[0] != D or weight.dtype != bcx.dtype or not weight.is_contiguous():
        raise ValueError("lfm2_conv_step: bcx (B, 3 D) and contiguous weight (D, K) in one dtype")
    if K > 1 and (state_table.shape[1:] != (D, K - 1) or state_table.dtype != bcx.dtype
                  or not state_table.is_contiguous()):
        raise ValueError(f"lfm2_conv_step: state_table must be contiguous (max_seqs, {D}, {K - 1}) in bcx's dtype")
    slots = slots.to(device=bcx.device, dtype=torch.int64).reshape(B).contiguous()
    out = torch.empty((B, D), device=bcx.device, dtype=bcx.dtype)
    rc = _lib.load().atma_lfm2_conv_step(bcx.data_ptr(), bcx.stride(0), weight.data_ptr(), K, slots.data_ptr(),
                                         state_table.data_ptr(), state_table.stride(0), state_table.shape[0],
                                         out.data_ptr(), out.stride(0), B, D, _lib.dtype_code(bcx.dtype),
                                         _lib.stream_handle(bcx.device))
    _lib.check(rc, "lfm2_conv_step")
    return out


@torch.no_grad()
def global_decode_prep(y, H, Hkv, d, cols, canon, tables, slots, eps, gate_bias=None):
    """q, k, v (and the memory gates) of the global layer's decode step from its fused
    input projection ``y`` (B, W): per head ``rms_norm`` of q and k (eps ``eps``), Canon
    residual convs of q / k / v with their state tables advanced in place, and
    ``gamma = sigmoid(z_g + bias_g)``, ``beta = sigmoid(z_b + bias_b)`` (fp32).
    cols: (ck, cv, cg, cb) column offsets of k, v and the two gate logits in y (q and its
    output gate interleave per head from column 0); canon / tables: (q, k, v) taps
    (C, Kc) and tables (max_seqs, C, Kc - 1).  gate_bias None: no memory gates."""
    _rows(y, "y")
    B = y.shape[0]
    ck, cv, cg, cb = cols
    Kc = canon[0].shape[1]
    for w, t, C in zip(canon, tables, (H * d, Hkv * d, Hkv * d)):
        if w.shape != (C, Kc) or not w.is_contiguous() or w.dtype != y.dtype:
            raise ValueError("global_decode_prep: Canon taps must be contiguous (C, Kc) in y's dtype")
        if Kc > 1 and (t.shape[1:] != (C, Kc - 1) or not t.is_contiguous() or t.dtype != y.dtype):
            raise ValueError("global_decode_prep: Canon tables must be contiguous (max_seqs, C, Kc - 1)")
    slots = slots.to(device=y.device, dtype=torch.int64).reshape(B).contiguous()
    q = torch.empty((B, H, d), device=y.device, dtype=y.dtype)
    k = torch.empty((B, Hkv, d), device=y.device, dtype=y.dtype)
    v = torch.empty_like(k)
    gamma = beta = None
    if gate_bias is not None:
        gamma = torch.empty((B, H), device=y.device, dtype=torch.float32)
        beta = torch.empty_like(gamma)
    tq, tk, tv = tables
    rc = _lib.load().atma_global_decode_prep(
        y.data_ptr(), y.stride(0), ck, cv, cg if gamma is not None else -1, cb if gamma is not None else -1,
        canon[0].data_ptr(), canon[1].data_ptr(), canon[2].data_ptr(), Kc, tq.data_ptr(), tq.stride(0),
        tk.data_ptr(), tk.stride(0), tv.data_ptr(), tv.stride(0), tq.shape[0], slots.data_ptr(), q.data_ptr(),
        k.data_ptr(), v.data_ptr(), _lib.ptr(gamma), _lib.ptr(beta), float(eps),
        float(gate_bias[0]) if gate_bias is not None else 0.0, float(gate_bias[1]) if gate_bias is not None else 0.0,
        B, H, Hkv, d, _lib.dtype_code(y.dtype), _lib.stream_handle(y.device))
    _lib.check(rc, "global_decode_prep")
    return q, k, v, gamma, beta


@torch.no_grad()
def global_decode_gate(c, r, y, mem_gate_col, mem_eps):
    """The gated inputs of the global layer's output projections, side by side:
    ``[c * sigmoid(gate) | rms_norm(r) * sigmoid(mem_gate)]`` (B, 2 H d), or only the
    first half when ``r`` is None.  c (B, H, d); r (B, H, d) fp32 memory readout; y the
    fused input projection (the output gate of head h at columns h 2d + d, the memory
    gate at ``mem_gate_col`` + h d)."""
    _rows(y, "y")
    B, H, d = c.shape
    c = c.contiguous()
    if r is not None:
        r = r.contiguous()
        if r.dtype != torch.float32 or r.shape != c.shape:
            raise ValueError("global_decode_gate: r must be fp32 (B, H, d)")
    x2 = torch.empty((B, (2 if r is not None else 1) * H * d), device=c.device, dtype=c.dtype)
    rc = _lib.load().atma_global_decode_gate(c.data_ptr(), _lib.ptr(r), y.data_ptr(), y.stride(0),
                                             mem_gate_col if r is not None else -1, x2.data_ptr(), x2.stride(0),
                                             float(mem_eps), B, H, d, _lib.dtype_code(c.dtype),
                                             _lib.stream_handle(c.device))
    _lib.check(rc, "global_decode_gate")
    return x2

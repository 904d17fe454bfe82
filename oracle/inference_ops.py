"""CPU oracle for the inference fusions (test infrastructure only; see ``oracle/__init__``).

numpy restatements of ``kernel/inference_ops_triton.py``: every arithmetic step in the
reference kernel's order, in float32, with bf16 rounding (round to nearest even) applied
exactly where the reference rounds.  Inputs and outputs are torch CPU tensors.
"""

import numpy as np
import torch


def _f32(t):
    return t.detach().to(torch.float32).numpy()


def round_bf16(a):
    """float32 -> nearest bf16 (ties to even), returned as float32; NaN stays NaN."""
    a = np.asarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, r).astype(np.float32)


def _out(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dtype)


def squared_relu_gate(x, gate):
    """``_squared_relu_gate_kernel`` (``kernel/inference_ops_triton.py:102-120``):
    ``pos = max(x, 0)``, ``square = pos * pos`` (rounded to bf16 for bf16 inputs),
    ``out = gate * square`` in fp32, stored in x's dtype.  NaN inputs stay NaN, as
    torch's relu (the reference test's eager form, ``tests/test_decode_kernels.py:62``)."""
    xf, gf = _f32(x), _f32(gate)
    with np.errstate(over="ignore", invalid="ignore"):   # inf / NaN inputs propagate as IEEE says
        pos = np.where(xf < 0, np.float32(0), xf).astype(np.float32)
        sq = (pos * pos).astype(np.float32)
        if x.dtype == torch.bfloat16:
            sq = round_bf16(sq)
        return _out(gf * sq, x.dtype)


def softcap_logits(logits):
    """``_softcap_kernel`` (``kernel/inference_ops_triton.py:194-211``):
    ``left = 15 x``, ``square = x x`` (both rounded to bf16 for bf16), ``denom = square +
    225`` (rounded), ``inv = 1 / sqrt(denom)`` (rounded), ``out = left * inv``.  The
    reciprocal square root is the correctly rounded ``1 / sqrt`` in float32."""
    x = _f32(logits)
    bf = logits.dtype == torch.bfloat16
    rnd = round_bf16 if bf else (lambda a: np.asarray(a, dtype=np.float32))
    with np.errstate(over="ignore", invalid="ignore"):   # huge inputs overflow to inf as IEEE says
        left = rnd(np.float32(15) * x)
        square = rnd(x * x)
        denom = rnd(square + np.float32(225))
        inv = rnd(np.float32(1) / np.sqrt(denom))
        return _out(left * inv, logits.dtype)


def _fma32(a, b, c):
    """fp32 fused multiply-add: the product is exact in float64, the sum rounds once
    there and once more to float32 (equal to a true fma except on exact float32 ties of
    an inexact float64 sum, which the tests' inputs do not produce in practice)."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def packed_causal_conv1d(x, weight, state_table, token_seq_starts, token_seq_ends, token_seq_slots):
    """``_packed_causal_conv1d_kernel`` (``kernel/inference_ops_triton.py:17-63``):
    ``acc = 0; for j < K: acc += x[t - (K-1-j)] * w[:, j]`` over sources at or after the
    token's sequence start (fma in tap order, fp32), stored in x's dtype; the last token
    of each sequence writes ``state[slot, :, j] = x[end - (K-1) + j]`` (0 before the start).
    ``state_table`` is updated IN PLACE.  Returns (tokens, channels) in x's dtype."""
    xf = _f32(x)
    wf = _f32(weight)
    T, C = xf.shape
    K = wf.shape[1]
    st = token_seq_starts.long().numpy()
    en = token_seq_ends.long().numpy()
    sl = token_seq_slots.long().numpy()
    acc = np.zeros((T, C), dtype=np.float32)
    t = np.arange(T)
    for j in range(K):
        src = t - (K - 1 - j)
        live = src >= st
        xv = np.where(live[:, None], xf[np.clip(src, 0, None)], np.float32(0)).astype(np.float32)
        acc = _fma32(xv, np.broadcast_to(wf[:, j], (T, C)), acc)
    for tt in np.nonzero(t == en - 1)[0]:
        slot = int(sl[tt])
        if not 0 <= slot < state_table.shape[0]:
            continue
        for j in range(K - 1):
            src = int(en[tt]) - (K - 1) + j
            row = torch.from_numpy(xf[src]) if src >= st[tt] else torch.zeros(C)
            state_table[slot, :, j] = row.to(state_table.dtype)
    return _out(acc, x.dtype)

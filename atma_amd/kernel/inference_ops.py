"""Forward-only fusions of the paged inference model, backed by libatma_hip.so.

Mirrors ``kernel/inference_ops_triton.py`` of the reference (same names, arguments and
errors): ``squared_relu_gate`` (:123-135, the MLP activation of
``inference/models/atma.py:87-96``), ``softcap_logits`` (:214-223, the output soft cap of
``inference/models/atma.py:750-754``) and ``packed_causal_conv1d`` (:138-160, the grouped
fresh prefill's depthwise convolutions, ``inference/models/atma.py:431-442, 648-652``);
``softcap_argmax`` is the soft cap fused with the greedy sampler's argmax.
The prototype ``linear_head_rms`` (:163-189) is not part of the served path and is not
provided.  ``linear_tokens`` has no counterpart there: the served model's projection of a
few token rows (one per decoding sequence), where the reference calls the vendor GEMM.
"""

import torch

from .. import _lib
from .. import _ops  # noqa: F401  (registers torch.ops.atma_hip.*)


@torch.no_grad()
def squared_relu_gate(x, gate):
    """Fused gate * relu(x)^2, preserving eager BF16's intermediate rounding.

    x, gate: (rows, width) (strided views such as the two halves of one fc output are
    read in place).  Returns a contiguous (rows, width) tensor in x's dtype."""
    if x.dim() != 2 or gate.shape != x.shape:
        raise ValueError("expected x and gate of the same [rows, width] shape")
    if gate.dtype != x.dtype:
        raise ValueError("x and gate must share a dtype")
    return torch.ops.atma_hip.squared_relu_gate(x, gate)


@torch.no_grad()
def softcap_logits(logits):
    """Fuse the elementwise 15*x/sqrt(x^2+225) output soft cap (any shape, logits' dtype)."""
    return torch.ops.atma_hip.softcap_logits(logits)


@torch.no_grad()
def softcap_argmax(logits, ids_out=None):
    """``capped = softcap_logits(logits)`` and ``capped.float().argmax(-1)`` in one launch
    (one workgroup per row): the decode step's soft cap and greedy pick.  logits (rows,
    V) 16-bit.  Returns (capped (rows, V), ids (rows,) int64); with ``ids_out`` (a
    contiguous int64 (rows,) tensor, inference only) the ids are written there.
    No counterpart in the reference's op set (its sampler takes the argmax in torch)."""
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("expected logits [rows, vocab] with unit inner stride")
    if logits.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("softcap_argmax takes 16-bit logits")
    if ids_out is None:
        return torch.ops.atma_hip.softcap_argmax(logits)
    rows, V = logits.shape
    if ids_out.shape != (rows,) or ids_out.dtype != torch.int64 or not ids_out.is_contiguous() \
            or ids_out.device != logits.device:
        raise ValueError(f"ids_out must be a contiguous int64 ({rows},) tensor on the logits' device")
    if not logits.is_cuda:
        raise RuntimeError("softcap_argmax requires a GPU (HIP)")
    out = torch.empty((rows, V), device=logits.device, dtype=logits.dtype)
    rc = _lib.load().atma_softcap_argmax(logits.data_ptr(), logits.stride(0), out.data_ptr(), out.stride(0),
                                         ids_out.data_ptr(), rows, V, _lib.dtype_code(logits.dtype),
                                         _lib.stream_handle(logits.device))
    _lib.check(rc, "softcap_argmax")
    return out, ids_out


@torch.no_grad()
def packed_causal_conv1d(x, weight, state_table, token_seq_starts, token_seq_ends, token_seq_slots):
    """Fresh causal depthwise convolution over packed variable-length sequences.

    x: (tokens, channels); weight: (channels, kernel) with kernel 3 or 4 (ATMA's sizes);
    state_table: (slots, channels, kernel - 1), updated IN PLACE with each sequence's last
    kernel - 1 inputs; token_seq_starts / ends / slots: (tokens,) int32 per-token maps.
    Returns the convolution (tokens, channels) in x's dtype."""
    if not x.is_cuda:
        raise RuntimeError("packed_causal_conv1d requires a GPU (HIP)")
    if x.ndim != 2 or weight.ndim != 2 or weight.shape[0] != x.shape[1]:
        raise ValueError("expected x [tokens, channels], weight [channels, kernel]")
    kernel_size = weight.shape[1]
    if kernel_size not in (3, 4):
        raise ValueError("packed convolution supports ATMA kernel sizes 3 and 4")
    if state_table.dim() != 3 or state_table.shape[1:] != (x.shape[1], kernel_size - 1):
        raise ValueError(f"state_table {tuple(state_table.shape)} must be (slots, {x.shape[1]}, "
                         f"{kernel_size - 1})")
    maps = [t.to(device=x.device, dtype=torch.int32).reshape(-1).contiguous()
            for t in (token_seq_starts, token_seq_ends, token_seq_slots)]
    if any(m.numel() != x.shape[0] for m in maps):
        raise ValueError("token maps must have one entry per token")
    weight = weight.to(dtype=x.dtype)
    return torch.ops.atma_hip.packed_causal_conv1d(x, weight, state_table, *maps)


def linear_tokens_supported(rows, out_features, in_features, dtype):
    """True for the shapes ``linear_tokens`` serves: 16-bit, at most 32 rows, out_features a
    multiple of 16 and in_features 256, 512, 1024 or 2048 (the C ABI's
    ``atma_linear_tokens_supported``: one wave per 256 inputs, at most eight per workgroup;
    a wider input is split across workgroups by ``linear_tokens_chunks`` instead)."""
    return (dtype in (torch.bfloat16, torch.float16) and 1 <= rows <= 32 and out_features >= 16
            and out_features % 16 == 0 and in_features in (256, 512, 1024, 2048))


@torch.no_grad()
def linear_tokens(x, weight, bias=None):
    """``F.linear(x, weight, bias)`` for x (rows, in_features) with rows <= 32: the weights
    are streamed once (one workgroup per 16 output features, 32 for wide outputs, K split
    256 per wave, fp32 accumulation, one rounding).  Deterministic."""
    if x.dim() != 2 or weight.dim() != 2 or weight.shape[1] != x.shape[1]:
        raise ValueError("expected x [rows, in_features], weight [out_features, in_features]")
    if not linear_tokens_supported(x.shape[0], weight.shape[0], x.shape[1], x.dtype):
        raise ValueError(f"linear_tokens: unsupported shape {tuple(x.shape)} x {tuple(weight.shape)} {x.dtype}")
    if weight.dtype != x.dtype or (bias is not None and bias.dtype != x.dtype):
        raise ValueError("x, weight and bias must share a dtype")
    return torch.ops.atma_hip.linear_tokens(x, weight, bias)

"""Decode-time causal convolution step backed by libatma_hip.so.

``causal_conv1d_decode_step`` mirrors ``kernel/causal_conv1d_triton.py:46-63``: one
depthwise convolution step per sequence with the slot-indexed state of the last K - 1
inputs advanced in place (the global layer's Canon q / k / v convolutions at decode,
``inference/models/atma.py:160-192``).
"""

import torch

from .. import _ops  # noqa: F401  (registers torch.ops.atma_hip.*)


@torch.no_grad()
def causal_conv1d_decode_step(x, weight, slots, state_table, residual=False):
    """x: (B, D); weight: (D, K) depthwise taps (cast to x's dtype); slots: (B,) rows of
    ``state_table`` (max_seqs, D, K - 1) in x's dtype, advanced IN PLACE.  Returns the
    convolution output (B, D) in x's dtype; ``residual=True`` (an extension) returns
    ``x + conv`` in the same launch, the layer's residual Canon form.  K = 1 touches no
    state, as the reference's early return (``:50-51``).  Graph capturable."""
    if x.dim() != 2 or weight.dim() != 2 or weight.shape[0] != x.shape[1]:
        raise ValueError("x must be (B, D) and weight (D, K)")
    B, D = x.shape
    K = weight.shape[1]
    if K > 1 and (state_table.dim() != 3 or state_table.shape[1] != D or state_table.shape[2] != K - 1):
        raise ValueError(f"state_table {tuple(state_table.shape)} must be (max_seqs, {D}, {K - 1})")
    if K > 1 and state_table.dtype != x.dtype:
        raise ValueError("state_table must have x's dtype")
    weight = weight.to(dtype=x.dtype)
    slots = slots.to(device=x.device, dtype=torch.int64).reshape(B).contiguous()
    return torch.ops.atma_hip.causal_conv1d_decode_step(x, weight, slots, state_table, bool(residual))

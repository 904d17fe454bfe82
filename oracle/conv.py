"""CPU oracle for the decode-time causal convolution step (test infrastructure only;
see ``oracle/__init__``)."""

import torch


def causal_conv1d_decode_step(x, weight, slots, state_table):
    """One depthwise causal-convolution step per sequence, state advanced IN PLACE.

    The reference's torch route ``_gpu_conv_step`` (``inference/models/atma.py:181-188``),
    the same contract as ``kernel/causal_conv1d_triton.py:18-63``: gather the (B, D, K-1)
    state rows, ``out = sum_j state[:, :, j] * w[:, j] + x * w[:, K-1]``, then the rows
    become ``(state[:, :, 1:], x)``.  Computed in x's dtype promoted to at least fp32.
    Returns the convolution output (B, D) (no residual)."""
    K = weight.shape[1]
    ct = torch.promote_types(x.dtype, torch.float32)
    w = weight.to(ct)
    if K < 2:
        return x.to(ct) * w[:, 0]
    idx = slots.long()
    states = state_table[idx].to(ct)                        # (B, D, K-1) gather
    out = (states * w[:, :-1].unsqueeze(0)).sum(2) + x.to(ct) * w[:, -1].unsqueeze(0)
    new_state = torch.cat([state_table[idx][:, :, 1:], x.to(state_table.dtype).unsqueeze(2)], dim=2)
    state_table[idx] = new_state                            # (B, D, K-1) scatter
    return out

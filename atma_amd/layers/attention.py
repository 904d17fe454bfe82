"""Paged KV write and the per-layer cache holder, mirroring
``inference/layers/attention.py`` of the reference."""

import torch
from torch import nn

from .. import _ops  # noqa: F401  (registers torch.ops.atma_hip.*)


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor):
    """Write (N, Hkv, d) key/value rows into paged KV cache slots, in place.

    Mirrors ``store_kvcache`` (``inference/layers/attention.py:30-56``): row i goes to
    flat cache row ``slot_mapping[i]`` (= page * page_size + offset), bit for bit;
    ``-1`` (any negative slot) is skipped.  Same layout assertions as the reference."""
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert slot_mapping.numel() == N
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    if key.dtype != k_cache.dtype or value.dtype != v_cache.dtype:
        raise ValueError("key/value dtype must match the cache dtype (bitwise copy)")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache / v_cache must be contiguous")
    if slot_mapping.dtype != torch.int32:
        slot_mapping = slot_mapping.to(torch.int32)
    torch.ops.atma_hip.store_kvcache(key, value, k_cache, v_cache, slot_mapping.contiguous())


class Attention(nn.Module):
    """Holds a layer's paged KV cache references and attention scale
    (``inference/layers/attention.py:59-73``)."""

    def __init__(self, num_heads: int, head_dim: int, scale: float, num_kv_heads: int):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = torch.tensor([])
        self.v_cache = torch.tensor([])

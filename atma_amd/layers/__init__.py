"""Host-side layers of the global-layer mixer: the paged KV write and cache holder
(``attention``) and the Polar + gated-delta mixer module with its prefill / decode
routes (``global_attention``)."""

from .attention import Attention, store_kvcache
from .global_attention import GlobalBlock, GlobalLayerCache, PolarAttention, TitansMemory

__all__ = ["Attention", "store_kvcache", "PolarAttention", "TitansMemory", "GlobalLayerCache",
           "GlobalBlock"]

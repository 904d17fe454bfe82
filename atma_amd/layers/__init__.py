"""Host-side layers of the global-layer mixer: the paged KV write and cache holder
(``attention``) and the Polar + gated-delta mixer module with its prefill / decode
routes (``global_attention``), and checkpoint loading in the reference's format
(``loader``)."""

from .attention import Attention, store_kvcache
from .global_attention import GlobalBlock, GlobalLayerCache, PolarAttention, TitansMemory
from .loader import load_model, save_checkpoint

__all__ = ["Attention", "store_kvcache", "PolarAttention", "TitansMemory", "GlobalLayerCache",
           "GlobalBlock", "load_model", "save_checkpoint"]

"""Model and engine configuration (``model/config.py:6-53``, ``inference/config.py:6-19``).

``AtmaConfig`` keeps the reference's field names and defaults that shape the served
model; ``Config`` is the engine's.  ``attn_window`` defaults to None here: the served
configuration of BASELINE configs[4] is full context (the reference's training default
is 1024)."""

from dataclasses import dataclass, field
from typing import Optional

import torch


@dataclass
class AtmaConfig:
    vocab_size: int = 50304
    num_hidden_layers: int = 16
    hidden_size: int = 1024
    head_dim: int = 128
    attn_kernel_size: int = 4
    conv_kernel_size: int = 3
    rms_norm_eps: float = 1e-6
    dtype: torch.dtype = torch.bfloat16
    attn_window: Optional[int] = None
    mem_enabled: bool = True
    mem_chunk: int = 64
    mem_gamma_bias: float = 3.9
    mem_beta_bias: float = 0.0

    @property
    def num_attention_heads(self) -> int:
        return self.hidden_size // self.head_dim

    @property
    def num_key_value_heads(self) -> int:
        return self.num_attention_heads // 4   # GQA 1:4 (model/config.py:51-53)

    @staticmethod
    def is_attention_layer(i: int) -> bool:
        """Local-Local-Global-Local: block i is a global (Polar + memory) block when
        i % 4 == 2 (``model/reference.py:245``)."""
        return i % 4 == 2


@dataclass
class Config:
    model: str = ""                         # checkpoint path ("" = random init)
    kvcache_block_size: int = 256
    gpu_memory_utilization: float = 0.9
    max_num_seqs: int = 2048
    max_num_batched_tokens: int = 16384 * 8
    max_model_len: int = 4096
    enforce_eager: bool = False
    strict_weights: bool = False
    eos: int = 50256
    num_kvcache_blocks: int = -1            # -1: enough for max_num_seqs x max_model_len, within memory
    init_std: float = 0.02                  # random init N(0, init_std) of every parameter
    seed: int = 0
    hf_config: AtmaConfig = field(default_factory=AtmaConfig)

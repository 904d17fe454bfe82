"""Thread-local forward context of the paged engine (``inference/utils/context.py:4-122``).

The model runner sets it before each forward; the layers read the routing decision
(dense / grouped / per-sequence prefill, or decode), the paged-cache maps and the
per-sequence state tables from it.  Same fields and semantics as the reference."""

import threading
from dataclasses import dataclass, field
from typing import Any, Optional


@dataclass
class Context:
    is_prefill: bool
    cu_seqlens_q: Any = None
    cu_seqlens_k: Any = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: Any = None
    context_lens: Any = None
    block_tables: Any = None
    seqlens_q: list = field(default_factory=list)
    context_lens_list: list = field(default_factory=list)
    conv_state_tables: Optional[dict] = None      # attn_{i}_{q,k,v}, conv_{i}_gated, mem_{i}
    seq_slots: Any = None                         # (bs,) int64 rows of the state tables
    dense_prefill: bool = False                   # fresh, complete, equal-length prompts
    dense_batch_size: int = 0
    dense_seq_len: int = 0
    grouped_polar_prefill: bool = False           # fresh ragged prompts, one tile-mapped launch
    polar_tile_seq_starts: Any = None
    polar_tile_q_starts: Any = None
    polar_tile_seq_lens: Any = None
    token_seq_starts: Any = None
    token_seq_ends: Any = None
    token_seq_slots: Any = None
    seqs: list = field(default_factory=list)      # the scheduled sequences (host objects)


_local = threading.local()


def set_context(is_prefill: bool, **kwargs) -> Context:
    _local.context = Context(is_prefill=is_prefill, **kwargs)
    return _local.context


def get_context() -> Context:
    ctx = getattr(_local, "context", None)
    if ctx is None:
        raise RuntimeError("No context has been set. Call set_context before running model layers.")
    return ctx


def reset_context():
    if hasattr(_local, "context"):
        del _local.context

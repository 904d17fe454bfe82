"""The gated-delta ops under the reference's module name ``kernel/gated_delta_triton.py``
(``gated_delta_decode_step``, ``kernel/gated_delta_triton.py:78-117``), plus the chunked
prefill ``chunk_gated_delta_rule`` that replaces the third-party
``fla.ops.gated_delta_rule`` import (``inference/models/atma.py:51-56``,
``model/blocks.py:23-30``).  ``HAS_TRITON`` keeps the reference's flag name.  Importing
raises ``ImportError`` when libatma_hip.so is absent."""

from . import HAS_HIP
from .gated_delta import chunk_gated_delta_rule, gated_delta_decode_step

HAS_TRITON = HAS_HIP

__all__ = ["gated_delta_decode_step", "chunk_gated_delta_rule", "HAS_TRITON"]

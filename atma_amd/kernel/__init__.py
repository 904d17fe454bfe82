"""Hot-path ops of ATMA's global-layer mixer under the reference's names
(``kernel/__init__.py:15-28`` of the reference), backed by libatma_hip.so.

``HAS_HIP`` mirrors the reference's ``HAS_TRITON``: True when the library is
built and a GPU is visible.  The functions are always importable; calling one
without the library or on CPU tensors raises (there is no silent fallback).
"""

import torch

from .. import _lib
from .conv import causal_conv1d_decode_step
from .inference_ops import packed_causal_conv1d, softcap_logits, squared_relu_gate
from .gated_delta import (StartSignal, chunk_gated_delta_rule, gated_delta_decode_step, gated_delta_gates,
                          recurrence_pays_to_overlap)
from .polar import polar_attention_decode, polar_attention_fwd, polar_attention_packed_fwd
from .polar_train import polar_attention

HAS_HIP = _lib.available() and torch.cuda.is_available()

__all__ = [
    "StartSignal",
    "recurrence_pays_to_overlap",
    "HAS_HIP",
    "polar_attention_fwd",
    "polar_attention",
    "polar_attention_packed_fwd",
    "polar_attention_decode",
    "gated_delta_decode_step",
    "chunk_gated_delta_rule",
    "gated_delta_gates",
    "causal_conv1d_decode_step",
    "squared_relu_gate",
    "softcap_logits",
    "packed_causal_conv1d",
]

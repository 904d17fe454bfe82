"""Hot-path ops of ATMA's global-layer mixer under the reference's names
(``kernel/__init__.py:15-28`` of the reference), backed by libatma_hip.so.

Importing this package loads the library.  Without it the import raises
``HipLibraryMissing``, an ``ImportError``: the reference's callers import their
kernels inside ``try/except`` and take their eager path on failure
(``inference/models/atma.py:31-80``, ``model/blocks.py:9-30``), and this package keeps
that contract.  There is no silent fallback inside: a CPU tensor raises.

``HAS_HIP`` (alias ``HAS_TRITON``, the reference's flag name) is True when a GPU is
visible.  The modules ``polar_triton``, ``gated_delta_triton``,
``causal_conv1d_triton`` and ``inference_ops_triton`` re-export the ops under the
reference's module names for a one-line import swap.
"""

import torch

from .. import _lib

_lib.load()   # raises HipLibraryMissing (ImportError) when the library is absent

from .conv import causal_conv1d_decode_step  # noqa: E402
from .inference_ops import (linear_tokens, linear_tokens_supported, packed_causal_conv1d,  # noqa: E402
                            softcap_argmax, softcap_logits, squared_relu_gate)
from .gated_delta import (StartSignal, chunk_gated_delta_rule, gated_delta_decode_step,  # noqa: E402
                          gated_delta_gates, recurrence_pays_to_overlap)
from .polar import (global_decode_step, global_decode_step_supported, polar_attention_decode,  # noqa: E402
                    polar_attention_fwd, polar_attention_packed_fwd)
from .polar_train import polar_attention  # noqa: E402

HAS_HIP = torch.cuda.is_available()
HAS_TRITON = HAS_HIP

__all__ = [
    "StartSignal",
    "recurrence_pays_to_overlap",
    "HAS_HIP",
    "HAS_TRITON",
    "polar_attention_fwd",
    "polar_attention",
    "polar_attention_packed_fwd",
    "polar_attention_decode",
    "global_decode_step",
    "global_decode_step_supported",
    "gated_delta_decode_step",
    "chunk_gated_delta_rule",
    "linear_tokens",
    "linear_tokens_supported",
    "gated_delta_gates",
    "causal_conv1d_decode_step",
    "squared_relu_gate",
    "softcap_logits",
    "softcap_argmax",
    "packed_causal_conv1d",
]

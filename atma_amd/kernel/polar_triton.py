"""The Polar ops under the reference's module name ``kernel/polar_triton.py``, so a
caller swaps one import line (``from kernel.polar_triton import ...`` ->
``from atma_amd.kernel.polar_triton import ...``).  The ops are the HIP kernels of
libatma_hip.so; ``HAS_TRITON`` keeps the reference's flag name (True when a GPU is
visible).  Importing raises ``ImportError`` when the library is absent, which the
reference's guarded imports (``inference/models/atma.py:31-39``) turn into their eager
path."""

from . import HAS_HIP
from .polar import polar_attention_decode, polar_attention_fwd, polar_attention_packed_fwd
from .polar_train import polar_attention

HAS_TRITON = HAS_HIP

__all__ = ["polar_attention", "polar_attention_fwd", "polar_attention_packed_fwd",
           "polar_attention_decode", "HAS_TRITON"]

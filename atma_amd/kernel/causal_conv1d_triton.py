"""The decode conv step under the reference's module name
``kernel/causal_conv1d_triton.py`` (``causal_conv1d_decode_step``, ``:46-63``).
``HAS_TRITON`` keeps the reference's flag name.  Importing raises ``ImportError`` when
libatma_hip.so is absent (the reference's guard, ``inference/models/atma.py:58-64``)."""

from . import HAS_HIP
from .conv import causal_conv1d_decode_step

HAS_TRITON = HAS_HIP

__all__ = ["causal_conv1d_decode_step", "HAS_TRITON"]

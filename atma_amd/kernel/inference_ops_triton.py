"""The inference fusions under the reference's module name
``kernel/inference_ops_triton.py`` (``squared_relu_gate``, ``softcap_logits``,
``packed_causal_conv1d``).  ``HAS_TRITON`` keeps the reference's flag name.  Importing
raises ``ImportError`` when libatma_hip.so is absent (the reference's guard,
``inference/models/atma.py:66-73``)."""

from . import HAS_HIP
from .inference_ops import packed_causal_conv1d, softcap_logits, squared_relu_gate

HAS_TRITON = HAS_HIP

__all__ = ["squared_relu_gate", "softcap_logits", "packed_causal_conv1d", "HAS_TRITON"]

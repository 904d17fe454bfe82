"""The paged serving engine around the global-layer mixer, restating the reference's
``inference/`` interfaces: ``Context`` (thread-local routing and cache maps),
``Sequence`` / ``SamplingParams``, ``PagePool`` (KV pages), ``Scheduler``,
``ModelRunner`` (state tables, KV cache, prefill / decode preparation, decode HIP
graphs), ``LLMEngine.generate`` over token ids, and the 16-block ``Atma`` model whose
global layers run the HIP kernels of ``atma_amd.kernel``."""

from .config import AtmaConfig, Config
from .context import Context, get_context, reset_context, set_context
from .llm_engine import LLMEngine
from .model import Atma, AtmaAttention, AtmaDecoderBlock, AtmaLFM2Conv, Sampler
from .model_runner import ModelRunner
from .scheduler import Scheduler
from .page_pool import PagePool
from .sequence import Phase, SamplingParams, Sequence

__all__ = ["AtmaConfig", "Config", "Context", "get_context", "set_context", "reset_context", "LLMEngine",
           "Atma", "AtmaAttention", "AtmaDecoderBlock", "AtmaLFM2Conv", "Sampler", "ModelRunner", "Scheduler",
           "PagePool", "Phase", "SamplingParams", "Sequence"]

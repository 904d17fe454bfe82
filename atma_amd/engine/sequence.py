"""One generation request of the engine, and its sampling parameters.

A request is a growing token list (prompt, then the tokens it has sampled) plus the
handles the model runner needs to place it on the device: its KV pages, its row of the
per-sequence state tables, and how much of the list is already in those caches.  The
runner reads exactly these attributes, under the names the reference's runner reads
(``inference/engine/model_runner.py:316-480``): ``token_ids`` (through ``len`` and slicing),
``block_table``, ``num_cached_tokens``, ``num_scheduled_tokens``, ``seq_slot``, ``last_token``
and ``temperature``.  The lifecycle (queued -> active -> done) belongs to the scheduler.

``temperature == 0`` asks for greedy decoding (the reference's sampler divides by the
temperature and has no greedy form, ``inference/layers/sampler.py:7-10``).
"""

from dataclasses import dataclass
from enum import Enum
from itertools import count


@dataclass(frozen=True)
class SamplingParams:
    temperature: float = 1.0
    max_tokens: int = 128
    ignore_eos: bool = False


class Phase(Enum):
    QUEUED = "queued"      # waiting for pages and a state-table row
    ACTIVE = "active"      # admitted: prompt being prefilled, then decoding
    DONE = "done"          # finished; pages and row released


_ids = count()


class Sequence:
    """A request's tokens and device handles.  ``len(seq)`` is the number of tokens so far;
    ``seq[a:b]`` slices them."""

    __slots__ = ("seq_id", "token_ids", "prompt_len", "params", "phase", "block_table", "seq_slot",
                 "num_cached_tokens", "num_scheduled_tokens")

    def __init__(self, token_ids, sampling_params: SamplingParams = None):
        self.seq_id = next(_ids)
        self.token_ids = list(token_ids)
        self.prompt_len = len(self.token_ids)
        self.params = sampling_params if sampling_params is not None else SamplingParams()
        self.phase = Phase.QUEUED
        self.block_table = []          # physical KV page of each logical page, in order
        self.seq_slot = -1             # row of the runner's state tables (-1: none held)
        self.num_cached_tokens = 0     # tokens whose K/V, conv tails and memory state are stored
        self.num_scheduled_tokens = 0  # tokens the current step feeds

    def __len__(self):
        return len(self.token_ids)

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def temperature(self):
        return self.params.temperature

    @property
    def last_token(self):
        return self.token_ids[-1]

    @property
    def prompt_done(self):
        """Every prompt token is in the caches: the next step is a decode step."""
        return self.num_cached_tokens >= self.prompt_len

    @property
    def completion_token_ids(self):
        return self.token_ids[self.prompt_len:]

    @property
    def is_finished(self):
        return self.phase is Phase.DONE

    def lifetime_tokens(self):
        """The most tokens this request can ever hold: prompt plus its token limit (the
        last sampled token is never fed back, but its slot is counted to keep this simple)."""
        return self.prompt_len + self.params.max_tokens

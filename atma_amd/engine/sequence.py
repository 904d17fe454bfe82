"""A request's token stream and paging state (``inference/engine/sequence.py:14-92``),
and its sampling parameters (``inference/sampling_params.py``) with a greedy mode:
``temperature == 0`` takes the argmax (the reference's sampler divides by the
temperature and has no greedy form, ``inference/layers/sampler.py:7-10``)."""

from copy import copy
from dataclasses import dataclass
from enum import Enum, auto
from itertools import count


@dataclass
class SamplingParams:
    temperature: float = 1.0
    max_tokens: int = 128
    ignore_eos: bool = False


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


class Sequence:
    block_size = 256
    counter = count()

    def __init__(self, token_ids, sampling_params: SamplingParams = None):
        sp = sampling_params or SamplingParams()
        self.seq_id = next(Sequence.counter)
        self.status = SequenceStatus.WAITING
        self.token_ids = copy(list(token_ids))
        self.last_token = self.token_ids[-1] if self.token_ids else 0
        self.num_tokens = len(self.token_ids)
        self.num_prompt_tokens = self.num_tokens
        self.num_cached_tokens = 0
        self.num_scheduled_tokens = 0
        self.is_prefill = True
        self.block_table = []
        self.temperature = sp.temperature
        self.max_tokens = sp.max_tokens
        self.ignore_eos = sp.ignore_eos
        self.seq_slot = -1           # row of the runner's per-sequence state tables

    def __len__(self):
        return self.num_tokens

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def is_finished(self):
        return self.status == SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self):
        return self.num_tokens - self.num_prompt_tokens

    @property
    def completion_token_ids(self):
        return self.token_ids[self.num_prompt_tokens:]

    @property
    def num_blocks(self):
        return (self.num_tokens + self.block_size - 1) // self.block_size

    @property
    def last_block_num_tokens(self):
        if self.num_tokens == 0:
            return 0
        rem = self.num_tokens % self.block_size
        return self.block_size if rem == 0 else rem

    def append_token(self, token_id: int):
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1

"""The serving loop (``inference/engine/llm_engine.py:16-145``) over token-id prompts.

``generate`` adds every prompt, then steps the scheduler until all requests finish:
one prefill batch or one decode step per ``step()``.  Prefill and decode throughput
are measured the reference's way -- HIP events around each step -- and kept in
``last_metrics``.  Prompts are token-id lists: there is no tokenizer (loading one is a
network fetch in the reference, ``:27-32``)."""

from dataclasses import fields

import torch

from .config import Config
from .model_runner import ModelRunner
from .scheduler import Scheduler
from .sequence import SamplingParams, Sequence


class LLMEngine:

    def __init__(self, config: Config = None, model=None, **kwargs):
        if config is None:
            names = {f.name for f in fields(Config)}
            config = Config(**{k: v for k, v in kwargs.items() if k in names})
        self.config = config
        Sequence.block_size = config.kvcache_block_size
        self.model_runner = ModelRunner(config, model)
        self.scheduler = Scheduler(config)
        self.last_metrics = {}

    def exit(self):
        if self.model_runner is not None:
            self.model_runner.exit()
            self.model_runner = None

    def add_request(self, token_ids, sampling_params: SamplingParams = None):
        seq = Sequence(token_ids, sampling_params)
        self.scheduler.add(seq)
        return seq

    def step(self):
        """Plan, run and account one batch.  Returns ``(finished, n)``: the requests that
        finished in this step as ``(seq_id, completion token ids)``, and the tokens the step
        fed -- positive for a prefill batch, negative (minus the batch size) for a decode
        batch, 0 when idle (the reference's throughput accounting)."""
        batch, is_prefill = self.scheduler.schedule()
        if not batch:
            return [], 0
        fed = sum(s.num_scheduled_tokens for s in batch)
        sampled = self.model_runner.run(batch, is_prefill)
        done = self.scheduler.commit(batch, sampled)
        for seq in done:
            self.model_runner.free_seq_slot(seq)
        return [(s.seq_id, s.completion_token_ids) for s in done], (fed if is_prefill else -fed)

    def is_finished(self):
        return self.scheduler.is_finished()

    def generate(self, prompts, sampling_params=None, on_step=None):
        """prompts: list of token-id lists.  Returns one dict ``{"token_ids": [...]}`` per
        prompt, in prompt order.  ``on_step(is_prefill, seqs_done, ms)`` (optional) sees
        every step."""
        sp = sampling_params if sampling_params is not None else SamplingParams()
        sps = sp if isinstance(sp, list) else [sp] * len(prompts)
        seqs = [self.add_request(p, s) for p, s in zip(prompts, sps)]
        outputs = {}
        t_pre = t_dec = 0.0
        n_pre = n_dec = 0
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        while not self.is_finished():
            e0.record()
            out, num_tokens = self.step()
            e1.record()
            e1.synchronize()
            ms = e0.elapsed_time(e1)
            if num_tokens > 0:
                t_pre += ms
                n_pre += num_tokens
            elif num_tokens < 0:
                t_dec += ms
                n_dec -= num_tokens
            if on_step is not None:
                on_step(num_tokens > 0, len(outputs), ms)
            for seq_id, toks in out:
                outputs[seq_id] = toks
        self.last_metrics = {
            "prefill_throughput": n_pre / (t_pre * 1e-3) if t_pre else 0.0,
            "decode_throughput": n_dec / (t_dec * 1e-3) if t_dec else 0.0,
            "prefill_tokens": n_pre, "decode_tokens": n_dec,
            "prefill_time": t_pre * 1e-3, "decode_time": t_dec * 1e-3,
        }
        return [{"token_ids": outputs[s.seq_id]} for s in seqs]

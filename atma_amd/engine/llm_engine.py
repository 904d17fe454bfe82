"""The serving loop (``inference/engine/llm_engine.py:16-145``) over token-id prompts.

``generate`` adds every prompt, then steps the scheduler until all requests finish:
one prefill batch or one decode step per ``step()``.  Inside ``generate`` the decode steps
of an unchanged greedy batch run as a pipeline (``_decode_run``): step n + 1 is launched
before step n's tokens are read back, so the host's accounting of step n overlaps the
device's work on step n + 1.  Prefill and decode throughput are measured with HIP events
around each step (around each pipelined run of decode steps) and kept in
``last_metrics``.  Prompts are token-id lists: there is no tokenizer (loading one is a
network fetch in the reference, ``:27-32``)."""

from dataclasses import fields

import torch

from .config import Config
from .model_runner import ModelRunner
from .scheduler import Scheduler
from .sequence import Phase, SamplingParams, Sequence


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
        return self._run_batch(batch, is_prefill)

    def _run_batch(self, batch, is_prefill):
        if not batch:
            return [], 0
        fed = sum(s.num_scheduled_tokens for s in batch)
        sampled = self.model_runner.run(batch, is_prefill)
        done = self.scheduler.commit(batch, sampled)
        self.model_runner.free_seq_slots(done)
        return [(s.seq_id, s.completion_token_ids) for s in done], (fed if is_prefill else -fed)

    def _decode_run(self, batch):
        """Decode steps of one batch, each launched before the previous one's tokens are read
        back (the graph leaves its greedy ids in place as the next step's inputs), while the
        batch stays the same: the run ends when a request finishes (its token limit, known in
        advance, or the end-of-sequence id, seen one step late: the step already launched
        still comes back, and its token for the finished request is dropped).  Returns what
        ``step`` returns for the whole run."""
        mr, sch = self.model_runner, self.scheduler
        left = min(s.params.max_tokens - (len(s.token_ids) - s.prompt_len) for s in batch)
        finished, fed = [], 0
        launch, n = mr.launch_decode(batch, ahead=0), 1
        while launch is not None:
            ahead = mr.launch_decode(batch, ahead=1) if n < left else None
            ids = mr.collect(launch)
            live = [s for s in batch if s.phase is Phase.ACTIVE]
            for s in live:
                s.num_scheduled_tokens = 1
            fed += len(live)
            done = sch.commit(batch, ids)
            finished += done
            if done and ahead is not None:   # a request left the batch: the launched step ends the run
                ids = mr.collect(ahead)
                live = [s for s in batch if s.phase is Phase.ACTIVE]
                for s in live:
                    s.num_scheduled_tokens = 1
                fed += len(live)
                finished += sch.commit(batch, ids)
                ahead = None
            launch, n = ahead, n + 1
        mr.free_seq_slots(finished)
        return [(s.seq_id, s.completion_token_ids) for s in finished], -fed

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
            batch, is_prefill = self.scheduler.schedule()
            if batch and not is_prefill and self.model_runner.can_pipeline(batch):
                out, num_tokens = self._decode_run(batch)
            else:
                out, num_tokens = self._run_batch(batch, is_prefill)
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

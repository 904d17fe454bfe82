"""Step planning for the paged engine.

Every engine step is one batch, either of prompt work (prefill) or of one new token for
each active request (decode).  The policy:

* **Admission.**  Queued requests are admitted in arrival order while a state-table row
  is free (at most ``max_num_seqs`` active) and the page pool holds every page the request
  can ever fill (``Sequence.lifetime_tokens``).  Admission is where a request's pages are
  taken, so a decode step never waits for a page and nothing is ever evicted.  A request
  that could not fit in the whole pool, or exceeds ``max_model_len``, is refused by ``add``.
* **Prefill before decode.**  While any active request has uncached prompt tokens, the
  step is a prefill batch: whole prompts, in admission order, as many as fit in
  ``max_num_batched_tokens``.  A prompt longer than that budget is fed alone, one
  budget-sized piece per step (the runner's continuation route); the sample of a piece
  that does not end the prompt is discarded.
* **Decode.**  Otherwise every active request feeds its newest token.  The decode batch is
  all active requests, which the runner's captured graph buckets are sized for.

``commit`` accounts a step's sampled tokens and returns the requests that finished (token
limit, or the end-of-sequence id unless ignored); their pages go back to the pool at once.
The caller releases their state-table rows (``ModelRunner.free_seq_slot``).
"""

from collections import deque

from .config import Config
from .page_pool import PagePool, pages_for
from .sequence import Phase, Sequence


class Scheduler:

    def __init__(self, config: Config):
        self.max_active = config.max_num_seqs
        self.token_budget = config.max_num_batched_tokens
        self.max_model_len = config.max_model_len
        self.eos = config.eos
        self.pool = PagePool(config.num_kvcache_blocks, config.kvcache_block_size)
        self.queue: deque = deque()
        self.active: list = []

    def add(self, seq: Sequence):
        if len(seq) == 0:
            raise ValueError("a request needs at least one prompt token")
        life = seq.lifetime_tokens()
        if life > self.max_model_len:
            raise ValueError(f"prompt {seq.prompt_len} + max_tokens {seq.params.max_tokens} exceeds "
                             f"max_model_len {self.max_model_len}")
        if pages_for(life, self.pool.page_size) > self.pool.num_pages:
            raise ValueError(f"a request of {life} tokens needs more pages than the pool's {self.pool.num_pages}")
        self.queue.append(seq)

    def is_finished(self) -> bool:
        return not self.queue and not self.active

    def _admit(self):
        while self.queue and len(self.active) < self.max_active:
            seq = self.queue[0]
            if not self.pool.fits(seq.lifetime_tokens()):
                return                          # arrival order: no request jumps the queue
            self.queue.popleft()
            self.pool.take(seq, seq.lifetime_tokens())
            seq.phase = Phase.ACTIVE
            self.active.append(seq)

    def schedule(self):
        """Plan the next step: ``(batch, is_prefill)``; ``([], False)`` when idle."""
        self._admit()
        prompt_work = [s for s in self.active if not s.prompt_done]
        if prompt_work:
            batch, used = [], 0
            for seq in prompt_work:
                rest = seq.prompt_len - seq.num_cached_tokens
                if used + rest > self.token_budget:
                    if not batch:               # longer than a whole step: one piece, alone
                        seq.num_scheduled_tokens = self.token_budget
                        batch.append(seq)
                    break
                seq.num_scheduled_tokens = rest
                batch.append(seq)
                used += rest
            return batch, True
        for seq in self.active:
            seq.num_scheduled_tokens = 1
        return list(self.active), False

    def commit(self, batch, token_ids):
        """Record one step's sampled tokens; returns the requests that finished."""
        finished = []
        for seq, tok in zip(batch, token_ids):
            if seq.phase is Phase.DONE:          # finished while a later step was in flight
                continue
            seq.num_cached_tokens += seq.num_scheduled_tokens
            seq.num_scheduled_tokens = 0
            if not seq.prompt_done:
                continue
            seq.token_ids.append(int(tok))
            hit_eos = not seq.params.ignore_eos and tok == self.eos
            if hit_eos or len(seq.token_ids) - seq.prompt_len >= seq.params.max_tokens:
                seq.phase = Phase.DONE
                self.pool.give_back(seq)
                finished.append(seq)
        if finished:
            self.active = [s for s in self.active if s.phase is Phase.ACTIVE]
        return finished

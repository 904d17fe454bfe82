"""The pool of KV-cache pages.

Pages are handed out whole for a request's lifetime: when the scheduler admits a request
it takes every page the request can ever fill (prompt plus token limit), so a running
request never needs a page another holds, and the engine never has to evict one.  That
trades some pool capacity for a scheduler with no preemption path (an evicted request
would have to restart its per-sequence conv and memory state as well as its pages).

There is no cross-request prefix sharing: two requests with one prefix would share K/V
pages, but their conv tails and memory states are per request.

Pages are reused last-freed-first, which keeps recently touched pages warm in the L2.
"""


def pages_for(num_tokens: int, page_size: int) -> int:
    return -(-num_tokens // page_size)


class PagePool:

    def __init__(self, num_pages: int, page_size: int):
        if num_pages <= 0 or page_size <= 0:
            raise ValueError(f"need a positive page count and size, got {num_pages} x {page_size}")
        self.num_pages = num_pages
        self.page_size = page_size
        self._free = list(range(num_pages - 1, -1, -1))     # a stack: pop() gives page 0 first
        self._owner = {}                                    # page -> seq_id

    @property
    def num_free(self) -> int:
        return len(self._free)

    def fits(self, num_tokens: int) -> bool:
        return pages_for(num_tokens, self.page_size) <= len(self._free)

    def take(self, seq, num_tokens: int):
        """Give ``seq`` pages for ``num_tokens`` tokens (appended to its table)."""
        need = pages_for(num_tokens, self.page_size) - len(seq.block_table)
        if need > len(self._free):
            raise RuntimeError(f"page pool exhausted: need {need}, {len(self._free)} free")
        for _ in range(max(need, 0)):
            page = self._free.pop()
            self._owner[page] = seq.seq_id
            seq.block_table.append(page)

    def give_back(self, seq):
        """Return every page ``seq`` holds (nothing is returned if any is not its own)."""
        stray = [p for p in seq.block_table if self._owner.get(p) != seq.seq_id]
        if stray:
            raise RuntimeError(f"pages {stray} are not held by sequence {seq.seq_id}")
        for page in reversed(seq.block_table):
            del self._owner[page]
            self._free.append(page)
        seq.block_table = []

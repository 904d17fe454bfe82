"""Paged KV-cache page allocator (``inference/engine/block_manager.py:32-135``).

Same contract as the reference's ``BlockManager`` -- ``can_allocate`` / ``allocate`` /
``deallocate`` / ``can_append`` / ``may_append`` -- without cross-request prefix
sharing: a shared prefix would share K/V pages but not the per-sequence Canon-conv and
memory states, which start from zero for the new request (the reference documents that
drift), so every request here gets its own pages and ``num_cached_tokens`` starts at 0.
"""

from collections import deque

from .sequence import Sequence


class BlockManager:

    def __init__(self, num_blocks: int, block_size: int):
        self.block_size = block_size
        self.free_block_ids: deque = deque(range(num_blocks))
        self.used_block_ids: set = set()

    def _allocate_block(self) -> int:
        block_id = self.free_block_ids.popleft()
        self.used_block_ids.add(block_id)
        return block_id

    def _deallocate_block(self, block_id: int):
        self.used_block_ids.remove(block_id)
        self.free_block_ids.append(block_id)

    def can_allocate(self, seq: Sequence) -> int:
        """Number of cached (shared) blocks, 0 here, or -1 when the pool is short."""
        return 0 if len(self.free_block_ids) >= seq.num_blocks else -1

    def allocate(self, seq: Sequence, num_cached_blocks: int = 0):
        assert not seq.block_table and num_cached_blocks == 0
        for _ in range(seq.num_blocks):
            seq.block_table.append(self._allocate_block())
        seq.num_cached_tokens = 0

    def deallocate(self, seq: Sequence):
        for block_id in reversed(seq.block_table):
            self._deallocate_block(block_id)
        seq.num_cached_tokens = 0
        seq.block_table.clear()

    def can_append(self, seq: Sequence) -> bool:
        """A decode step needs a new page when the token it appends starts one."""
        return len(self.free_block_ids) >= (len(seq) % self.block_size == 1)

    def may_append(self, seq: Sequence):
        if len(seq) % self.block_size == 1:
            seq.block_table.append(self._allocate_block())

    def hash_blocks(self, seq: Sequence):
        """Prefix registration of the reference; nothing to record without sharing."""

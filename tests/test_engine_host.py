"""Host logic of the paged engine, no GPU: prefill routing and the maps it builds
(the reference's ``tests/test_dense_prefill.py:31-95`` pattern, a runner made without
its device state), decode inputs, the page allocator and the scheduler's policy."""

from types import SimpleNamespace

import torch

from atma_amd.engine import Config, ModelRunner, Scheduler, Sequence, get_context, reset_context
from atma_amd.engine.block_manager import BlockManager
from atma_amd.engine.sequence import SamplingParams, SequenceStatus


def _runner(max_tokens=128, dtype=torch.bfloat16, block=16):
    r = ModelRunner.__new__(ModelRunner)
    r.block_size = block
    r.device = torch.device("cpu")
    r.config = SimpleNamespace(max_num_batched_tokens=max_tokens, hf_config=SimpleNamespace(dtype=dtype))
    r.conv_state_tables = {}
    return r


def _seq(length, slot, scheduled=None, cached=0, first_block=None, block=16):
    Sequence.block_size = block
    s = Sequence(list(range(length)))
    s.seq_slot = slot
    s.num_cached_tokens = cached
    s.num_scheduled_tokens = length - cached if scheduled is None else scheduled
    base = slot * 16 if first_block is None else first_block
    s.block_table = list(range(base, base + s.num_blocks))
    return s


def test_dense_route_only_for_fresh_complete_equal_batches():
    r = _runner()
    r.prepare_prefill([_seq(8, 0), _seq(8, 1)])
    ctx = get_context()
    assert ctx.dense_prefill and (ctx.dense_batch_size, ctx.dense_seq_len) == (2, 8)
    assert torch.equal(ctx.seq_slots, torch.tensor([0, 1]))
    assert torch.equal(ctx.token_seq_starts, torch.tensor([0] * 8 + [8] * 8, dtype=torch.int32))
    reset_context()
    for batch in ([_seq(8, 0)], [_seq(8, 0), _seq(7, 1)], [_seq(8, 0, cached=1), _seq(8, 1)],
                  [_seq(8, 0, scheduled=4), _seq(8, 1)]):
        r.prepare_prefill(batch)
        assert not get_context().dense_prefill
        reset_context()


def test_grouped_route_and_tile_map():
    """The reference test's lengths (33, 65, 129): one tile entry per 128 query rows."""
    r = _runner(max_tokens=512)
    r.prepare_prefill([_seq(33, 0), _seq(65, 1), _seq(129, 2)])
    ctx = get_context()
    assert ctx.grouped_polar_prefill and not ctx.dense_prefill
    assert ctx.polar_tile_seq_starts.tolist() == [0, 33, 98, 98]
    assert ctx.polar_tile_q_starts.tolist() == [0, 0, 0, 128]
    assert ctx.polar_tile_seq_lens.tolist() == [33, 65, 129, 129]
    assert ctx.token_seq_starts.numel() == 227 and int(ctx.token_seq_ends[-1]) == 227
    assert int(ctx.token_seq_slots[-1]) == 2 and ctx.cu_seqlens_q.tolist() == [0, 33, 98, 227]
    reset_context()
    r32 = _runner(max_tokens=512, dtype=torch.float32)       # the packed Polar kernel is 16-bit only
    r32.prepare_prefill([_seq(33, 0), _seq(65, 1)])
    assert not get_context().grouped_polar_prefill and get_context().token_seq_starts is not None
    reset_context()


def test_prefill_slot_mapping_follows_pages():
    """slot = block_table[pos // page] * page + pos % page, for a continuation too."""
    r = _runner()
    s = _seq(40, 0, cached=20, first_block=0)
    s.block_table = [7, 3, 9]
    r.prepare_prefill([s])
    ctx = get_context()
    want = [s.block_table[p // 16] * 16 + p % 16 for p in range(20, 40)]
    assert ctx.slot_mapping.tolist() == want and ctx.block_tables.tolist() == [[7, 3, 9]]
    assert ctx.token_seq_starts is None and not ctx.dense_prefill    # a continuation: per-sequence route
    reset_context()


def test_decode_inputs():
    r = _runner()
    a, b = _seq(17, 0), _seq(32, 1)
    a.block_table, b.block_table = [4, 6], [2, 5]
    r.prepare_decode([a, b])
    ctx = get_context()
    assert ctx.context_lens.tolist() == [17, 32]
    assert ctx.slot_mapping.tolist() == [6 * 16 + 0, 5 * 16 + 15]
    assert ctx.block_tables.tolist() == [[4, 6], [2, 5]]
    reset_context()


def test_block_manager_pages():
    Sequence.block_size = 16
    bm = BlockManager(4, 16)
    s = Sequence(list(range(20)))
    assert bm.can_allocate(s) == 0
    bm.allocate(s)
    assert s.block_table == [0, 1] and s.num_cached_tokens == 0
    big = Sequence(list(range(50)))
    assert bm.can_allocate(big) == -1
    for t in range(12):
        s.append_token(t)
    assert bm.can_append(s)                      # token 32 still fits page 1
    s.append_token(0)                            # token 33 opens page 2
    bm.may_append(s)
    assert s.block_table == [0, 1, 2]
    bm.deallocate(s)
    assert s.block_table == [] and len(bm.free_block_ids) == 4


def test_scheduler_prefill_then_decode_then_finish():
    cfg = Config(kvcache_block_size=16, max_num_seqs=4, max_num_batched_tokens=64, num_kvcache_blocks=8)
    Sequence.block_size = 16
    sch = Scheduler(cfg)
    seqs = [Sequence(list(range(30)), SamplingParams(temperature=0, max_tokens=2, ignore_eos=True))
            for _ in range(3)]
    for s in seqs:
        sch.add(s)
    batch, is_prefill = sch.schedule()
    assert is_prefill and batch == seqs[:2]      # 30 + 30 <= 64; the third would be chunked, not first
    sch.postprocess(batch, [1, 1], True)
    batch, is_prefill = sch.schedule()
    assert is_prefill and batch == [seqs[2]]
    sch.postprocess(batch, [1], True)
    batch, is_prefill = sch.schedule()
    assert not is_prefill and batch == seqs
    sch.postprocess(batch, [2, 2, 2], False)
    assert all(s.status == SequenceStatus.FINISHED for s in seqs) and sch.is_finished()
    assert [s.completion_token_ids for s in seqs] == [[1, 2]] * 3
    assert len(sch.block_manager.free_block_ids) == 8

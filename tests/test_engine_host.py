"""Host logic of the paged engine, no GPU: prefill routing and the maps it builds
(the reference's ``tests/test_dense_prefill.py:31-95`` pattern, a runner made without
its device state), decode inputs, the page allocator and the scheduler's policy."""

from types import SimpleNamespace

import torch

import pytest

from atma_amd.engine import Config, ModelRunner, PagePool, Phase, Scheduler, Sequence, get_context, reset_context
from atma_amd.engine.page_pool import pages_for
from atma_amd.engine.sequence import SamplingParams


def _runner(max_tokens=128, dtype=torch.bfloat16, block=16):
    r = ModelRunner.__new__(ModelRunner)
    r.block_size = block
    r.device = torch.device("cpu")
    r.config = SimpleNamespace(max_num_batched_tokens=max_tokens, hf_config=SimpleNamespace(dtype=dtype))
    r.conv_state_tables = {}
    return r


def _seq(length, slot, scheduled=None, cached=0, first_block=None, block=16):
    s = Sequence(list(range(length)))
    s.seq_slot = slot
    s.num_cached_tokens = cached
    s.num_scheduled_tokens = length - cached if scheduled is None else scheduled
    base = slot * 16 if first_block is None else first_block
    s.block_table = list(range(base, base + pages_for(length, block)))
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


def test_decode_slot_uses_the_position_page_when_pages_are_reserved_ahead():
    """Pages are held for a request's lifetime, so the table runs past the current length:
    the new token's slot is its position's row in its position's page, not the last page."""
    r = _runner()
    a = _seq(17, 0)
    a.block_table = [4, 6, 9, 11]
    r.prepare_decode([a])
    assert get_context().slot_mapping.tolist() == [6 * 16 + 0]
    reset_context()


def test_page_pool_lifetime_pages_and_ownership():
    pool = PagePool(4, 16)
    s, t = Sequence(list(range(20))), Sequence(list(range(5)))
    assert pool.fits(64) and not pool.fits(65)
    pool.take(s, 20)
    assert s.block_table == [0, 1] and pool.num_free == 2
    pool.take(s, 33)                             # growing to 33 tokens adds page 2 only
    assert s.block_table == [0, 1, 2]
    with pytest.raises(RuntimeError):
        pool.take(t, 32)                         # two pages wanted, one free
    pool.take(t, 5)
    t.block_table.append(0)                      # a page t does not own
    with pytest.raises(RuntimeError):
        pool.give_back(t)
    assert t.block_table == [3, 0] and pool.num_free == 0    # refused whole: nothing moved
    t.block_table.pop()
    pool.give_back(s)
    assert s.block_table == [] and pool.num_free == 3
    u = Sequence([1])
    pool.take(u, 1)                              # last freed, first reused
    assert u.block_table == [0]


def _sched(pages=8, budget=64, max_seqs=4, max_len=4096, eos=50256):
    return Scheduler(Config(kvcache_block_size=16, max_num_seqs=max_seqs, max_num_batched_tokens=budget,
                            num_kvcache_blocks=pages, max_model_len=max_len, eos=eos))


def _req(n, new, eos=True, first=0):
    return Sequence(list(range(first, first + n)), SamplingParams(temperature=0, max_tokens=new, ignore_eos=eos))


def test_scheduler_prefill_then_decode_then_finish():
    sch = _sched()
    seqs = [_req(30, 2) for _ in range(3)]       # 32 tokens each: two pages for life
    for s in seqs:
        sch.add(s)
    batch, is_prefill = sch.schedule()
    assert is_prefill and batch == seqs[:2]      # 30 + 30 <= 64; the third waits for the next step
    assert all(len(s.block_table) == 2 for s in seqs) and sch.pool.num_free == 2
    assert sch.commit(batch, [1, 1]) == []
    batch, is_prefill = sch.schedule()
    assert is_prefill and batch == [seqs[2]]
    sch.commit(batch, [1])
    batch, is_prefill = sch.schedule()
    assert not is_prefill and batch == seqs and all(s.num_scheduled_tokens == 1 for s in seqs)
    assert sch.commit(batch, [2, 2, 2]) == seqs
    assert all(s.phase is Phase.DONE for s in seqs) and sch.is_finished()
    assert [s.completion_token_ids for s in seqs] == [[1, 2]] * 3
    assert sch.pool.num_free == 8


def test_scheduler_admits_only_what_the_pool_holds_for_life_and_never_evicts():
    """With room for one request's lifetime pages at a time, the second waits (queued, no
    pages) until the first finishes, then runs from a clean start."""
    sch = _sched(pages=3)
    a, b = _req(20, 20), _req(20, 20, first=100)  # 40 tokens: three pages each
    sch.add(a)
    sch.add(b)
    batch, is_prefill = sch.schedule()
    assert is_prefill and batch == [a] and b.phase is Phase.QUEUED and b.block_table == []
    sch.commit(batch, [7])
    for step in range(19):
        batch, is_prefill = sch.schedule()
        assert not is_prefill and batch == [a]
        done = sch.commit(batch, [7])
    assert done == [a] and len(a.completion_token_ids) == 20
    batch, is_prefill = sch.schedule()
    assert is_prefill and batch == [b] and b.num_cached_tokens == 0 and len(b.block_table) == 3


def test_scheduler_feeds_a_long_prompt_in_budget_pieces_alone():
    sch = _sched(pages=16, budget=64)
    long_, short = _req(150, 2), _req(10, 2, first=500)
    sch.add(long_)
    sch.add(short)
    fed = []
    while True:
        batch, is_prefill = sch.schedule()
        if not is_prefill:
            break
        fed.append([(s is long_, s.num_scheduled_tokens) for s in batch])
        sch.commit(batch, [9] * len(batch))
    assert fed == [[(True, 64)], [(True, 64)], [(True, 22), (False, 10)]]
    assert long_.completion_token_ids == [9] and long_.num_cached_tokens == 150    # pieces' samples dropped


def test_scheduler_stops_at_eos_unless_ignored():
    sch = _sched(eos=3)
    a, b = _req(5, 10, eos=False), _req(5, 10, eos=True)
    sch.add(a)
    sch.add(b)
    batch, _ = sch.schedule()
    assert sch.commit(batch, [3, 3]) == [a]
    assert a.completion_token_ids == [3] and b.phase is Phase.ACTIVE and sch.active == [b]


def test_scheduler_refuses_requests_that_can_never_run():
    sch = _sched(pages=4, max_len=100)
    with pytest.raises(ValueError):
        sch.add(_req(90, 20))                    # beyond max_model_len
    with pytest.raises(ValueError):
        _sched(pages=2).add(_req(30, 10))         # three pages for life, two in the pool
    with pytest.raises(ValueError):
        sch.add(Sequence([]))


def test_scheduler_caps_active_requests_at_the_table_rows():
    sch = _sched(pages=64, max_seqs=2)
    reqs = [_req(8, 1, first=10 * i) for i in range(3)]
    for r in reqs:
        sch.add(r)
    batch, _ = sch.schedule()
    assert batch == reqs[:2] and reqs[2].phase is Phase.QUEUED
    assert sch.commit(batch, [1, 1]) == reqs[:2]
    batch, _ = sch.schedule()
    assert batch == [reqs[2]]

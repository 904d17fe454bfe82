"""GPU parity of the fused global-layer decode step (``global_decode_step``) against the
three calls it replaces, made in the reference's order (store_kvcache,
polar_attention_decode, gated_delta_decode_step; ``inference/models/atma.py:546-618``),
and against the CPU oracle.

The caches and the memory state come out bit-identical to the separate calls (the same
bytes are written, the memory step is the same code).  c and mag differ only in the
order the newest key's term is summed (it joins in the merge instead of in a split), so
they are held to the bf16 bar against the separate path and against the oracle."""

import pytest
import torch

from helpers import polar_params, rel_err
from oracle import gated_delta as OG
from oracle import polar as OP

pytestmark = pytest.mark.gpu


def _setup(B, Hq, Hkv, d, ctx, page, dtype, seed, max_seqs=None):
    """Paged caches holding positions 0 .. ctx-2 of each sequence; the newest token
    (position ctx-1) arrives as k_new / v_new with its slot in slot_mapping."""
    g = torch.Generator().manual_seed(seed)
    npg = [(n + page - 1) // page for n in ctx]
    max_pages = max(npg)
    pool = sum(npg) + 2
    perm = torch.randperm(pool, generator=g)
    bt = torch.full((B, max_pages), -1, dtype=torch.int32)
    used = 0
    for b, m in enumerate(npg):
        bt[b, :m] = perm[used:used + m].int()
        used += m
    kc = torch.randn(pool, page, Hkv, d, generator=g).to(dtype)
    vc = torch.randn(pool, page, Hkv, d, generator=g).to(dtype)
    slot = torch.tensor([int(bt[b, (n - 1) // page]) * page + (n - 1) % page for b, n in enumerate(ctx)],
                        dtype=torch.int32)
    q = torch.randn(B, Hq, d, generator=g).to(dtype)
    k_new = torch.randn(B, Hkv, d, generator=g).to(dtype)
    v_new = torch.randn(B, Hkv, d, generator=g).to(dtype)
    gamma = torch.sigmoid(torch.randn(B, Hq, generator=g) + 3.0)
    beta = torch.sigmoid(torch.randn(B, Hq, generator=g))
    max_seqs = max_seqs or 2 * B
    table = torch.randn(max_seqs, Hq, d, d, generator=g) * 0.1
    slots = torch.randperm(max_seqs, generator=g)[:B].long()
    return dict(q=q, k_new=k_new, v_new=v_new, kc=kc, vc=vc, slot=slot, bt=bt,
                ctx=torch.tensor(ctx, dtype=torch.int32), gamma=gamma, beta=beta, table=table, slots=slots)


def _to(dev, s):
    return {k: v.to(dev).clone() for k, v in s.items()}


def _fused(s, p, window=None):
    from atma_amd.kernel import global_decode_step
    c, mag, r = global_decode_step(s["q"], s["k_new"], s["v_new"], s["kc"], s["vc"], s["slot"], s["bt"],
                                   s["ctx"], s["gamma"], s["beta"], s["table"], s["slots"], window=window, **p)
    torch.cuda.synchronize()
    return c, mag, r


def _separate(s, p, window=None):
    from atma_amd.kernel import gated_delta_decode_step, polar_attention_decode
    from atma_amd.layers.attention import store_kvcache
    store_kvcache(s["k_new"], s["v_new"], s["kc"], s["vc"], s["slot"])
    c, mag = polar_attention_decode(s["q"], s["kc"], s["vc"], s["bt"], s["ctx"], window=window, **p)
    r = gated_delta_decode_step(s["q"], s["k_new"], s["v_new"], s["gamma"], s["beta"], s["table"], s["slots"])
    torch.cuda.synchronize()
    return c, mag, r


CASES = [  # (ctx, page, Hq, Hkv, d, dtype, window)
    ([1, 2, 31, 32, 33, 700, 1024, 1025], 64, 8, 2, 128, torch.bfloat16, None),
    ([5, 300, 64, 2049, 96], 32, 8, 2, 128, torch.float16, None),
    ([1, 130, 257, 640], 256, 16, 2, 64, torch.bfloat16, None),
    ([40, 700, 1500, 33], 64, 8, 2, 128, torch.bfloat16, 100),
    ([3, 77, 512], 64, 4, 4, 64, torch.bfloat16, 32),
]


@pytest.mark.parametrize("ctx,page,Hq,Hkv,d,dtype,window", CASES)
def test_fused_equals_separate_calls(dev, ctx, page, Hq, Hkv, d, dtype, window):
    s = _setup(len(ctx), Hq, Hkv, d, ctx, page, dtype, seed=len(ctx) * 7 + d)
    p = {k: v.to(dev) for k, v in polar_params(Hq, d, seed=5).items()}
    a, b = _to(dev, s), _to(dev, s)
    from atma_amd.kernel import global_decode_step_supported
    assert global_decode_step_supported(a["q"], a["kc"], a["bt"])
    c1, m1, r1 = _fused(a, p, window)
    c2, m2, r2 = _separate(b, p, window)
    # the caches and the memory state: the same bytes
    assert torch.equal(a["kc"], b["kc"]) and torch.equal(a["vc"], b["vc"])
    assert torch.equal(a["table"], b["table"]) and torch.equal(r1, r2)
    # attention: the newest key's term summed in another order
    assert torch.isfinite(c1.float()).all() and torch.isfinite(m1.float()).all()
    assert rel_err(c1, c2) <= 2e-2 and rel_err(m1, m2) <= 2e-2


def test_fused_vs_oracle(dev):
    ctx, page, Hq, Hkv, d = [1, 63, 64, 65, 900, 2000], 64, 8, 2, 128
    s = _setup(len(ctx), Hq, Hkv, d, ctx, page, torch.bfloat16, seed=11)
    p = polar_params(Hq, d, seed=2, prior=True)
    a = _to(dev, s)
    c, mag, r = _fused(a, {k: v.to(dev) for k, v in p.items()})
    # oracle: the cache with the newest rows written, then attention and the memory step
    kc, vc = s["kc"].clone(), s["vc"].clone()
    Hkv_, dd = kc.shape[2], kc.shape[3]
    kc.view(-1, Hkv_, dd)[s["slot"].long()] = s["k_new"]
    vc.view(-1, Hkv_, dd)[s["slot"].long()] = s["v_new"]
    p64 = {k: v.double() for k, v in p.items()}
    c_ref, m_ref = OP.polar_decode_paged(s["q"].double(), kc.float(), vc.float(), s["bt"], s["ctx"], params=p64)
    assert rel_err(c, c_ref) <= 2e-2 and rel_err(mag, m_ref) <= 2e-2
    table = s["table"].clone()
    G = Hq // Hkv  # the oracle takes the expanded heads
    r_ref = OG.gated_delta_decode_step(s["q"].float(), s["k_new"].float().repeat_interleave(G, 1),
                                       s["v_new"].float().repeat_interleave(G, 1), s["gamma"], s["beta"],
                                       table, s["slots"])
    assert rel_err(r, r_ref) <= 1e-4 and rel_err(a["table"], table) <= 1e-5
    assert torch.equal(a["kc"].cpu(), kc) and torch.equal(a["vc"].cpu(), vc)


def test_unwritten_slot_attends_new_key(dev):
    """A row whose slot is -1 leaves the cache alone and still attends k_new / v_new as
    its newest key (the engine's padding rows)."""
    ctx, page, Hq, Hkv, d = [300, 129], 64, 8, 2, 128
    s = _setup(2, Hq, Hkv, d, ctx, page, torch.bfloat16, seed=4)
    s["slot"][1] = -1
    p = polar_params(Hq, d, seed=6, prior=True)
    a = _to(dev, s)
    c, mag, _ = _fused(a, {k: v.to(dev) for k, v in p.items()})
    kc, vc = s["kc"].clone(), s["vc"].clone()
    pos = ctx[1] - 1  # row 1's newest position: not written
    pg = int(s["bt"][1, pos // page])
    assert torch.equal(a["kc"][pg, pos % page].cpu(), kc[pg, pos % page])
    assert torch.equal(a["vc"][pg, pos % page].cpu(), vc[pg, pos % page])
    assert torch.equal(a["kc"].view(-1, Hkv, d)[int(s["slot"][0])].cpu(), s["k_new"][0])
    # the oracle sees k_new / v_new at position ctx-1 of both rows
    for b in range(2):
        pos = ctx[b] - 1
        kc[s["bt"][b, pos // page], pos % page] = s["k_new"][b]
        vc[s["bt"][b, pos // page], pos % page] = s["v_new"][b]
    p64 = {k: v.double() for k, v in p.items()}
    c_ref, m_ref = OP.polar_decode_paged(s["q"].double(), kc.float(), vc.float(), s["bt"], s["ctx"], params=p64)
    assert rel_err(c, c_ref) <= 2e-2 and rel_err(mag, m_ref) <= 2e-2


def test_fused_configs3_size_and_graph_replay(dev):
    """BASELINE configs[3] shape (64 sequences, contexts U[1024, 32768], 256-token pages,
    8/2 heads, d = 128): fused == separate calls, and a captured replay == eager, bitwise."""
    g = torch.Generator().manual_seed(0)
    ctx = torch.randint(1024, 32769, (64,), generator=g).tolist()
    s = _setup(64, 8, 2, 128, ctx, 256, torch.bfloat16, seed=1)
    p = {k: v.to(dev) for k, v in polar_params(8, 128, seed=0, prior=True).items()}
    a, b = _to(dev, s), _to(dev, s)
    c1, m1, r1 = _fused(a, p)
    c2, m2, r2 = _separate(b, p)
    assert torch.equal(a["kc"], b["kc"]) and torch.equal(a["table"], b["table"]) and torch.equal(r1, r2)
    assert rel_err(c1, c2) <= 2e-2 and rel_err(m1, m2) <= 2e-2
    # graph replay: the same inputs give the same outputs (the state table is restored
    # between calls, the cache writes are idempotent)
    from atma_amd.kernel import global_decode_step
    t0 = a["table"].clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        global_decode_step(a["q"], a["k_new"], a["v_new"], a["kc"], a["vc"], a["slot"], a["bt"], a["ctx"],
                           a["gamma"], a["beta"], a["table"], a["slots"], **p)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = global_decode_step(a["q"], a["k_new"], a["v_new"], a["kc"], a["vc"], a["slot"], a["bt"],
                                 a["ctx"], a["gamma"], a["beta"], a["table"], a["slots"], **p)
    for _ in range(3):
        a["table"].copy_(t0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ce, me, re = global_decode_step(a["q"], a["k_new"], a["v_new"], a["kc"], a["vc"], a["slot"], a["bt"],
                                        a["ctx"], a["gamma"], a["beta"], t0.clone(), a["slots"], **p)
        torch.cuda.synchronize()
        assert torch.equal(out[0], ce) and torch.equal(out[1], me) and torch.equal(out[2], re)

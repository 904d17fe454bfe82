"""GPU parity of the paged Polar decode (split-K + merge) against the CPU oracle.

Page/index handling must be bit-exact: the same logical K/V placed in a shuffled page
pool or in an identity pool gives bitwise-identical outputs, and pages the sequence
does not own are never read (they are NaN-poisoned here).
"""

import pytest
import torch

from helpers import max_abs, polar_params, rel_err
from oracle import polar as OP

pytestmark = pytest.mark.gpu


def _paged(B, Hq, Hkv, d, ctx, page, dtype, seed, extra_pages=3, shuffle=True, poison=True):
    g = torch.Generator().manual_seed(seed)
    npg = [(n + page - 1) // page for n in ctx]
    max_pages = max(max(npg), 1)
    pool = sum(npg) + extra_pages
    perm = torch.randperm(pool, generator=g)           # drawn either way: same content below
    if not shuffle:
        perm = torch.arange(pool)
    bt = torch.full((B, max_pages), -1, dtype=torch.int32)
    used = 0
    for b, m in enumerate(npg):
        bt[b, :m] = perm[used:used + m].int()
        used += m
    fill = float("nan") if poison else 0.0
    kc = torch.full((pool, page, Hkv, d), fill)
    vc = torch.full((pool, page, Hkv, d), fill)
    klog = torch.randn(B, max(ctx + [1]), Hkv, d, generator=g)
    vlog = torch.randn(B, max(ctx + [1]), Hkv, d, generator=g)
    for b, n in enumerate(ctx):
        for pos in range(0, n, page):
            m = min(page, n - pos)
            kc[bt[b, pos // page], :m] = klog[b, pos:pos + m]
            vc[bt[b, pos // page], :m] = vlog[b, pos:pos + m]
    q = torch.randn(B, Hq, d, generator=g)
    return q.to(dtype), kc.to(dtype), vc.to(dtype), bt, torch.tensor(ctx, dtype=torch.int32)


def _run(dev, q, kc, vc, bt, ctx, p, **kw):
    from atma_amd.kernel import polar_attention_decode
    c, m = polar_attention_decode(q.to(dev), kc.to(dev), vc.to(dev), bt.to(dev), ctx.to(dev),
                                  **{a: b.to(dev) for a, b in p.items()}, **kw)
    torch.cuda.synchronize()
    return c.cpu(), m.cpu()


def _oracle(q, kc, vc, bt, ctx, p, **kw):
    """fp64 oracle on the same (possibly rounded) cache values; pages are gathered before
    any upcast so only the used rows are converted."""
    p64 = {a: b.double() for a, b in p.items()}
    return OP.polar_decode_paged(q.double(), kc, vc, bt, ctx, params=p64, **kw)


CTX = [1, 255, 256, 257, 700, 1023, 64, 513]


@pytest.mark.parametrize("dtype,d,page", [(torch.float32, 128, 256), (torch.float32, 64, 16),
                                          (torch.bfloat16, 128, 256), (torch.float16, 128, 64),
                                          (torch.bfloat16, 64, 48)])
def test_decode_vs_oracle(dev, dtype, d, page):
    B, Hq, Hkv = len(CTX), 8, 2
    q, kc, vc, bt, ctx = _paged(B, Hq, Hkv, d, CTX, page, dtype, seed=d + page)
    p = polar_params(Hq, d, seed=3)
    c, m = _run(dev, q, kc, vc, bt, ctx, p)
    c_ref, m_ref = _oracle(q.float(), kc.float(), vc.float(), bt, ctx, p)
    assert torch.isfinite(c.float()).all() and torch.isfinite(m.float()).all()
    if dtype == torch.float32:
        assert max_abs(c, c_ref) <= 1e-4 and max_abs(m, m_ref) <= 1e-4
    else:
        assert rel_err(c, c_ref) <= 2e-2 and rel_err(m, m_ref) <= 2e-2


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 2), (4, 4), (2, 1)])
def test_decode_group_sizes(dev, Hq, Hkv):
    ctx = [300, 1, 77]
    q, kc, vc, bt, c_ = _paged(3, Hq, Hkv, 128, ctx, 256, torch.float32, seed=Hq * 10 + Hkv)
    p = polar_params(Hq, 128, seed=Hq)
    c, m = _run(dev, q, kc, vc, bt, c_, p)
    c_ref, m_ref = _oracle(q, kc, vc, bt, c_, p)
    assert max_abs(c, c_ref) <= 1e-4 and max_abs(m, m_ref) <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_shuffled_pool_bitwise_equals_identity_pool(dev, dtype):
    ctx = [1000, 3, 256, 511]
    args = dict(B=4, Hq=8, Hkv=2, d=128, ctx=ctx, page=256, dtype=dtype, seed=11)
    q1, k1, v1, bt1, c1_ = _paged(**args, shuffle=True)
    q2, k2, v2, bt2, c2_ = _paged(**args, shuffle=False)
    p = polar_params(8, 128, seed=11)
    a = _run(dev, q1, k1, v1, bt1, c1_, p)
    b = _run(dev, q2, k2, v2, bt2, c2_, p)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_window_and_zero_context(dev):
    ctx = [0, 5, 700, 1500]
    q, kc, vc, bt, c_ = _paged(4, 8, 2, 128, ctx, 256, torch.float32, seed=12)
    p = polar_params(8, 128, seed=12)
    for window in (None, 100, 300):
        c, m = _run(dev, q, kc, vc, bt, c_, p, window=window)
        c_ref, m_ref = _oracle(q, kc, vc, bt, c_, p, window=window)
        assert max_abs(c, c_ref) <= 1e-4 and max_abs(m, m_ref) <= 1e-4
    # ctx = 0 drains to the null sink
    assert m[0].abs().max() < 1e-6


def test_decode_equals_prefill_row(dev):
    """Decode over a cached prefix == the prefill kernel's row with n_keys = ctx."""
    from atma_amd.kernel import polar_attention_fwd
    ctx = [777]
    q, kc, vc, bt, c_ = _paged(1, 8, 2, 128, ctx, 256, torch.float32, seed=13, poison=False)
    p = polar_params(8, 128, seed=13)
    c, m = _run(dev, q, kc, vc, bt, c_, p)
    kg = OP.gather_paged_kv(kc, bt, c_)[0, :777].permute(1, 0, 2)[None]
    vg = OP.gather_paged_kv(vc, bt, c_)[0, :777].permute(1, 0, 2)[None]
    cp, mp = polar_attention_fwd(q[0][None, :, None].to(dev), kg.to(dev), vg.to(dev),
                                 torch.tensor([777.0], device=dev), is_causal=False,
                                 **{a: b.to(dev) for a, b in p.items()})
    assert max_abs(c[0], cp[0, :, 0].cpu()) <= 2e-5 and max_abs(m[0], mp[0, :, 0].cpu()) <= 2e-5


def test_full_size_decode_bf16(dev):
    """64 sequences, ctx ~ U[1024, 32768], 256-token pages in a
    shuffled pool, bf16; checked on sampled sequences."""
    g = torch.Generator().manual_seed(0)
    B, Hq, Hkv, d, page = 64, 8, 2, 128, 256
    ctx = torch.randint(1024, 32769, (B,), generator=g)
    npg = (ctx + page - 1) // page
    pool = int(npg.sum())
    perm = torch.randperm(pool, generator=g).int()
    bt = torch.full((B, int(npg.max())), -1, dtype=torch.int32)
    used = 0
    for b in range(B):
        bt[b, :npg[b]] = perm[used:used + npg[b]]
        used += int(npg[b])
    kc = torch.randn(pool, page, Hkv, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(pool, page, Hkv, d, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, d, generator=g).to(torch.bfloat16)
    ctx = ctx.int()
    p = polar_params(Hq, d, seed=0, prior=True)
    c, m = _run(dev, q, kc, vc, bt, ctx, p)
    sample = [0, 1, 17, 33, 63]
    c_ref, m_ref = _oracle(q[sample].float(), kc, vc, bt[sample], ctx[sample], p)
    assert rel_err(c[sample], c_ref) <= 2e-2 and rel_err(m[sample], m_ref) <= 2e-2


@pytest.mark.parametrize("dtype,page", [(torch.bfloat16, 32), (torch.float16, 256), (torch.bfloat16, 256)])
@pytest.mark.parametrize("Hq,Hkv", [(8, 2), (16, 2), (8, 8), (4, 1)])
def test_balanced_split_16bit(dev, dtype, page, Hq, Hkv):
    """The length-balanced split (16-bit caches, pages of whole 32-key units): waves take
    equal unit ranges across ragged, empty and windowed contexts and flush a record per
    (sequence, KV head) they touch; NaN-poisoned unused pages are never read."""
    ctx = [0, 1, 31, 32, 33, 700, 2049, 64, 0, 5000]
    d = 128
    q, kc, vc, bt, c_ = _paged(len(ctx), Hq, Hkv, d, ctx, page, dtype, seed=Hq + Hkv + page)
    p = polar_params(Hq, d, seed=Hq + 5)
    for window in (None, 100, 1500):
        c, m = _run(dev, q, kc, vc, bt, c_, p, window=window)
        c_ref, m_ref = _oracle(q.float(), kc.float(), vc.float(), bt, c_, p, window=window)
        assert torch.isfinite(c.float()).all() and torch.isfinite(m.float()).all()
        assert rel_err(c, c_ref) <= 2e-2 and rel_err(m, m_ref) <= 2e-2, window
        assert m[0].abs().max() == 0 and m[8].abs().max() == 0      # empty contexts drain to the sink


def test_balanced_split_many_short_sequences(dev):
    """More sequences than waves' worth of units per pair: each wave crosses many
    (sequence, KV head) boundaries; ragged contexts of a few units each."""
    g = torch.Generator().manual_seed(21)
    ctx = torch.randint(0, 200, (300,), generator=g).tolist()
    q, kc, vc, bt, c_ = _paged(300, 8, 2, 128, ctx, 64, torch.bfloat16, seed=21)
    p = polar_params(8, 128, seed=21)
    c, m = _run(dev, q, kc, vc, bt, c_, p)
    c_ref, m_ref = _oracle(q.float(), kc.float(), vc.float(), bt, c_, p)
    assert rel_err(c, c_ref) <= 2e-2 and rel_err(m, m_ref) <= 2e-2

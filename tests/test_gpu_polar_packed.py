"""GPU parity of the packed ragged fresh prefill (polar_attention_packed_fwd,
kernel/polar_triton.py:194-309,613-669): each packed sequence equals the dense causal
kernel on that sequence alone, bitwise (same kernel arithmetic, per-workgroup bounds),
and the fp32 oracle within the 16-bit bar (max|a-b| / max|b| <= 2e-2).  Tile maps are
built as the serving context builds them (inference/engine/model_runner.py:390-404)."""

import pytest
import torch

from helpers import polar_params, rel_err
from oracle import polar as OP

pytestmark = pytest.mark.gpu


def _tile_map(lengths, bm=128):
    starts, qstarts, lens, start = [], [], [], 0
    for L in lengths:
        for qs in range(0, L, bm):
            starts.append(start)
            qstarts.append(qs)
            lens.append(L)
        start += L
    return (torch.tensor(starts, dtype=torch.int32), torch.tensor(qstarts, dtype=torch.int32),
            torch.tensor(lens, dtype=torch.int32))


def _packed_inputs(lengths, Hq, Hkv, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    q = torch.randn(total, Hq, d, generator=g).to(dtype)
    k = torch.randn(total, Hkv, d, generator=g).to(dtype)
    v = torch.randn(total, Hkv, d, generator=g).to(dtype)
    return q, k, v


def _packed(dev, q, k, v, maps, p, **kw):
    from atma_amd.kernel import polar_attention_packed_fwd
    c, m = polar_attention_packed_fwd(q.to(dev), k.to(dev), v.to(dev), *[t.to(dev) for t in maps],
                                      **{a: b.to(dev) for a, b in p.items()}, **kw)
    torch.cuda.synchronize()
    return c.cpu(), m.cpu()


def _dense(dev, q, k, v, p, **kw):
    """The dense causal kernel on one sequence of packed (L, H, d) rows."""
    from atma_amd.kernel import polar_attention_fwd
    L = q.shape[0]
    qh, kh, vh = (t.transpose(0, 1).unsqueeze(0).contiguous().to(dev) for t in (q, k, v))
    n = torch.arange(1, L + 1, dtype=torch.float32, device=dev)
    c, m = polar_attention_fwd(qh, kh, vh, n, is_causal=True,
                               **{a: b.to(dev) for a, b in p.items()}, **kw)
    torch.cuda.synchronize()
    return c[0].transpose(0, 1).cpu(), m[0].transpose(0, 1).cpu()


CASES = [
    # lengths, Hq, Hkv, d, dtype, window
    ([130, 1, 257, 64, 500], 8, 2, 128, torch.bfloat16, None),
    ([300, 128, 17], 4, 4, 64, torch.float16, None),
    ([200, 90, 385], 8, 2, 128, torch.bfloat16, 48),
]


@pytest.mark.parametrize("lengths,Hq,Hkv,d,dtype,window", CASES,
                         ids=["bf16-gqa", "fp16-d64-expanded", "bf16-window48"])
def test_packed_equals_dense_per_sequence_bitwise(dev, lengths, Hq, Hkv, d, dtype, window):
    q, k, v = _packed_inputs(lengths, Hq, Hkv, d, dtype, seed=sum(lengths))
    p = polar_params(Hq, d, seed=3)
    maps = _tile_map(lengths)
    c, m = _packed(dev, q, k, v, maps, p, window=window)
    assert c.shape == q.shape and m.shape == q.shape[:2] and c.dtype == dtype
    start = 0
    for L in lengths:
        sl = slice(start, start + L)
        cd, md = _dense(dev, q[sl], k[sl], v[sl], p, window=window)
        assert torch.equal(c[sl], cd) and torch.equal(m[sl], md), (L, start)
        start += L


def test_packed_vs_fp32_oracle_and_tile_order(dev):
    lengths = [257, 33, 400]
    q, k, v = _packed_inputs(lengths, 8, 2, 128, torch.bfloat16, seed=7)
    p = polar_params(8, 128, seed=5)
    maps = _tile_map(lengths)
    c, m = _packed(dev, q, k, v, maps, p)
    perm = torch.randperm(maps[0].numel(), generator=torch.Generator().manual_seed(1))
    c2, m2 = _packed(dev, q, k, v, [t[perm] for t in maps], p)
    assert torch.equal(c, c2) and torch.equal(m, m2)   # the map's order does not matter
    start = 0
    for L in lengths:
        sl = slice(start, start + L)
        qh, kh, vh = (t[sl].float().transpose(0, 1).unsqueeze(0).double() for t in (q, k, v))
        kh, vh = kh.repeat_interleave(4, 1), vh.repeat_interleave(4, 1)
        n = torch.arange(1, L + 1, dtype=torch.float64)
        co, mo = OP.polar_online(qh, kh, vh, n, params={a: b.double() for a, b in p.items()},
                                 k_block=256)
        assert rel_err(c[sl], co[0].transpose(0, 1)) <= 2e-2
        assert rel_err(m[sl], mo[0].transpose(0, 1)) <= 2e-2
        start += L


def test_tile_outside_the_tokens_is_skipped(dev):
    """A map entry past the packed tokens is skipped by the kernel's own bounds check;
    the valid tiles are unaffected."""
    lengths = [150, 60]
    q, k, v = _packed_inputs(lengths, 4, 2, 64, torch.bfloat16, seed=9)
    p = polar_params(4, 64, seed=2)
    maps = _tile_map(lengths)
    c, m = _packed(dev, q, k, v, maps, p)
    bad = [torch.cat([t, torch.tensor([x], dtype=torch.int32)])
           for t, x in zip(maps, (sum(lengths), 0, 64))]   # sequence starting at total_tokens
    c2, m2 = _packed(dev, q, k, v, bad, p)
    assert torch.equal(c, c2) and torch.equal(m, m2)

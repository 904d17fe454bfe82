"""The balanced paged-decode schedule's index math, restated on the CPU (no GPU).

The balanced split kernel (``csrc/polar_decode.hip``) orders the 32-key units of every
(sequence, KV head) pair as (b, head, sub-block), gives wave w of NW = min(waves, U) the
units [w U / NW, (w + 1) U / NW), writes one record per pair a wave touches at index
w + sh, and the merge reads records w_first(sh) .. w_last(sh).  These properties keep
every access inside the workspace and every key counted once; here they are checked on
random and edge-case shapes with an independent brute-force walk of the same schedule."""

import random

import pytest


def units_of(ctx, window):
    lo = max(ctx - window, 0) if window > 0 else 0
    return (ctx - (lo & ~31) + 31) >> 5 if ctx > lo else 0


def waves_launched(B, Hkv, max_pages, page):
    units = B * Hkv * ((max_pages * page + 31) // 32)
    return 4 * min(2048 // 4, (units + 3) // 4)


def check(ctx, Hkv, window, max_pages, page):
    B = len(ctx)
    n = [units_of(c, window) for c in ctx]
    pre = [0]
    for x in n:
        pre.append(pre[-1] + x)
    U = Hkv * pre[B]
    nw = waves_launched(B, Hkv, max_pages, page)
    NW = min(nw, U)
    records = set()
    touched = {}                 # pair -> waves whose range holds one of its units
    covered = [0] * U
    for w in range(NW):
        u0, u1 = w * U // NW, (w + 1) * U // NW
        assert u1 > u0           # NW <= U: no empty range
        for u in range(u0, u1):
            # the kernel's lookup: last b with Hkv * pre[b] <= u, then head and sub-block
            b = max(i for i in range(B) if Hkv * pre[i] <= u)
            assert n[b] > 0
            r = u - Hkv * pre[b]
            hk, j = divmod(r, n[b])
            sh = b * Hkv + hk
            pos = ((max(ctx[b] - window, 0) if window > 0 else 0) & ~31) + 32 * j
            assert pos < ctx[b] and pos // page < max_pages          # a real key, a mapped page
            covered[u] += 1
            touched.setdefault(sh, set()).add(w)
        for sh in {s for s, ws in touched.items() if w in ws}:
            rec = w + sh
            assert rec not in records and 0 <= rec < nw + B * Hkv
            records.add(rec)
    assert all(c == 1 for c in covered)
    # the merge's wave range of each pair equals the waves that touched it
    for b in range(B):
        for hk in range(Hkv):
            sh = b * Hkv + hk
            if n[b] == 0:
                assert sh not in touched
                continue
            x0 = Hkv * pre[b] + hk * n[b]
            w0 = ((x0 + 1) * NW - 1) // U
            w1 = ((x0 + n[b]) * NW - 1) // U
            assert set(range(w0, w1 + 1)) == touched[sh], (b, hk)


@pytest.mark.parametrize("seed", range(6))
def test_random_batches(seed):
    rng = random.Random(seed)
    page = rng.choice([32, 64, 256])
    B = rng.randint(1, 40)
    max_pages = rng.randint(1, 12)
    ctx = [rng.randint(0, max_pages * page) for _ in range(B)]
    window = rng.choice([0, 0, 1, 37, 300])
    check(ctx, rng.choice([1, 2, 4]), window, max_pages, page)


def test_edges():
    check([0, 0, 5], 2, 0, 1, 256)             # empty sequences around a tiny one
    check([1], 1, 0, 1, 32)                    # one key
    check([256, 257, 512], 2, 0, 3, 256)       # page boundaries
    check([4096] * 3, 2, 100, 16, 256)         # a window inside long contexts
    check([32768] * 64, 2, 0, 128, 256)        # configs[3]'s worst case: more units than waves


def test_configs3_draw():
    """The benchmarked configs[3] draw (torch.randint(1024, 32769, (64,)) with seed 0)."""
    import torch
    ctx = torch.randint(1024, 32769, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    check(ctx, 2, 0, 128, 256)

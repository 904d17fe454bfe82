"""Pin for the CPU paged-KV-write oracle (oracle/kvcache.py): an explicit per-token loop."""

import torch

from oracle.kvcache import store_kvcache


def test_store_kvcache_matches_explicit_loop_and_skips_negative():
    pages, page, hkv, d, N = 5, 4, 2, 3, 9
    g = torch.Generator().manual_seed(0)
    key = torch.randn(N, hkv, d, generator=g)
    val = torch.randn(N, hkv, d, generator=g)
    slots = torch.tensor([7, -1, 0, 19, 3, -1, 12, 8, 1], dtype=torch.int32)
    kc = torch.full((pages, page, hkv, d), float("nan"))
    vc = torch.full((pages, page, hkv, d), float("nan"))
    store_kvcache(key, val, kc, vc, slots)
    ek = torch.full_like(kc, float("nan"))
    ev = torch.full_like(vc, float("nan"))
    for i, s in enumerate(slots.tolist()):
        if s >= 0:
            ek[s // page, s % page] = key[i]
            ev[s // page, s % page] = val[i]
    assert torch.equal(torch.nan_to_num(kc, 7.0), torch.nan_to_num(ek, 7.0))
    assert torch.equal(torch.nan_to_num(vc, 7.0), torch.nan_to_num(ev, 7.0))

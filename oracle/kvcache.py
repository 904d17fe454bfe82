"""CPU oracle for the paged KV write (test infrastructure only; see ``oracle/__init__``)."""

import torch


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    """Scatter token rows into the paged cache IN PLACE.

    Token i's (Hkv, d) key/value row goes to flat cache row ``slot_mapping[i]``
    (slot = page * page_size + offset); negative slots are skipped.  This is the
    reference's CPU route, a masked ``index_put`` on the flattened cache
    (``inference/layers/attention.py:41-49``)."""
    n, hkv, d = key.shape
    keep = slot_mapping.long() >= 0
    rows = slot_mapping.long()[keep]
    k_cache.view(-1, hkv, d)[rows] = key[keep].to(k_cache.dtype)
    v_cache.view(-1, hkv, d)[rows] = value[keep].to(v_cache.dtype)

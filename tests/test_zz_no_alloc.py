"""The no-allocation paged-decode entry point (``atma_polar_attention_decode_noalloc``,
no counterpart in the reference; for callers that cannot allocate: graph capture,
tight serving loops).  Called through the C ABI, its outputs equal the workspace entry
point's (``polar_attention_decode``) bit for bit -- the same kernels run -- on two calls
in a row, the second with a smaller input, so the fixed scratch array's leftover
contents from the first call never leak into the second; and under HIP graph capture:
the first call on the device made inside a capture (in a child process), and replays
interleaved with other calls that reuse the array."""

import pytest
import torch

from atma_amd import _lib
from tests.helpers import polar_params

pytestmark = pytest.mark.gpu


def _case(dev, B, ctx_hi, seed, dtype=torch.bfloat16, Hq=8, Hkv=2, d=128, page=256):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(1, ctx_hi + 1, (B,), generator=g)
    npg = (ctx + page - 1) // page
    pool = int(npg.sum()) + 3
    perm = torch.randperm(pool, generator=g).int()
    max_pages = int(npg.max())
    bt = torch.full((B, max_pages), -1, dtype=torch.int32)
    used = 0
    for b in range(B):
        bt[b, :npg[b]] = perm[used:used + npg[b]]
        used += int(npg[b])
    kc = torch.randn(pool, page, Hkv, d, generator=g).to(dtype)
    vc = torch.randn(pool, page, Hkv, d, generator=g).to(dtype)
    q = torch.randn(B, Hq, d, generator=g).to(dtype)
    p = polar_params(Hq, d, seed=seed, prior=True)
    return (q.to(dev), kc.to(dev), vc.to(dev), bt.to(dev), ctx.int().to(dev),
            {n: t.to(dev) for n, t in p.items()})


def _noalloc(q, kc, vc, bt, ctx, p, window=0, eps=1e-6):
    lib = _lib.load()
    B, Hq, d = q.shape
    num_pages, page, Hkv, _ = kc.shape
    c = torch.empty((B, Hq, d), device=q.device, dtype=q.dtype)
    mag = torch.empty((B, Hq), device=q.device, dtype=q.dtype)
    rc = lib.atma_polar_attention_decode_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), num_pages, page, Hkv,
        bt.data_ptr(), bt.stride(0), bt.shape[1], ctx.data_ptr(), p["v_null"].data_ptr(),
        p["null_base"].data_ptr(), p["null_slope_raw"].data_ptr(), p["len_gain_raw"].data_ptr(),
        p["mag_beta_raw"].data_ptr(), c.data_ptr(), mag.data_ptr(), B, Hq, d, _lib.dtype_code(q.dtype),
        window, eps, _lib.stream_handle(q.device))
    _lib.check(rc, "polar_attention_decode_noalloc")
    return c, mag


def test_noalloc_decode_equals_workspace_entry_point(dev):
    from atma_amd.kernel import polar_attention_decode
    for i, (B, ctx_hi, seed) in enumerate([(48, 20000, 1), (7, 3000, 2)]):   # second call smaller
        print(f"[no-alloc] call {i}: B={B} ctx<= {ctx_hi}", flush=True)
        q, kc, vc, bt, ctx, p = _case(dev, B, ctx_hi, seed)
        c_ref, m_ref = polar_attention_decode(q, kc, vc, bt, ctx, **p)
        c, m = _noalloc(q, kc, vc, bt, ctx, p)
        torch.cuda.synchronize()
        assert torch.equal(c, c_ref) and torch.equal(m, m_ref), i
        assert torch.isfinite(c.float()).all()


def test_noalloc_decode_first_call_inside_graph_capture(dev):
    """The entry point's first call on the device made under ``torch.cuda.graph`` capture
    (a fresh child process, so no earlier call has looked the scratch address up), replayed
    three times: every replay equals the workspace entry point bit for bit."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    child = Path(__file__).resolve().parent / "noalloc_capture_child.py"
    r = subprocess.run([sys.executable, "-u", str(child)], capture_output=True, text=True, timeout=110,
                       env=dict(os.environ))
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK")


def test_noalloc_decode_replayed_from_a_graph_equals_eager(dev):
    """Captured after earlier calls (the address already known): replays equal the workspace
    entry point, with a different launch between replays reusing the same scratch array."""
    from atma_amd.kernel import polar_attention_decode
    q, kc, vc, bt, ctx, p = _case(dev, 16, 5000, 9)
    c_ref, m_ref = polar_attention_decode(q, kc, vc, bt, ctx, **p)
    _noalloc(q, kc, vc, bt, ctx, p)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        c, m = _noalloc(q, kc, vc, bt, ctx, p)
    other = _case(dev, 5, 2000, 10)
    for i in range(3):
        _noalloc(*other)                         # overwrites the scratch records in between
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, c_ref) and torch.equal(m, m_ref), i

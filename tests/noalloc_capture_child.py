"""Child process of ``tests/test_zz_no_alloc.py``: the FIRST call of the no-allocation
decode entry point on the device is made inside a HIP graph capture (so its one-time
scratch-address lookup runs under capture), then the graph is replayed three times with
eager work in between and each replay is compared with the workspace entry point, bit for
bit.  Prints ``OK`` and exits 0 on success."""

import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

from tests.test_zz_no_alloc import _case, _noalloc  # noqa: E402


def main():
    from atma_amd.kernel import polar_attention_decode
    dev = torch.device("cuda:0")
    q, kc, vc, bt, ctx, p = _case(dev, 24, 9000, 7)
    c_ref, m_ref = polar_attention_decode(q, kc, vc, bt, ctx, **p)     # workspace entry point
    torch.cuda.synchronize()
    print("[no-alloc capture] capturing the first no-alloc call", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        c, m = _noalloc(q, kc, vc, bt, ctx, p)
    torch.cuda.synchronize()
    for i in range(3):
        c.fill_(float("nan"))
        m.fill_(float("nan"))
        junk = torch.randn(1 << 20, device=dev).sum()                  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        ok = torch.equal(c, c_ref) and torch.equal(m, m_ref)
        print(f"[no-alloc capture] replay {i}: {'equal' if ok else 'DIFFERENT'} ({float(junk):.1f})", flush=True)
        if not ok:
            return 1
    print("OK", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

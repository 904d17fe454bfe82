"""GPU parity of the decode-time conv step (causal_conv1d_decode_step,
kernel/causal_conv1d_triton.py:18-63) against the fp32/fp64 oracle of the reference's
torch route (inference/models/atma.py:181-188): outputs within one rounding of the
input dtype (fp32: 1e-6 relative), the rolled state rows bitwise (a pure copy), rows
of other slots untouched, an out-of-range slot leaving the table alone (NaN output),
and HIP-graph replays equal to eager steps."""

import pytest
import torch

from helpers import max_abs
from oracle import conv as OC

pytestmark = pytest.mark.gpu


def _case(B, D, K, S, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, D, generator=g).to(dtype)
    w = (torch.randn(D, K, generator=g) * 0.5).to(dtype)
    table = torch.randn(S, D, max(K - 1, 0), generator=g).to(dtype)
    slots = torch.randperm(S, generator=g)[:B]
    return x, w, table, slots


@pytest.mark.parametrize("dtype,K,D", [(torch.float32, 4, 300), (torch.bfloat16, 4, 1024),
                                       (torch.float16, 3, 257), (torch.bfloat16, 1, 64)])
def test_conv_step_vs_oracle(dev, dtype, K, D):
    from atma_amd.kernel import causal_conv1d_decode_step
    B, S = 5, 9
    x, w, table, slots = _case(B, D, K, S, dtype, seed=D + K)
    t_dev = table.to(dev)
    out = causal_conv1d_decode_step(x.to(dev), w.to(dev), slots.to(dev), t_dev)
    res = causal_conv1d_decode_step(x.to(dev), w.to(dev), slots.to(dev), table.clone().to(dev),
                                    residual=True)
    torch.cuda.synchronize()
    ref_table = table.clone()
    ref = OC.causal_conv1d_decode_step(x.double(), w.double(), slots, ref_table)
    tol = 1e-6 if dtype == torch.float32 else (2 ** -7 if dtype == torch.bfloat16 else 2 ** -10)
    scale = ref.abs().max().item()
    assert out.dtype == dtype and max_abs(out, ref) <= tol * scale
    assert max_abs(res, ref + x.double()) <= 2 * tol * (scale + x.double().abs().max().item())
    if K > 1:
        assert torch.equal(t_dev.cpu(), ref_table)   # rolled rows bitwise, others untouched


def test_conv_step_invalid_slot_leaves_table(dev):
    from atma_amd.kernel import causal_conv1d_decode_step
    x, w, table, _ = _case(3, 128, 4, 4, torch.bfloat16, seed=2)
    slots = torch.tensor([1, 7, -1])           # 7 and -1 are outside the 4-row table
    t_dev = table.to(dev)
    out = causal_conv1d_decode_step(x.to(dev), w.to(dev), slots.to(dev), t_dev).cpu()
    ref_table = table.clone()
    ref = OC.causal_conv1d_decode_step(x[:1].double(), w.double(), slots[:1], ref_table)
    assert torch.isnan(out[1:].float()).all() and not torch.isnan(out[0].float()).any()
    assert max_abs(out[:1], ref) <= 2 ** -7 * ref.abs().max().item()
    assert torch.equal(t_dev.cpu(), ref_table)


def test_conv_step_graph_replays_match_eager(dev):
    """Captured once, replayed several times with eager work and syncs in between; each
    replay advances the state like an eager step would."""
    from atma_amd.kernel import causal_conv1d_decode_step
    x, w, table, slots = _case(4, 512, 4, 6, torch.bfloat16, seed=3)
    x, w, slots = x.to(dev), w.to(dev), slots.to(dev)
    t_graph, t_eager = table.to(dev), table.to(dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        causal_conv1d_decode_step(x, w, slots, table.clone().to(dev))   # warm-up on a scratch table
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = causal_conv1d_decode_step(x, w, slots, t_graph)
    for _ in range(3):
        graph.replay()
        out_e = causal_conv1d_decode_step(x, w, slots, t_eager)
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e) and torch.equal(t_graph, t_eager)

"""GPU parity: paged KV write (bit-exact) and the gated-delta decode step."""

import pytest
import torch

from helpers import max_abs, rel_err
from oracle import gated_delta as OG
from oracle import kvcache as OK

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_store_kvcache_bitwise(dev, dtype):
    from atma_amd.layers.attention import store_kvcache
    pages, page, hkv, d, N = 9, 16, 2, 128, 40
    g = torch.Generator().manual_seed(1)
    fused = torch.randn(N, 3, hkv, d, generator=g).to(dtype)       # key/value as strided views
    key, val = fused[:, 0], fused[:, 2]
    perm = torch.randperm(pages * page, generator=g)[:N].to(torch.int32)
    perm[3] = -1
    perm[17] = -1
    kc = torch.randn(pages, page, hkv, d, generator=g).to(dtype)
    vc = torch.randn(pages, page, hkv, d, generator=g).to(dtype)
    ek, ev = kc.clone(), vc.clone()
    OK.store_kvcache(key, val, ek, ev, perm)
    dk_, dv_ = kc.to(dev), vc.to(dev)
    store_kvcache(key.to(dev), val.to(dev), dk_, dv_, perm.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(dk_.cpu().view(torch.uint8), ek.view(torch.uint8))
    assert torch.equal(dv_.cpu().view(torch.uint8), ev.view(torch.uint8))


@pytest.mark.parametrize("dtype,D", [(torch.float32, 128), (torch.bfloat16, 128), (torch.float32, 64),
                                     (torch.float16, 128)])
def test_gated_delta_step_matches_oracle(dev, dtype, D):
    from atma_amd.kernel import gated_delta_decode_step
    B, H, max_seqs = 6, 8, 11
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(B, H, D, generator=g).to(dtype) for _ in range(3))
    gamma = torch.rand(B, H, generator=g)
    beta = torch.rand(B, H, generator=g)
    table = torch.randn(max_seqs, H, D, D, generator=g)
    slots = torch.randperm(max_seqs, generator=g)[:B]
    ref_table = table.clone()
    r_ref = OG.gated_delta_decode_step(q, k, v, gamma, beta, ref_table, slots)
    t_dev = table.to(dev)
    r = gated_delta_decode_step(q.to(dev), k.to(dev), v.to(dev), gamma.to(dev), beta.to(dev), t_dev,
                                slots.to(dev))
    torch.cuda.synchronize()
    # fp32 arithmetic on both sides (reference bar: 2e-4 out, 2e-5 state; ours is tighter)
    assert max_abs(r, r_ref) < 2e-5
    assert max_abs(t_dev, ref_table) < 2e-6
    untouched = [i for i in range(max_seqs) if i not in slots.tolist()]
    assert torch.equal(t_dev.cpu()[untouched], table[untouched])


def test_gated_delta_step_repeated_calls_track_oracle(dev):
    """Ten consecutive steps on the same slots (state carried in place)."""
    from atma_amd.kernel import gated_delta_decode_step
    B, H, D = 4, 8, 128
    g = torch.Generator().manual_seed(5)
    table = torch.zeros(B, H, D, D)
    t_dev = table.to(dev)
    slots = torch.arange(B)
    for _ in range(10):
        q, k, v = (torch.randn(B, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
        gamma = torch.sigmoid(torch.randn(B, H, generator=g) + 3.9)
        beta = torch.sigmoid(torch.randn(B, H, generator=g))
        r_ref = OG.gated_delta_decode_step(q, k, v, gamma, beta, table, slots)
        r = gated_delta_decode_step(q.to(dev), k.to(dev), v.to(dev), gamma.to(dev), beta.to(dev),
                                    t_dev, slots.to(dev))
        assert rel_err(r, r_ref) < 1e-5
    assert max_abs(t_dev, table) < 1e-5


@pytest.mark.parametrize("dtype,D", [(torch.float32, 128), (torch.bfloat16, 64)])
def test_gated_delta_step_grouped_kv_heads(dev, dtype, D):
    """k / v with Hkv < H heads == the expanded call (bitwise, outputs and table), and
    both track the oracle on the expanded tensors."""
    from atma_amd.kernel import gated_delta_decode_step
    B, H, Hkv, max_seqs = 5, 8, 2, 7
    g = torch.Generator().manual_seed(9)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    k, v = (torch.randn(B, Hkv, D, generator=g).to(dtype) for _ in range(2))
    gamma = torch.rand(B, H, generator=g)
    beta = torch.rand(B, H, generator=g)
    table = torch.randn(max_seqs, H, D, D, generator=g) * 0.1
    slots = torch.randperm(max_seqs, generator=g)[:B]
    kx, vx = (t.repeat_interleave(H // Hkv, 1) for t in (k, v))
    t1, t2 = table.to(dev), table.to(dev)
    args = (gamma.to(dev), beta.to(dev))
    r1 = gated_delta_decode_step(q.to(dev), k.to(dev), v.to(dev), *args, t1, slots.to(dev))
    r2 = gated_delta_decode_step(q.to(dev), kx.to(dev), vx.to(dev), *args, t2, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(r1, r2) and torch.equal(t1, t2)
    ref_table = table.clone()
    r_ref = OG.gated_delta_decode_step(q, kx, vx, gamma, beta, ref_table, slots)
    assert max_abs(r1, r_ref) < 2e-5 and max_abs(t1, ref_table) < 2e-6


@pytest.mark.parametrize("decay_as_prob", [False, True])
def test_gate_activations_vs_torch(dev, decay_as_prob):
    """The fused gate kernel == torch's logsigmoid / sigmoid of the biased logits
    (TitansMemory, model/blocks.py:426-490), including saturated logits on both sides."""
    from atma_amd.kernel import gated_delta_gates
    g = torch.Generator().manual_seed(5)
    zg = torch.randn(3, 100, 8, generator=g) * 6
    zb = torch.randn(3, 100, 8, generator=g) * 6
    zg[0, :4, 0] = torch.tensor([-200.0, 200.0, -3.9, 0.0])
    zb[0, :4, 0] = torch.tensor([-200.0, 200.0, 0.0, 1e-3])
    ga, be = gated_delta_gates(zg.to(dev), zb.to(dev), 3.9, 0.5, decay_as_prob=decay_as_prob)
    ref_g = torch.nn.functional.logsigmoid(zg.double() + 3.9)
    if decay_as_prob:
        ref_g = ref_g.exp()
    ref_b = torch.sigmoid(zb.double() + 0.5)
    assert ga.dtype == torch.float32 and be.dtype == torch.float32
    assert torch.allclose(ga.cpu().double(), ref_g, rtol=2e-6, atol=1e-30)
    assert torch.allclose(be.cpu().double(), ref_b, rtol=2e-6, atol=1e-30)

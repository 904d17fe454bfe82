"""The conv decode-step oracle against what the mathematics fixes: K = 1 is a plain
scale, a unit tap at position j returns the state column j (or x for j = K - 1), the
state rolls left by one with x appended, and K steps from zero state reproduce the
causal depthwise convolution F.conv1d of the last K inputs."""

import torch
import torch.nn.functional as F

from oracle import conv as OC


def test_unit_taps_select_state_columns_and_roll():
    g = torch.Generator().manual_seed(0)
    B, D, K, S = 3, 5, 4, 6
    x = torch.randn(B, D, generator=g)
    table = torch.randn(S, D, K - 1, generator=g)
    slots = torch.tensor([4, 0, 2])
    for j in range(K):
        t = table.clone()
        w = torch.zeros(D, K)
        w[:, j] = 1.0
        out = OC.causal_conv1d_decode_step(x, w, slots, t)
        want = x if j == K - 1 else table[slots][:, :, j]
        assert torch.equal(out, want)
        assert torch.equal(t[slots], torch.cat([table[slots][:, :, 1:], x.unsqueeze(2)], 2))
        untouched = [i for i in range(S) if i not in slots.tolist()]
        assert torch.equal(t[untouched], table[untouched])


def test_k1_is_a_scale():
    x = torch.randn(2, 7)
    w = torch.randn(7, 1)
    assert torch.equal(OC.causal_conv1d_decode_step(x, w, torch.tensor([0, 1]), torch.empty(0)), x * w[:, 0])


def test_steps_from_zero_state_equal_conv1d():
    g = torch.Generator().manual_seed(1)
    D, K, T = 6, 4, 9
    seq = torch.randn(1, D, T, generator=g, dtype=torch.float64)
    w = torch.randn(D, K, generator=g, dtype=torch.float64)
    ref = F.conv1d(F.pad(seq, (K - 1, 0)), w.unsqueeze(1), groups=D)[0]      # (D, T)
    table = torch.zeros(1, D, K - 1, dtype=torch.float64)
    for t in range(T):
        out = OC.causal_conv1d_decode_step(seq[:, :, t], w, torch.tensor([0]), table)
        assert torch.allclose(out[0], ref[:, t], atol=1e-12)

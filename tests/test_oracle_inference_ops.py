"""The inference-fusion oracle against what fixes it independently:

* squared_relu_gate equals torch's eager ``gate * x.relu().square()`` bit for bit (the
  reference test's own expected form, ``tests/test_decode_kernels.py:54-62``): eager bf16
  rounds the square before the multiply exactly as the reference kernel does;
* softcap_logits equals eager ``15 * x * (x^2 + 225).rsqrt()`` (``:64-66``) up to at most
  one bf16 unit in the last place on a tiny fraction of elements (torch's rsqrt and the
  correctly rounded 1 / sqrt may differ by one float32 ulp before the bf16 rounding), and
  is odd, bounded by 15, monotone (to float32 rounding) and zero at zero;
* packed_causal_conv1d equals F.conv1d of each sequence alone (zero left padding) in
  float64, and writes each sequence's last K - 1 inputs (zero-padded) as its state, on
  the reference test's ragged layout (``tests/test_decode_kernels.py:135-160``)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import inference_ops as OI


def test_round_bf16_matches_torch():
    g = torch.Generator().manual_seed(0)
    a = torch.cat([torch.randn(100000, generator=g) * 10.0 ** torch.randint(-6, 6, (100000,), generator=g),
                   torch.tensor([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, float("inf"), 3.4e38])])
    assert torch.equal(torch.from_numpy(OI.round_bf16(a.numpy())), a.to(torch.bfloat16).float())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_squared_relu_gate_is_eager_form(dtype):
    torch.manual_seed(5)
    packed = torch.randn(32, 1024).to(dtype)
    x, gate = packed.chunk(2, dim=-1)
    assert torch.equal(OI.squared_relu_gate(x, gate), gate * x.relu().square())


def test_squared_relu_gate_fp16_rounds_once():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(64, 96, generator=g).half()
    gate = torch.randn(64, 96, generator=g).half()
    want = (gate.double() * x.double().clamp_min(0) ** 2).half()   # one rounding of the exact value
    got = OI.squared_relu_gate(x, gate)
    # fp32 intermediate then one fp16 rounding: equal except on rare double-rounding ties
    assert (got != want).float().mean() < 1e-3
    assert (got.float() - want.float()).abs().max() <= 2 ** -10 * want.float().abs().max()


def test_softcap_against_eager_and_invariants():
    torch.manual_seed(5)
    logits = torch.randn(32, 50304).to(torch.bfloat16)
    eager = 15.0 * logits * (logits.square() + 225.0).rsqrt()
    got = OI.softcap_logits(logits)
    diff = (got.float() - eager.float()).abs()
    ulp = torch.finfo(torch.bfloat16).eps * eager.float().abs().clamp_min(1e-30)
    assert (diff <= ulp).all()
    assert (got != eager).float().mean() < 1e-3
    x = torch.linspace(-1e4, 1e4, 200001)
    y = OI.softcap_logits(x)
    assert torch.equal(OI.softcap_logits(-x), -y)
    # monotone up to the float32 rounding of the separately rounded product
    assert (y.abs() < 15.0).all() and (y[1:] >= y[:-1] - 4 * 2 ** -24 * 15).all()
    assert OI.softcap_logits(torch.zeros(3)).eq(0).all()
    small = torch.tensor([1e-3, -2e-3])
    assert torch.allclose(OI.softcap_logits(small), small, rtol=1e-5)
    f32 = torch.randn(4096)
    exact = (15.0 * f32.double() / (f32.double() ** 2 + 225.0).sqrt()).float()
    assert torch.allclose(OI.softcap_logits(f32), exact, rtol=3e-7, atol=0)


def _maps(lengths):
    starts, ends, slots, p = [], [], [], 0
    for slot, n in enumerate(lengths):
        starts += [p] * n
        ends += [p + n] * n
        slots += [slot] * n
        p += n
    return [torch.tensor(v, dtype=torch.int32) for v in (starts, ends, slots)]


@pytest.mark.parametrize("K,lengths,C", [(4, [1, 3, 7, 17], 257), (3, [2, 40, 1, 33], 16)])
def test_packed_conv_is_per_sequence_conv1d(K, lengths, C):
    g = torch.Generator().manual_seed(8)
    total = sum(lengths)
    x = torch.randn(total, C, generator=g)
    w = torch.randn(C, K, generator=g)
    state = torch.full((len(lengths) + 1, C, K - 1), 7.0)
    out = OI.packed_causal_conv1d(x, w, state, *_maps(lengths))
    p = 0
    for slot, n in enumerate(lengths):
        seq = x[p:p + n].double().t().unsqueeze(0)                     # (1, C, n)
        ref = F.conv1d(F.pad(seq, (K - 1, 0)), w.double().unsqueeze(1), groups=C)[0].t()
        assert torch.allclose(out[p:p + n].double(), ref, rtol=1e-6, atol=1e-6)
        tail = F.pad(x[p:p + n].t(), (K - 1, 0))[:, -(K - 1):]          # last K-1 inputs, zero-padded
        assert torch.equal(state[slot], tail)
        p += n
    assert state[len(lengths)].eq(7.0).all()                            # a slot no sequence names

"""The global layer's per-head glue and the LFM2 prefill conv as fused kernels
(``kernel/layer_fusions.py``; no reference counterpart, each the one-launch form of a chain
of the reference's eager ops) against those chains in torch on the same 16-bit inputs:

* ``head_rms_norm`` on the strided q half of a q|gate projection and on contiguous k: within
  one bf16 ulp of ``F.rms_norm`` (the reciprocal square root's last bit);
* ``global_gate`` at prefill layouts (c head-major from Polar, the gate a strided view, the
  readout in 16 bits or fp32): within 1e-2 relative of ``c * sigmoid(gate)`` and
  ``rms_norm(r) * sigmoid(mem_gate)`` (a sigmoid or norm one ulp apart carries through a
  product), the gate-only form equal to the first half;
* ``lfm2_conv_packed``: bit for bit the chain ``b * x`` -> ``packed_causal_conv1d`` ->
  ``c * (.)`` on ragged packed sequences, state rows included.
"""

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import rel_err

pytestmark = pytest.mark.gpu


def _g(dev, seed):
    return torch.Generator(device=dev).manual_seed(seed)


def _ulps(a, b):
    a, b = a.double(), b.double()
    spacing = torch.exp2(torch.floor(torch.log2(b.abs().clamp_min(1e-30))) - 7)
    return ((a - b).abs() / spacing).max().item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("rows", [1, 300, 4097])
def test_head_rms_norm_strided_q(dev, rows, d, dtype):
    from atma_amd.kernel.layer_fusions import head_rms_norm
    H = 8
    y = torch.randn(rows, H, 2 * d, device=dev, generator=_g(dev, rows + d)).to(dtype)
    q = y[..., :d]                                       # the q half of each head, in place
    out = head_rms_norm(q, torch.finfo(torch.float32).eps)
    assert out.is_contiguous() and out.shape == q.shape
    ref = F.rms_norm(q.float(), (d,), eps=torch.finfo(torch.float32).eps)
    assert _ulps(out, ref) <= 1.0 if dtype == torch.bfloat16 else rel_err(out, ref) <= 2e-3
    k = torch.randn(2, rows, 2, d, device=dev, generator=_g(dev, 7)).to(dtype)
    assert rel_err(head_rms_norm(k, 1e-6), F.rms_norm(k.float(), (d,), eps=1e-6)) <= 1e-2


@pytest.mark.parametrize("r_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 128])
def test_global_gate_prefill_layout(dev, d, r_dtype):
    from atma_amd.kernel.layer_fusions import global_gate
    g = _g(dev, d)
    B, T, H = 2, 77, 8
    rows = B * T
    c_head_major = torch.randn(B, H, T, d, device=dev, generator=g).bfloat16()
    c = c_head_major.transpose(1, 2)                    # (B, T, H, d) view, as the layer passes it
    qg = torch.randn(rows, H, 2 * d, device=dev, generator=g).bfloat16()
    gate = qg[..., d:]                                   # strided view of the projection
    r = (torch.randn(rows, H, d, device=dev, generator=g) * 0.1).to(r_dtype)
    mgate = torch.randn(rows, H * d, device=dev, generator=g).bfloat16()
    xa, xm = global_gate(c, gate, r, mgate, torch.finfo(torch.float32).eps)
    ref_a = (c.reshape(rows, H, d) * torch.sigmoid(gate)).reshape(rows, H * d)
    ref_m = F.rms_norm(r, (d,)).reshape(rows, H * d).to(torch.bfloat16) * torch.sigmoid(mgate)
    assert rel_err(xa, ref_a) <= 1e-2 and rel_err(xm, ref_m) <= 1e-2
    only, none = global_gate(c, gate, None, mgate, 0.0)
    assert none is None and torch.equal(only, xa)


@pytest.mark.parametrize("K", [3, 4])
def test_lfm2_conv_packed_equals_eager_chain(dev, K):
    from atma_amd.kernel import packed_causal_conv1d
    from atma_amd.kernel.layer_fusions import lfm2_conv_packed
    g = _g(dev, K)
    lens = [1, 3, 7, 17, 40]
    D, S = 256, 8
    total = sum(lens)
    bcx = torch.randn(total, 3 * D, device=dev, generator=g).bfloat16()
    w = (torch.randn(D, K, device=dev, generator=g) * 0.5).bfloat16()
    starts, ends, slots, pos = [], [], [], 0
    for i, n in enumerate(lens):
        starts += [pos] * n
        ends += [pos + n] * n
        slots += [7 - i] * n
        pos += n
    maps = [torch.tensor(m, device=dev, dtype=torch.int32) for m in (starts, ends, slots)]
    t_fused = torch.full((S, D, K - 1), 9.0, device=dev).bfloat16()
    t_eager = t_fused.clone()
    out = lfm2_conv_packed(bcx, w, t_fused, *maps)
    b, c, x = bcx.chunk(3, dim=-1)
    ref = c * packed_causal_conv1d(b * x, w, t_eager, *maps)
    assert torch.equal(out, ref)
    assert torch.equal(t_fused, t_eager)

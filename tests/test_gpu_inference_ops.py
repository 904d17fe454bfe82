"""GPU parity of the inference fusions (kernel/inference_ops_triton.py) against the
numpy oracle: squared_relu_gate and softcap_logits bitwise in bf16 / fp16 / fp32, on
the 16-byte vector path (the halves of one fc output, contiguous logits) and on the
element path (odd widths, unaligned views, a length that leaves a tail); the packed
depthwise convolution bitwise in the output dtype with its state rows bitwise, on the
reference test's ragged layout and on sequences that cross strip boundaries."""

import pytest
import torch

from oracle import inference_ops as OI

pytestmark = pytest.mark.gpu

DT = [torch.bfloat16, torch.float16, torch.float32]


def _eq(a, b):
    return torch.equal(a.cpu(), b.cpu()) or torch.equal(a.cpu().isnan(), b.cpu().isnan()) and \
        torch.equal(a.cpu().nan_to_num(), b.cpu().nan_to_num())


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("shape,halves", [((32, 1024), True), ((7, 257), False), ((64, 4096), False),
                                          ((5, 514), True), ((9, 4112), True)])
def test_squared_relu_gate_bitwise(dev, dtype, shape, halves):
    from atma_amd.kernel import squared_relu_gate
    g = torch.Generator().manual_seed(shape[1])
    if halves:
        packed = torch.randn(*shape, generator=g).to(dtype)
        x, gate = packed.chunk(2, dim=-1)
        xd, gd = packed.to(dev).chunk(2, dim=-1)
    else:
        x = torch.randn(*shape, generator=g).to(dtype)
        gate = torch.randn(*shape, generator=g).to(dtype)
        x[0, :4] = torch.tensor([float("nan"), float("inf"), -0.0, -float("inf")]).to(dtype)
        xd, gd = x.to(dev), gate.to(dev)
    out = squared_relu_gate(xd, gd)
    assert out.is_contiguous() and out.dtype == dtype
    assert _eq(out, OI.squared_relu_gate(x, gate))
    if dtype == torch.bfloat16:      # the reference test's own expected form
        assert _eq(out, gate * x.relu().square())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_squared_relu_gate_stream_bitwise(dev, dtype):
    """Rows of at least 256 vectors run one row per workgroup row; an operand stream beyond
    256 MiB (here 270 MB) takes non-temporal loads and stores. Bitwise equal to the oracle."""
    from atma_amd.kernel import squared_relu_gate
    g = torch.Generator().manual_seed(5)
    packed = torch.randn(11000, 8192, generator=g).to(dtype)
    packed[3, :4] = torch.tensor([float("nan"), float("inf"), -0.0, -float("inf")]).to(dtype)
    x, gate = packed.chunk(2, dim=-1)
    xd, gd = packed.to(dev).chunk(2, dim=-1)
    assert 3 * x.numel() * x.element_size() > 256 << 20
    out = squared_relu_gate(xd, gd)
    assert _eq(out, OI.squared_relu_gate(x, gate))


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("n,offset", [(32 * 50304, 0), (3 * 1001, 0), (4099, 1)])
def test_softcap_bitwise(dev, dtype, n, offset):
    from atma_amd.kernel import softcap_logits
    g = torch.Generator().manual_seed(n)
    flat = (torch.randn(n + offset, generator=g) * 20).to(dtype)
    flat[offset:offset + 3] = torch.tensor([0.0, 1e30, -1e30]).to(dtype)
    x = flat[offset:]
    out = softcap_logits(flat.to(dev)[offset:])
    assert out.dtype == dtype and out.shape == x.shape
    assert _eq(out, OI.softcap_logits(x))


def _maps(lengths, slots):
    starts, ends, sl, p = [], [], [], 0
    for slot, n in zip(slots, lengths):
        starts += [p] * n
        ends += [p + n] * n
        sl += [slot] * n
        p += n
    return [torch.tensor(v, dtype=torch.int32) for v in (starts, ends, sl)]


@pytest.mark.parametrize("dtype,sdtype,K,C,lengths", [
    (torch.bfloat16, torch.bfloat16, 4, 257, [1, 3, 7, 17]),            # the reference test's layout
    (torch.bfloat16, torch.bfloat16, 3, 1024, [33, 1, 64, 100, 2, 31]),
    (torch.float16, torch.float32, 4, 256, [65, 5, 40]),
    (torch.float32, torch.float32, 4, 24, [1, 2, 3]),
    (torch.bfloat16, torch.bfloat16, 4, 1024, [2048, 1500, 548]),
])
def test_packed_conv_bitwise(dev, dtype, sdtype, K, C, lengths):
    from atma_amd.kernel import packed_causal_conv1d
    g = torch.Generator().manual_seed(C + K)
    total = sum(lengths)
    x = torch.randn(total, C, generator=g).to(dtype)
    w = torch.randn(C, K, generator=g).to(dtype)
    S = len(lengths) + 3
    slots = torch.randperm(S, generator=g)[:len(lengths)].tolist()
    table = torch.randn(S, C, K - 1, generator=g).to(sdtype)
    maps = _maps(lengths, slots)
    t_dev = table.to(dev)
    out = packed_causal_conv1d(x.to(dev), w.to(dev), t_dev, *[m.to(dev) for m in maps])
    ref_table = table.clone()
    ref = OI.packed_causal_conv1d(x, w, ref_table, *maps)
    assert out.dtype == dtype
    assert torch.equal(out.cpu(), ref)
    assert torch.equal(t_dev.cpu(), ref_table)                # named rows rewritten, others untouched


def test_packed_conv_strided_input_and_bad_slot(dev):
    from atma_amd.kernel import packed_causal_conv1d
    g = torch.Generator().manual_seed(3)
    lengths, C, K = [9, 4], 64, 4
    big = torch.randn(sum(lengths), 3 * C, generator=g).to(torch.bfloat16)
    x = big[:, C:2 * C]                                       # a column slice: row stride 3 C
    w = torch.randn(C, K, generator=g).to(torch.bfloat16)
    table = torch.randn(2, C, K - 1, generator=g).to(torch.bfloat16)
    maps = _maps(lengths, [1, 5])                             # slot 5 is outside the table
    t_dev = table.to(dev)
    out = packed_causal_conv1d(big.to(dev)[:, C:2 * C], w.to(dev), t_dev, *[m.to(dev) for m in maps])
    ref_table = table.clone()
    ref = OI.packed_causal_conv1d(x, w, ref_table, *maps)
    assert torch.equal(out.cpu(), ref)
    assert torch.equal(t_dev.cpu(), ref_table) and torch.equal(t_dev[0].cpu(), table[0])


@pytest.mark.parametrize("layout", ["contiguous", "transposed", "misaligned"])
def test_packed_conv_weight_layouts(dev, layout):
    """The taps of a contiguous, 16-byte aligned weight are read as whole 16-byte words; a
    transposed view and one whose storage starts 2 bytes in take the strided gather. All
    three equal the oracle bitwise."""
    from atma_amd.kernel import packed_causal_conv1d
    g = torch.Generator().manual_seed(11)
    lengths, C, K = [300, 1, 95, 40], 1024, 4
    x = torch.randn(sum(lengths), C, generator=g).to(torch.bfloat16)
    w = torch.randn(C, K, generator=g).to(torch.bfloat16)
    if layout == "contiguous":
        w_dev = w.to(dev)
    elif layout == "transposed":
        w_dev = w.t().contiguous().to(dev).t()                # strides (1, C)
    else:
        buf = torch.zeros(C * K + 1, dtype=torch.bfloat16, device=dev)
        buf[1:] = w.reshape(-1).to(dev)
        w_dev = buf[1:].view(C, K)                            # contiguous, 2 bytes off alignment
        assert w_dev.data_ptr() % 16 != 0
    table = torch.randn(6, C, K - 1, generator=g).to(torch.bfloat16)
    maps = _maps(lengths, [4, 0, 2, 5])
    t_dev = table.to(dev)
    out = packed_causal_conv1d(x.to(dev), w_dev, t_dev, *[m.to(dev) for m in maps])
    ref_table = table.clone()
    ref = OI.packed_causal_conv1d(x, w, ref_table, *maps)
    assert torch.equal(out.cpu(), ref)
    assert torch.equal(t_dev.cpu(), ref_table)


def test_reference_errors():
    from atma_amd.kernel import packed_causal_conv1d
    x = torch.zeros(4, 8)
    with pytest.raises(RuntimeError):
        packed_causal_conv1d(x, torch.zeros(8, 4), torch.zeros(1, 8, 3), *[torch.zeros(4)] * 3)

"""The decode projection ``linear_tokens`` (``atma_linear_tokens``, no reference counterpart:
the served model's projection of one token row per sequence) against an fp32 torch
reference of ``F.linear`` on the same 16-bit inputs: relative error max|a-b| / max|b| <= 1e-2
(one rounding of the output to 16 bits, fp32 accumulation), at the configs[4] decode shapes,
ragged row counts (1 .. 32, rows past M never written), strided rows, fp16, no bias; bitwise
deterministic; and the host ``Linear`` module takes it for inference calls on few rows."""

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import rel_err

pytestmark = pytest.mark.gpu

SHAPES = [(1024, 1024), (3072, 1024), (8192, 1024), (1024, 2048), (256, 1024), (2048, 1024), (4112, 1024),
          (50304, 1024), (32768, 512)]


def _ref(x, w, b):
    return F.linear(x.float(), w.float(), None if b is None else b.float())


@pytest.mark.parametrize("N,K", SHAPES, ids=lambda s: str(s))
@pytest.mark.parametrize("M", [1, 5, 16, 17, 32])
def test_linear_tokens_vs_fp32(dev, M, N, K):
    from atma_amd.kernel import linear_tokens
    g = torch.Generator(device=dev).manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, device=dev, generator=g).bfloat16()
    w = (torch.randn(N, K, device=dev, generator=g) * 0.02).bfloat16()
    b = (torch.randn(N, device=dev, generator=g) * 0.02).bfloat16()
    y = linear_tokens(x, w, b)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    assert rel_err(y, _ref(x, w, b)) <= 1e-2
    y2 = linear_tokens(x, w, b)
    assert torch.equal(y, y2)                      # deterministic


def test_linear_tokens_tile_width_does_not_change_results(dev):
    """The LM head's 50,304 outputs (32 features per workgroup) and the same rows as a
    narrower projection (the first 4,112 outputs: 16 per workgroup) give the same bits -- the
    per-feature sums do not depend on the tile width or the grid."""
    from atma_amd.kernel import linear_tokens
    g = torch.Generator(device=dev).manual_seed(11)
    x = torch.randn(32, 1024, device=dev, generator=g).bfloat16()
    w = (torch.randn(50304, 1024, device=dev, generator=g) * 0.02).bfloat16()
    b = (torch.randn(50304, device=dev, generator=g) * 0.02).bfloat16()
    full = linear_tokens(x, w, b)
    assert torch.equal(full[:, :4096], linear_tokens(x, w[:4096], b[:4096]))
    assert torch.equal(full[:, :4112], linear_tokens(x, w[:4112], b[:4112]))


def test_linear_tokens_fp16_strided_no_bias(dev):
    from atma_amd.kernel import linear_tokens
    g = torch.Generator(device=dev).manual_seed(3)
    M, N, K = 23, 1024, 2048
    big = torch.randn(M, K + 64, device=dev, generator=g).half()
    x = big[:, 32:32 + K]                          # row stride K + 64, 64-byte offset
    w = (torch.randn(N, K, device=dev, generator=g) * 0.02).half()
    y = linear_tokens(x, w, None)
    assert rel_err(y, _ref(x, w, None)) <= 1e-2
    out = torch.full((M + 3, N), float("nan"), device=dev, dtype=torch.float16)
    out[:M] = y
    assert torch.isnan(out[M:]).all()


def test_linear_tokens_rejects_unsupported(dev):
    from atma_amd.kernel import linear_tokens
    x = torch.randn(33, 1024, device=dev).bfloat16()
    w = torch.randn(64, 1024, device=dev).bfloat16()
    with pytest.raises(ValueError):
        linear_tokens(x, w)                        # 33 rows
    with pytest.raises(ValueError):
        linear_tokens(x[:4, :1000], w[:, :1000])   # K not 256 / 512 / 1024 / 2048
    with pytest.raises(ValueError):
        linear_tokens(torch.randn(4, 4096, device=dev).bfloat16(), torch.randn(64, 4096, device=dev).bfloat16())


def test_host_linear_takes_it_for_few_rows(dev):
    """Inference on <= 32 rows: the module's output equals linear_tokens bit for bit; with
    grad enabled (training) or many rows it is F.linear."""
    from atma_amd.kernel import linear_tokens
    from atma_amd.layers.global_attention import Linear
    torch.manual_seed(0)
    lin = Linear(1024, 3072).to(dev).bfloat16()
    x = torch.randn(32, 1024, device=dev).bfloat16()
    with torch.no_grad():
        y = lin(x)
        y3 = lin(x.view(4, 8, 1024))
        many = lin(torch.randn(64, 1024, device=dev).bfloat16())
    assert torch.equal(y, linear_tokens(x, lin.weight, lin.bias))
    assert torch.equal(y3.view(32, 3072), y)
    assert many.shape == (64, 3072)
    y_train = lin(x)                               # grad enabled: F.linear
    assert y_train.requires_grad and rel_err(y_train.detach(), y) <= 1e-2

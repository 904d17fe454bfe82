"""``linear_gated`` (the MLP's gated first projection over many rows, one MFMA kernel; no
reference counterpart as one call) against the chain it replaces -- ``F.linear`` then
``squared_relu_gate`` (``model/layers.py:19-31``, ``inference/models/atma.py:87-96``).

The reference chain is computed exactly: the projections in fp64, each rounded once to the
16-bit type (what a GEMM with fp32 accumulation returns up to its summation order), then the
activation's eager 16-bit arithmetic.  The kernel sums in fp32 in its own order, so a
projection value can round to the neighbouring 16-bit number where the exact sum lies
within fp32 error of a rounding boundary: at most 1 in 1,000 outputs may differ in bf16 (2 in
1,000 in fp16, whose spacing is finer), the whole within 1e-2 relative.  Rows past M (a partial
last tile) are never written.
"""

import pytest
import torch

from tests.helpers import rel_err

pytestmark = pytest.mark.gpu


def _reference(x, w, b):
    y = x.double() @ w.double().t()
    if b is not None:
        y = y + b.double()
    a, g = y.to(x.dtype).chunk(2, dim=-1)
    from atma_amd.kernel import squared_relu_gate
    return squared_relu_gate(a.contiguous(), g.contiguous())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,H,bias", [(4096, 1024, 4096, True), (5000, 256, 128, True), (8192, 512, 384, False),
                                        (4352, 128, 256, True), (4100, 2048, 640, True)])
def test_linear_gated_vs_exact_chain(dev, dtype, M, K, H, bias):
    from atma_amd.kernel.layer_fusions import linear_gated
    g = torch.Generator(device=dev).manual_seed(M + K + H)
    x = torch.randn(M, K, device=dev, generator=g).to(dtype)
    w = (torch.randn(2 * H, K, device=dev, generator=g) * K ** -0.5).to(dtype)
    b = (torch.randn(2 * H, device=dev, generator=g) * 0.1).to(dtype) if bias else None
    out = linear_gated(x, w, b)
    ref = _reference(x, w, b)
    differ = (out.view(torch.int16) != ref.view(torch.int16))
    # fp16's finer spacing meets fp32 summation error more often (0.10% at K = 2,048)
    assert differ.float().mean().item() <= (1e-3 if dtype == torch.bfloat16 else 2e-3), differ.float().mean().item()
    assert rel_err(out, ref) <= 1e-2


def test_linear_gated_partial_tile_writes_only_its_rows(dev):
    """The C ABI with an output of more rows than M: the rows past M keep their contents."""
    from atma_amd import _lib
    M, K, H = 300, 128, 128
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(2 * H, K, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    y = torch.full((M + 40, H), 7.0, device=dev, dtype=torch.bfloat16)
    rc = _lib.load().atma_linear_gated(x.data_ptr(), K, w.data_ptr(), K, None, y.data_ptr(), H, M, H, K,
                                       _lib.dtype_code(torch.bfloat16), _lib.stream_handle(x.device))
    assert rc == 0
    assert (y[M:] == 7.0).all()
    ref = _reference(x, w, None)
    assert (y[:M].view(torch.int16) != ref.view(torch.int16)).float().mean().item() <= 1e-3


def test_linear_gated_rejects(dev):
    from atma_amd.kernel.layer_fusions import linear_gated
    x = torch.zeros(4096, 1024, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        linear_gated(x, torch.zeros(8192, 512, device=dev, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):        # H not a multiple of 128: the library refuses
        linear_gated(x, torch.zeros(200, 1024, device=dev, dtype=torch.bfloat16))

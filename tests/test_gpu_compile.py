"""The training ops under ``torch.compile`` (the reference trains under it, ``train.py:86``,
with its gated-delta op opaque to the compiler, ``model/blocks.py:52-84``).

A module step calling ``polar_attention`` and the differentiable
``chunk_gated_delta_rule`` (raw gate logits, the memory branch's call) is compiled as
ONE graph (``fullgraph=True``: no graph break) with AOTAutograd tracing the backward
through the ops' fake implementations (``backend="aot_eager"``, so no code is
generated for the glue); its loss and every gradient match the eager step."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _step(q, k, v, n, vn, nb, ns, lg, mb, zg, zb):
    from atma_amd.kernel import chunk_gated_delta_rule, polar_attention
    c, mag = polar_attention(q, k, v, n, v_null=vn, null_base=nb, null_slope_raw=ns, len_gain_raw=lg,
                             mag_beta_raw=mb)
    o, _ = chunk_gated_delta_rule(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), zg, zb, scale=1.0,
                                  use_qk_l2norm_in_kernel=True, gate_bias=(3.9, 0.0))
    return (c.float() * c.float()).sum() + mag.float().sum() + o.float().square().sum()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_compiled_training_step_matches_eager(dev, dtype):
    B, H, Hkv, T, d = 2, 8, 2, 200, 128
    g = torch.Generator().manual_seed(3)

    def leaves():
        gg = torch.Generator().manual_seed(3)
        xs = [torch.randn(B, H, T, d, generator=gg), torch.randn(B, Hkv, T, d, generator=gg),
              torch.randn(B, Hkv, T, d, generator=gg)]
        xs = [x.to(dev, dtype).requires_grad_(True) for x in xs]
        ps = [torch.randn(H, d, generator=gg) * 0.1] + [torch.randn(H, generator=gg) for _ in range(4)]
        ps = [p.to(dev).requires_grad_(True) for p in ps]
        zs = [torch.randn(B, T, H, generator=gg).to(dev).requires_grad_(True) for _ in range(2)]
        return xs + [torch.arange(1, T + 1, dtype=torch.float32, device=dev)] + ps + zs

    del g
    a = leaves()
    loss_e = _step(*a)
    grads_e = torch.autograd.grad(loss_e, [t for t in a if t.requires_grad])
    torch._dynamo.reset()
    cstep = torch.compile(_step, backend="aot_eager", fullgraph=True)
    b = leaves()
    loss_c = cstep(*b)
    grads_c = torch.autograd.grad(loss_c, [t for t in b if t.requires_grad])
    assert torch.allclose(loss_c, loss_e, rtol=1e-6, atol=0), (loss_c.item(), loss_e.item())
    for i, (x, y) in enumerate(zip(grads_c, grads_e)):
        assert torch.allclose(x.float(), y.float(), rtol=1e-5, atol=1e-6 * y.float().abs().max().item()), i

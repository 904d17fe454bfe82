"""GPU parity of the gated-delta training backward (the FLA autograd of
chunk_gated_delta_rule that TitansMemory trains through, model/blocks.py:44-84) against
fp64 torch autograd of the sequential definition (scripts/titans_proto.py:53-76; the
oracle's autograd is pinned by gradcheck in test_oracle_gated_delta).  Every gradient
(q, k, v, g, beta, initial state) within 1e-4 of max|grad| per tensor for fp32 inputs,
2e-2 for bf16; lengths across the 64-token checkpoints and 8-token sub-blocks, both
head dims (dk = dv, the forward kernel's shapes; 4 and 8 column blocks), grouped KV heads, l2norm on and off,
a final-state cotangent or none, and an unused output."""

import pytest
import torch

from oracle import gated_delta as OG
from tests.helpers import rel_err

pytestmark = pytest.mark.gpu


def _oracle(q, k, v, g, beta, S0, scale, l2):
    """chunk_gated_delta_rule's contract in fp64 through the sequential definition."""
    H = q.shape[2]
    if k.shape[2] != H:
        k, v = k.repeat_interleave(H // k.shape[2], 2), v.repeat_interleave(H // k.shape[2], 2)
    qf, kf, vf = (x.double().transpose(1, 2) for x in (q, k, v))
    if l2:
        qf, kf = OG.l2_normalize(qf), OG.l2_normalize(kf)
    R, S = OG.gated_delta_sequential(qf * scale, kf, vf, torch.exp(g.double()).transpose(1, 2),
                                     beta.double().transpose(1, 2),
                                     None if S0 is None else S0.double().transpose(-1, -2))
    return R.transpose(1, 2), S.transpose(-1, -2)


@pytest.mark.parametrize("B,T,H,Hkv,dk,dv,l2,s0,dfinal,dtype", [
    (2, 1, 2, 2, 64, 64, True, False, False, torch.float32),
    (1, 65, 2, 2, 128, 128, True, True, True, torch.float32),
    (2, 130, 3, 3, 64, 64, False, True, False, torch.float32),
    (1, 200, 4, 2, 128, 128, True, False, True, torch.float32),
    (1, 77, 2, 1, 64, 64, True, True, True, torch.float32),
    (2, 96, 2, 2, 128, 128, True, True, True, torch.bfloat16),
])
def test_gated_delta_backward_vs_fp64_autograd(dev, B, T, H, Hkv, dk, dv, l2, s0, dfinal, dtype):
    from atma_amd.kernel import chunk_gated_delta_rule
    gen = torch.Generator().manual_seed(T * 7 + dk + dv)
    q = torch.randn(B, T, H, dk, generator=gen).to(dtype)
    k = torch.randn(B, T, Hkv, dk, generator=gen).to(dtype)
    v = torch.randn(B, T, Hkv, dv, generator=gen).to(dtype)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen) + 2.0)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    S0 = torch.randn(B, H, dk, dv, generator=gen) * 0.3 if s0 else None
    scale = 1.0 if l2 else dk ** -0.5
    if not l2:   # unnormalised keys: keep the recurrence contractive
        k = (k.float() / k.float().norm(dim=-1, keepdim=True)).to(dtype)
    Wo = torch.randn(B, T, H, dv, generator=gen)
    Ws = torch.randn(B, H, dk, dv, generator=gen)

    leaves = [x.clone().double().requires_grad_(True) for x in (q, k, v, g, beta)]
    S0r = S0.clone().double().requires_grad_(True) if s0 else None
    o, S = _oracle(*leaves, S0r, scale, l2)
    loss = (o * Wo.double()).sum() + ((S * Ws.double()).sum() if dfinal else 0.0)
    ref = torch.autograd.grad(loss, leaves + ([S0r] if s0 else []))

    dl = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, beta)]
    S0d = S0.to(dev).requires_grad_(True) if s0 else None
    od, Sd = chunk_gated_delta_rule(*dl, scale=scale, initial_state=S0d, output_final_state=True,
                                    use_qk_l2norm_in_kernel=l2)
    assert od.dtype == dtype
    lossd = (od.float() * Wo.to(dev)).sum() + ((Sd * Ws.to(dev)).sum() if dfinal else 0.0)
    got = torch.autograd.grad(lossd, dl + ([S0d] if s0 else []))
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    names = ["dq", "dk", "dv", "dg", "dbeta", "dS0"]
    for name, a, b in zip(names, got, ref):
        assert a.shape == b.shape, name
        err = rel_err(a.float(), b)
        assert err <= tol, (name, err)


def test_unused_output_and_determinism(dev):
    from atma_amd.kernel import chunk_gated_delta_rule
    gen = torch.Generator().manual_seed(5)
    B, T, H, d = 1, 70, 2, 64
    q, k, v = (torch.randn(B, T, H, d, generator=gen).to(dev).requires_grad_(True) for _ in range(3))
    g = torch.full((B, T, H), -0.05, device=dev, requires_grad=True)
    beta = torch.full((B, T, H), 0.5, device=dev, requires_grad=True)
    runs = []
    for _ in range(2):
        _, S = chunk_gated_delta_rule(q, k, v, g, beta, scale=1.0, output_final_state=True,
                                      use_qk_l2norm_in_kernel=True)
        runs.append(torch.autograd.grad(S.square().sum(), (q, k, v, g, beta)))
    assert runs[0][0].abs().max() == 0            # o unused: no gradient reaches q
    for a, b in zip(*runs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,T,H,Hkv,d,dtype,tol", [
    (2, 130, 4, 2, 64, torch.float32, 1e-4),
    (1, 2048, 8, 2, 128, torch.bfloat16, 2e-2),    # configs[1] heads at training shape
])
def test_raw_logit_gates_backward_vs_fp64(dev, B, T, H, Hkv, d, dtype, tol):
    """TitansMemory's call: raw gate logits with gate_bias=(3.9, 0.0), differentiated
    through logsigmoid(z + 3.9) / sigmoid(z) and the recurrence, against fp64 autograd of
    the same activations through the oracle (the sequential definition for the short
    case; the chunked form, pinned against it, for T = 2,048)."""
    from atma_amd.kernel import chunk_gated_delta_rule
    gen = torch.Generator().manual_seed(T + d)
    q = torch.randn(B, T, H, d, generator=gen).to(dtype)
    k = torch.randn(B, T, Hkv, d, generator=gen).to(dtype)
    v = torch.randn(B, T, Hkv, d, generator=gen).to(dtype)
    zg, zb = torch.randn(B, T, H, generator=gen), torch.randn(B, T, H, generator=gen)
    Wo = torch.randn(B, T, H, d, generator=gen)

    leaves = [x.clone().double().requires_grad_(True) for x in (q, k, v, zg, zb)]
    q64, k64, v64, zg64, zb64 = leaves
    rep = H // Hkv
    kx, vx = k64.repeat_interleave(rep, 2), v64.repeat_interleave(rep, 2)
    gl, bt = torch.nn.functional.logsigmoid(zg64 + 3.9), torch.sigmoid(zb64)
    if T <= 256:
        o_ref, _ = _oracle(q64, kx, vx, gl, bt, None, 1.0, True)
    else:
        o_ref, _ = OG.chunk_gated_delta_rule(q64, kx, vx, gl, bt, scale=1.0, use_qk_l2norm_in_kernel=True)
    ref = torch.autograd.grad((o_ref * Wo.double()).sum(), leaves)

    dl = [x.to(dev).requires_grad_(True) for x in (q, k, v, zg, zb)]
    od, _ = chunk_gated_delta_rule(*dl, scale=1.0, use_qk_l2norm_in_kernel=True, gate_bias=(3.9, 0.0))
    got = torch.autograd.grad((od.float() * Wo.to(dev)).sum(), dl)
    errs = {n: rel_err(a, b) for n, a, b in zip(["dq", "dk", "dv", "dzg", "dzb"], got, ref)}
    assert all(e <= tol for e in errs.values()), errs

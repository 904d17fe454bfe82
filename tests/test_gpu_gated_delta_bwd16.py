"""GPU parity of the chunked (WY) 16-bit training backward of the gated-delta recurrence
(the algorithm of the FLA autograd the reference trains through, model/blocks.py:44-84).

  * each of its three launches against its fp32 torch restatement (tests/helpers.py; the
    restatements composed are pinned against the oracle's chunked backward on the CPU):
    the prep's tiles (16-bit copies exact; T, T^T, Rq^T within 2e-2 of max|x|, the kernel
    forming K K^T and Q K^T from 16-bit rows as the restatement does here), the chain's
    states and U / dY on the prep's own tiles, and the local gradients on the chain's own
    outputs, each within 2e-2 of max|x| (the kernels round products' operands to 16 bits);
  * the whole 16-bit route of ``chunk_gated_delta_rule``'s autograd against fp64 autograd
    of the sequential definition (scripts/titans_proto.py:53-76, pinned by gradcheck in
    the oracle tests): every gradient within 2e-2 of max|grad| per tensor, over ragged
    lengths, both head dims, bf16 and fp16, grouped KV heads, an initial state and a
    final-state cotangent or none."""

import pytest
import torch

from helpers import (CHAIN_TILES, bwd16_chain_reference, bwd16_local_reference, bwd16_prep_reference,
                     rel_err)
from oracle import gated_delta as OG

pytestmark = pytest.mark.gpu


def _prepared(B, T, H, d, dtype, seed, dev, l2norm):
    g = torch.Generator().manual_seed(seed)
    q, k = torch.randn(B, T, H, d, generator=g), torch.randn(B, T, H, d, generator=g)
    if not l2norm:   # unit keys keep the recurrence contractive
        q, k = OG.l2_normalize(q), OG.l2_normalize(k)
    q, k = q.to(dtype), k.to(dtype)
    v, dO = torch.randn(B, T, H, d, generator=g).to(dtype), torch.randn(B, T, H, d, generator=g).to(dtype)
    gl = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=g) + 3.0)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    S0 = torch.randn(B, H, d, d, generator=g) * 0.3
    dST = torch.randn(B, H, d, d, generator=g)
    return [x.to(dev) for x in (q, k, v, gl, beta, dO, S0, dST)]


STAGE_CASES = [  # (B, T, H, d, dtype, states, l2norm)
    (1, 64, 1, 128, torch.bfloat16, True, True),
    (2, 300, 3, 64, torch.bfloat16, True, True),
    (1, 1000, 2, 128, torch.float16, False, True),
    (1, 77, 2, 64, torch.float16, True, False),
    (8, 2048, 8, 128, torch.bfloat16, False, True),   # configs[1] training shape
]


def _stages(B, T, H, d, dtype, states, l2norm, dev):
    from atma_amd._ops import gated_delta_bwd16_stages
    q, k, v, gl, beta, dO, S0, dST = _prepared(B, T, H, d, dtype, T + d, dev, l2norm)
    if not states:
        S0 = dST = None
    scale = 1.0 if l2norm else d ** -0.5
    print(f"bwd16 stages B={B} T={T} H={H} d={d} {dtype} l2norm={l2norm}", flush=True)
    st = gated_delta_bwd16_stages(q, k, v, gl, beta, S0, dO, dST, scale, l2norm)
    torch.cuda.synchronize()
    return (q, k, v, gl, beta, dO, S0, dST, scale), st


@pytest.mark.parametrize("B,T,H,d,dtype,states,l2norm", STAGE_CASES)
def test_prep_kernel_vs_restatement(dev, B, T, H, d, dtype, states, l2norm):
    (q, k, v, gl, beta, dO, _, _, scale), st = _stages(B, T, H, d, dtype, states, l2norm, dev)
    ref = bwd16_prep_reference(q, k, v, gl, beta, dO, dtype, scale, l2norm)
    for name in ("kr", "kt", "qr", "qt", "vt", "ot", "got"):
        assert torch.equal(st[name], ref[name]) or rel_err(st[name], ref[name]) <= 1e-2, name
    for name in ("tm", "tt", "rt"):
        assert rel_err(st[name], ref[name]) <= 2e-2, (name, rel_err(st[name], ref[name]))
    for r in range(9):   # per-token factors: decays, beta, row-norm factors
        assert rel_err(st["f"][:, :, r], ref["f"][:, :, r]) <= 1e-5, r


@pytest.mark.parametrize("B,T,H,d,dtype,states,l2norm", STAGE_CASES)
def test_chain_kernel_vs_restatement(dev, B, T, H, d, dtype, states, l2norm):
    (_, _, _, _, _, _, S0, dST, _), st = _stages(B, T, H, d, dtype, states, l2norm, dev)
    BH = B * H
    ref = bwd16_chain_reference(*(st[n] for n in CHAIN_TILES), None if S0 is None else S0.reshape(BH, d, d),
                                None if dST is None else dST.reshape(BH, d, d))
    for name, r in zip(["s_entry", "ds_end", "u", "dy", "ds0"], ref):
        assert torch.isfinite(st[name].float()).all(), name
        assert rel_err(st[name], r) <= 2e-2, (name, rel_err(st[name], r))


@pytest.mark.parametrize("B,T,H,d,dtype,states,l2norm", STAGE_CASES)
def test_local_kernel_vs_restatement(dev, B, T, H, d, dtype, states, l2norm):
    (q, k, v, gl, beta, dO, _, _, scale), st = _stages(B, T, H, d, dtype, states, l2norm, dev)
    p = bwd16_prep_reference(q, k, v, gl, beta, dO, dtype, scale, l2norm)
    ref = bwd16_local_reference(p, st["s_entry"], st["ds_end"], st["u"], st["dy"])
    for name, r in zip(["dq", "dk", "dv", "dg", "db"], ref):
        assert st[name].shape == r.shape, name
        assert torch.isfinite(st[name].float()).all(), name
        assert rel_err(st[name], r) <= 2e-2, (name, rel_err(st[name], r))


def _oracle(q, k, v, g, beta, S0, scale):
    H = q.shape[2]
    if k.shape[2] != H:
        k, v = k.repeat_interleave(H // k.shape[2], 2), v.repeat_interleave(H // k.shape[2], 2)
    qf, kf, vf = (OG.l2_normalize(x.double().transpose(1, 2)) if i < 2 else x.double().transpose(1, 2)
                  for i, x in enumerate((q, k, v)))
    R, S = OG.gated_delta_sequential(qf * scale, kf, vf, torch.exp(g.double()).transpose(1, 2),
                                     beta.double().transpose(1, 2),
                                     None if S0 is None else S0.double().transpose(-1, -2))
    return R.transpose(1, 2), S.transpose(-1, -2)


@pytest.mark.parametrize("B,T,H,Hkv,d,dtype,s0,dfinal", [
    (1, 1, 2, 2, 64, torch.bfloat16, True, True),
    (1, 63, 2, 1, 128, torch.bfloat16, False, True),
    (2, 129, 2, 2, 64, torch.float16, True, False),
    (1, 200, 4, 2, 128, torch.bfloat16, True, True),
    (2, 256, 2, 2, 128, torch.float16, False, False),
])
def test_bwd16_route_vs_fp64_autograd(dev, B, T, H, Hkv, d, dtype, s0, dfinal):
    from atma_amd.kernel import chunk_gated_delta_rule
    gen = torch.Generator().manual_seed(T * 3 + d)
    q = torch.randn(B, T, H, d, generator=gen).to(dtype)
    k = torch.randn(B, T, Hkv, d, generator=gen).to(dtype)
    v = torch.randn(B, T, Hkv, d, generator=gen).to(dtype)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen) + 2.0)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    S0 = torch.randn(B, H, d, d, generator=gen) * 0.3 if s0 else None
    Wo, Ws = torch.randn(B, T, H, d, generator=gen), torch.randn(B, H, d, d, generator=gen)

    leaves = [x.clone().double().requires_grad_(True) for x in (q, k, v, g, beta)]
    S0r = S0.clone().double().requires_grad_(True) if s0 else None
    o, S = _oracle(*leaves, S0r, 1.0)
    loss = (o * Wo.double()).sum() + ((S * Ws.double()).sum() if dfinal else 0.0)
    ref = torch.autograd.grad(loss, leaves + ([S0r] if s0 else []))

    print(f"route B={B} T={T} H={H}/{Hkv} d={d} {dtype}", flush=True)
    dl = [x.to(dev).requires_grad_(True) for x in (q, k, v, g, beta)]
    S0d = S0.to(dev).requires_grad_(True) if s0 else None
    od, Sd = chunk_gated_delta_rule(*dl, scale=1.0, initial_state=S0d, output_final_state=True,
                                    use_qk_l2norm_in_kernel=True)
    assert od.dtype == dtype
    lossd = (od.float() * Wo.to(dev)).sum() + ((Sd * Ws.to(dev)).sum() if dfinal else 0.0)
    got = torch.autograd.grad(lossd, dl + ([S0d] if s0 else []))
    for name, a, b in zip(["dq", "dk", "dv", "dg", "dbeta", "dS0"], got, ref):
        assert a.shape == b.shape, name
        assert torch.isfinite(a.float()).all(), name
        assert rel_err(a.float(), b) <= 2e-2, (name, rel_err(a.float(), b))

"""Pins for the CPU gated-delta oracle (oracle/gated_delta.py), fp64, no GPU.

  * closed forms of the sequential definition (scripts/titans_proto.py:53-66):
      - beta = 0: pure decay, r_t = (prod gamma) M0 q_t;
      - gamma = 1, beta = 1, orthonormal keys: exact associative recall;
      - gamma < 1, orthonormal keys: decay applies to OLD memories only (decay first,
        undecayed write, self-inclusive readout);
      - a repeated key with beta = 1 is fully overwritten even under decay (the
        prediction is taken on the decayed state);
  * chunked == sequential across chunk sizes incl. ragged tails (the bar of
    tests/verify_titans.py:26-34: < 1e-9 in fp64);
  * the decode step == the sequential definition with N = 1, in place, untouched slots
    bitwise unchanged, [K, V] layout;
  * the FLA contract: g = log gamma, L2-normalised q/k, scale, [K, V] initial/final
    state (checked with a NON-symmetric state so a transpose slip fails), state carry
    across a split.
"""

import pytest
import torch

from oracle import gated_delta as G


@pytest.fixture(autouse=True)
def _fp64_default():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _inputs(B, H, N, dk, dv, seed):
    g = torch.Generator().manual_seed(seed)
    q = G.l2_normalize(torch.randn(B, H, N, dk, generator=g))
    k = G.l2_normalize(torch.randn(B, H, N, dk, generator=g))
    v = torch.randn(B, H, N, dv, generator=g)
    gamma = torch.sigmoid(torch.randn(B, H, N, generator=g) + 2.0)
    beta = torch.sigmoid(torch.randn(B, H, N, generator=g))
    return q, k, v, gamma, beta


def test_beta_zero_is_pure_decay():
    B, H, N, d = 1, 2, 9, 5
    q, k, v, gamma, _ = _inputs(B, H, N, d, d, 1)
    S0 = torch.randn(B, H, d, d, generator=torch.Generator().manual_seed(2))
    R, S = G.gated_delta_sequential(q, k, v, gamma, torch.zeros(B, H, N), S0=S0)
    cum = torch.cumprod(gamma, dim=-1)
    ref = cum[..., None] * (S0[:, :, None] @ q[..., None])[..., 0]
    assert (R - ref).abs().max() < 1e-12
    assert (S - cum[..., -1, None, None] * S0).abs().max() < 1e-12


def test_orthonormal_keys_associative_recall_with_decay_order():
    d, N = 8, 6
    keys = torch.eye(d)[torch.tensor([3, 0, 5, 1, 7, 2])]          # distinct basis vectors
    g = torch.Generator().manual_seed(3)
    v = torch.randn(1, 1, N, d, generator=g)
    q = G.l2_normalize(torch.randn(1, 1, N, d, generator=g))
    k = keys[None, None]
    for gam in (1.0, 0.7):
        gamma = torch.full((1, 1, N), gam)
        R, _ = G.gated_delta_sequential(q, k, v, gamma, torch.ones(1, 1, N))
        for t in range(N):
            ref = sum((gam ** (t - s)) * (keys[s] @ q[0, 0, t]) * v[0, 0, s] for s in range(t + 1))
            assert (R[0, 0, t] - ref).abs().max() < 1e-12


def test_repeated_key_is_overwritten_on_decayed_state():
    d = 4
    k1 = torch.tensor([1.0, 0.0, 0.0, 0.0])
    k = torch.stack([k1, k1])[None, None]
    v = torch.tensor([[1.0, 2.0, 3.0, 4.0], [-1.0, 0.5, 0.0, 2.0]])[None, None]
    q = k.clone()
    R, S = G.gated_delta_sequential(q, k, v, torch.tensor([[[0.9, 0.6]]]), torch.ones(1, 1, 2))
    assert (R[0, 0, 1] - v[0, 0, 1]).abs().max() < 1e-12           # M_2 k1 = v_2 exactly
    assert (R[0, 0, 0] - v[0, 0, 0]).abs().max() < 1e-12


@pytest.mark.parametrize("chunk", [1, 8, 32, 64, 128, 257])
def test_chunked_equals_sequential(chunk):
    q, k, v, gamma, beta = _inputs(2, 3, 257, 16, 24, 11)
    S0 = torch.randn(2, 3, 24, 16, generator=torch.Generator().manual_seed(12)) * 0.3
    Rs, Ss = G.gated_delta_sequential(q, k, v, gamma, beta, S0=S0)
    Rc, Sc = G.gated_delta_chunked(q, k, v, gamma, beta, chunk=chunk, S0=S0)
    assert (Rs - Rc).abs().max() < 1e-9 and (Ss - Sc).abs().max() < 1e-9


def test_decode_step_equals_sequential_and_is_in_place():
    B, H, d, slots_total = 3, 2, 6, 7
    g = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn(B, H, d, generator=g) for _ in range(3))
    gamma = torch.rand(B, H, generator=g)
    beta = torch.rand(B, H, generator=g)
    table = torch.randn(slots_total, H, d, d, generator=g)
    before = table.clone()
    slots = torch.tensor([4, 0, 5])
    r = G.gated_delta_decode_step(q, k, v, gamma, beta, table, slots)
    S0 = before[slots].transpose(-1, -2)                            # [K,V] -> (dv, dk)
    Rs, Ss = G.gated_delta_sequential(G.l2_normalize(q)[:, :, None], G.l2_normalize(k)[:, :, None],
                                      v[:, :, None], gamma[..., None], beta[..., None], S0=S0)
    assert (r - Rs[:, :, 0]).abs().max() < 1e-12
    assert (table[slots] - Ss.transpose(-1, -2)).abs().max() < 1e-12
    untouched = [i for i in range(slots_total) if i not in slots.tolist()]
    assert torch.equal(table[untouched], before[untouched])


def test_fla_contract_layout_and_carry():
    B, T, H, d = 2, 150, 2, 8
    g = torch.Generator().manual_seed(31)
    q = torch.randn(B, T, H, d, generator=g)
    k = torch.randn(B, T, H, d, generator=g)
    v = torch.randn(B, T, H, d, generator=g)
    logit = torch.randn(B, T, H, generator=g)
    glog = torch.nn.functional.logsigmoid(logit + 3.9)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    S0 = torch.randn(B, H, d, d, generator=g)                       # non-symmetric [K, V]
    o, S = G.chunk_gated_delta_rule(q, k, v, glog, beta, scale=0.7, initial_state=S0,
                                    output_final_state=True, use_qk_l2norm_in_kernel=True)
    qt = 0.7 * G.l2_normalize(q).transpose(1, 2)
    kt = G.l2_normalize(k).transpose(1, 2)
    R, M = G.gated_delta_sequential(qt, kt, v.transpose(1, 2), torch.exp(glog).transpose(1, 2),
                                    beta.transpose(1, 2), S0=S0.transpose(-1, -2))
    assert (o - R.transpose(1, 2)).abs().max() < 1e-9
    assert (S - M.transpose(-1, -2)).abs().max() < 1e-9
    # carry across a split reproduces the whole
    o1, S1 = G.chunk_gated_delta_rule(q[:, :70], k[:, :70], v[:, :70], glog[:, :70], beta[:, :70],
                                      scale=0.7, initial_state=S0, output_final_state=True,
                                      use_qk_l2norm_in_kernel=True)
    o2, S2 = G.chunk_gated_delta_rule(q[:, 70:], k[:, 70:], v[:, 70:], glog[:, 70:], beta[:, 70:],
                                      scale=0.7, initial_state=S1, output_final_state=True,
                                      use_qk_l2norm_in_kernel=True)
    assert (torch.cat([o1, o2], 1) - o).abs().max() < 1e-9 and (S2 - S).abs().max() < 1e-9
    # transposed initial state gives a different answer (layout is observable)
    o_t, _ = G.chunk_gated_delta_rule(q, k, v, glog, beta, scale=0.7, initial_state=S0.transpose(-1, -2),
                                      use_qk_l2norm_in_kernel=True)
    assert (o_t - o).abs().max() > 1e-3


def test_flops_formula():
    assert G.prefill_flops(8, 2048, 8, 128) == pytest.approx(1.718e10, rel=1e-3)
    from oracle.polar import prefill_flops
    assert prefill_flops(8, 8, 2048, 128) == pytest.approx(6.875e10, rel=1e-3)
    assert prefill_flops(1, 8, 65536, 128) == pytest.approx(8.796e12, rel=1e-3)


def test_sequential_autograd_is_pinned_by_gradcheck():
    """The backward's oracle is torch autograd through ``gated_delta_sequential``; central
    differences (fp64) pin it for every input, the initial state included."""
    g = torch.Generator().manual_seed(11)
    B, H, N, dk, dv = 1, 2, 5, 4, 3
    q = torch.randn(B, H, N, dk, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.nn.functional.normalize(torch.randn(B, H, N, dk, generator=g, dtype=torch.float64), dim=-1)
    k.requires_grad_(True)
    v = torch.randn(B, H, N, dv, generator=g, dtype=torch.float64, requires_grad=True)
    gam = torch.rand(B, H, N, generator=g, dtype=torch.float64).mul(0.5).add(0.45).requires_grad_(True)
    bet = torch.rand(B, H, N, generator=g, dtype=torch.float64).requires_grad_(True)
    S0 = torch.randn(B, H, dv, dk, generator=g, dtype=torch.float64, requires_grad=True)
    f = lambda *a: G.gated_delta_sequential(*a)  # noqa: E731
    assert torch.autograd.gradcheck(f, (q, k, v, gam, bet, S0))


@pytest.mark.parametrize("T,chunk,dk,dv", [(1, 4, 4, 3), (7, 4, 5, 4), (33, 8, 8, 6), (130, 64, 16, 16)])
def test_chunked_backward_equals_sequential_autograd(T, chunk, dk, dv):
    """The chunked backward restatement (the algorithm the HIP training backward follows)
    equals fp64 autograd through ``gated_delta_sequential`` (itself pinned by gradcheck
    above) for every input: q, k, v, the log decay, beta and the initial state, partial
    last chunks included."""
    g = torch.Generator().manual_seed(T + chunk)
    q = torch.randn(T, dk, generator=g, dtype=torch.float64)
    k = torch.nn.functional.normalize(torch.randn(T, dk, generator=g, dtype=torch.float64), dim=-1)
    v = torch.randn(T, dv, generator=g, dtype=torch.float64)
    gl = torch.nn.functional.logsigmoid(torch.randn(T, generator=g, dtype=torch.float64) + 2.0)
    beta = torch.sigmoid(torch.randn(T, generator=g, dtype=torch.float64))
    S0 = torch.randn(dk, dv, generator=g, dtype=torch.float64) * 0.3
    dO = torch.randn(T, dv, generator=g, dtype=torch.float64)
    dST = torch.randn(dk, dv, generator=g, dtype=torch.float64)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v, gl, beta, S0)]
    # the oracle's sequential form takes (B, H, N, d) and M = S^T
    R, M = G.gated_delta_sequential(leaves[0][None, None], leaves[1][None, None], leaves[2][None, None],
                                    torch.exp(leaves[3])[None, None], leaves[4][None, None],
                                    leaves[5].T[None, None])
    loss = (R[0, 0] * dO).sum() + (M[0, 0].T * dST).sum()
    ref = torch.autograd.grad(loss, leaves)
    got = G.gated_delta_chunked_backward(q, k, v, gl, beta, S0, dO, dST, chunk=chunk)
    for name, a, b in zip(("dq", "dk", "dv", "dgl", "dbeta", "dS0"), got, ref):
        assert torch.allclose(a, b, rtol=1e-9, atol=1e-10), name


@pytest.mark.parametrize("B,T,H,d,s0,dfinal,l2norm", [(1, 150, 2, 64, True, True, True),
                                                      (2, 64, 1, 128, False, True, True),
                                                      (1, 33, 3, 64, True, False, False)])
def test_bwd16_restatements_vs_oracle(B, T, H, d, s0, dfinal, l2norm):
    """The torch restatements of the three launches of the 16-bit chunked backward (prep:
    l2 norm and scale of the raw rows, chunk matrices and padding to 64-token chunks;
    chain: the state and state-gradient chains; local: the chunk-local gradients taken
    back through the l2 norm), composed in fp32, against the oracle's chunked backward in
    fp64 with fp64 autograd of the l2 norm and scale, to 1e-4 of max|grad|.  The GPU tests
    hold each HIP launch to its restatement."""
    from helpers import (CHAIN_TILES, bwd16_chain_reference, bwd16_local_reference, bwd16_prep_reference,
                         rel_err)
    g = torch.Generator().manual_seed(T + d)
    f32 = dict(dtype=torch.float32)
    scale = 0.7
    q = torch.randn(B, T, H, d, generator=g, **f32)
    k = torch.randn(B, T, H, d, generator=g, **f32)
    if not l2norm:   # keep the recurrence contractive
        q, k = G.l2_normalize(q), G.l2_normalize(k)
    v, dO = torch.randn(B, T, H, d, generator=g, **f32), torch.randn(B, T, H, d, generator=g, **f32)
    gl = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=g, **f32) + 2.0)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g, **f32))
    S0 = torch.randn(B, H, d, d, generator=g, **f32) * 0.3 if s0 else None
    dST = torch.randn(B, H, d, d, generator=g, **f32) if dfinal else None
    prep = bwd16_prep_reference(q, k, v, gl, beta, dO, torch.float32, scale, l2norm)
    st = lambda x: None if x is None else x.reshape(B * H, d, d)  # noqa: E731
    s_entry, ds_end, u, dy, ds0 = bwd16_chain_reference(*(prep[n] for n in CHAIN_TILES), st(S0), st(dST))
    got = bwd16_local_reference(prep, s_entry, ds_end, u, dy) + (ds0.reshape(B, H, d, d),)
    ref = [torch.zeros(B, T, H, d) for _ in range(3)] + [torch.zeros(B, T, H) for _ in range(2)] + \
          [torch.zeros(B, H, d, d)]
    for b in range(B):
        for h in range(H):
            z = torch.zeros(d, d)
            qr_ = q[b, :, h].double().requires_grad_(True)
            kr_ = k[b, :, h].double().requires_grad_(True)
            qn, kn = (scale * G.l2_normalize(qr_), G.l2_normalize(kr_)) if l2norm else (scale * qr_, kr_)
            out = G.gated_delta_chunked_backward(
                qn.detach(), kn.detach(), v[b, :, h].double(), gl[b, :, h].double(), beta[b, :, h].double(),
                z if S0 is None else S0[b, h].double(), dO[b, :, h].double(), z if dST is None else dST[b, h].double())
            dq_raw, dk_raw = torch.autograd.grad((qn, kn), (qr_, kr_), (out[0], out[1]))
            for r, o in zip(ref[:5], (dq_raw, dk_raw) + tuple(out[2:5])):
                r[b, :, h] = o
            ref[5][b, h] = out[5]
    for name, a, r in zip(["dq", "dk", "dv", "dg", "dbeta", "dS0"], got, ref):
        assert a.shape == r.shape, name
        assert rel_err(a, r) <= 1e-4, (name, rel_err(a, r))

"""The decode-step fusions (``kernel/decode_fusions.py``; no reference counterpart, each
the one-launch form of a chain of the reference's decode ops) against the chains they
replace, run in torch on the same 16-bit inputs:

* ``linear_tokens_multi`` / ``linear_tokens_chunks`` against fp32 ``F.linear`` (fp32
  accumulation: parts within 2e-5 relative of the fp64 product, 16-bit outputs within
  1e-2, the ``linear_tokens`` bar); ``linear_tokens_gated`` bit for bit against
  ``linear_tokens`` then ``squared_relu_gate`` (the same products and roundings);
* ``residual_rms_norm``: the new stream equal to the eager bf16 add bit for bit (one
  rounding of the same fp32 sum), a branch of partial sums + biases + low-rank term
  within one bf16 ulp of its fp64 sum (one rounding), the normed row within one ulp of
  ``F.rms_norm`` (the reciprocal square root's last bit);
* ``lfm2_conv_step``: equal bit for bit to ``b * x`` -> ``causal_conv1d_decode_step`` ->
  ``c * (.)``, state tables included; ``linear_tokens_conv`` bit for bit to
  ``linear_tokens`` then ``lfm2_conv_step`` (state tables included, a row without a state
  slot NaN and its table untouched);
* ``global_decode_prep`` / ``global_decode_gate``: the head RMSNorm + Canon conv + gates
  chain and the gated projection inputs within 1e-2 relative (a normed or sigmoid value
  one bf16 ulp apart from torch's carries through a product), the un-normed v conv, the
  gates and the v table bit for bit, the normed tables within one ulp.
"""

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import rel_err

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _g(dev, seed):
    return torch.Generator(device=dev).manual_seed(seed)


def _ulps(a, b):
    """max |a - b| in units of b's bf16 spacing (2^(e-7) for |b| in [2^e, 2^(e+1)))."""
    a, b = a.double(), b.double()
    spacing = torch.exp2(torch.floor(torch.log2(b.abs().clamp_min(1e-30))) - 7)
    return ((a - b).abs() / spacing).max().item()


# --------------------------------------------------------------------------- projections
@pytest.mark.parametrize("K", [256, 512, 1024, 2048])
@pytest.mark.parametrize("M", [1, 7, 32])
def test_linear_tokens_multi_segments_vs_fp32(dev, M, K):
    from atma_amd.kernel.decode_fusions import linear_tokens_multi
    g = _g(dev, M * 13 + K)
    ns = [2048, 256, 256, 1024, 8, 4, 36]
    x = torch.randn(M, K, device=dev, generator=g).to(BF)
    ws = [(torch.randn(n, K, device=dev, generator=g) * 0.03).to(BF) for n in ns]
    bs = [(torch.randn(n, device=dev, generator=g) * 0.1).to(BF) if i != 2 else None for i, n in enumerate(ns)]
    y = linear_tokens_multi(x, ws, bs)
    assert y.shape == (M, sum(ns))
    off = 0
    for w, b, n in zip(ws, bs, ns):
        ref = F.linear(x.float(), w.float(), None if b is None else b.float())
        assert rel_err(y[:, off:off + n], ref) <= 1e-2, (n, rel_err(y[:, off:off + n], ref))
        off += n
    assert torch.equal(y, linear_tokens_multi(x, ws, bs))


def test_linear_tokens_multi_wide_segments(dev):
    """Every segment a multiple of 32 and 4096+ outputs in all: 32 features per workgroup."""
    from atma_amd.kernel.decode_fusions import linear_tokens_multi
    g = _g(dev, 5)
    x = torch.randn(32, 1024, device=dev, generator=g).half()
    ws = [(torch.randn(n, 1024, device=dev, generator=g) * 0.03).half() for n in (4096, 1056)]
    y = linear_tokens_multi(x, ws, [None, None])
    assert rel_err(y[:, :4096], x.float() @ ws[0].float().t()) <= 1e-2
    assert rel_err(y[:, 4096:], x.float() @ ws[1].float().t()) <= 1e-2


@pytest.mark.parametrize("chunk_k,C", [(1024, 4), (256, 4), (512, 2), (1024, 1), (256, 8)])
@pytest.mark.parametrize("M", [3, 32])
def test_linear_tokens_chunks_vs_fp64(dev, M, chunk_k, C):
    from atma_amd.kernel.decode_fusions import linear_tokens_chunks
    g = _g(dev, M + chunk_k + C)
    N = 1024
    x = torch.randn(M, C * chunk_k + 64, device=dev, generator=g).to(BF)
    w = (torch.randn(N, C * chunk_k, device=dev, generator=g) * 0.03).to(BF)
    parts = linear_tokens_chunks(x, [w[:, c * chunk_k:(c + 1) * chunk_k] for c in range(C)], chunk_k)
    assert parts.shape == (C, M, N) and parts.dtype == torch.float32
    for c in range(C):
        sl = slice(c * chunk_k, (c + 1) * chunk_k)
        ref = x[:, sl].double() @ w[:, sl].double().t()
        assert rel_err(parts[c], ref) <= 2e-5


@pytest.mark.parametrize("K", [256, 1024, 2048])
@pytest.mark.parametrize("M", [1, 32])
def test_linear_tokens_gated_equals_projection_then_activation(dev, M, K):
    """The MLP's first projection with the activation in its epilogue equals
    ``linear_tokens`` (same products, same rounding) followed by ``squared_relu_gate``."""
    from atma_amd.kernel import linear_tokens, squared_relu_gate
    from atma_amd.kernel.decode_fusions import linear_tokens_gated
    g = _g(dev, 40 + M + K)
    H = 4096 if K == 1024 else 1024
    x = torch.randn(M, K, device=dev, generator=g).to(BF)
    w = (torch.randn(2 * H, K, device=dev, generator=g) * 0.03).to(BF)
    b = (torch.randn(2 * H, device=dev, generator=g) * 0.1).to(BF)
    h = linear_tokens_gated(x, w, b)
    y = F.linear(x.float(), w.float(), b.float())
    ref = squared_relu_gate(y[:, :H].to(BF), y[:, H:].to(BF))
    assert rel_err(h, ref) <= 1e-2
    yk = linear_tokens(x, w, b)
    assert torch.equal(h, squared_relu_gate(yk[:, :H], yk[:, H:]))     # bitwise, same products
    eager = yk[:, H:] * yk[:, :H].relu().square()
    assert torch.equal(squared_relu_gate(yk[:, :H], yk[:, H:]), eager)


def test_linear_tokens_chunks_rejects(dev):
    from atma_amd.kernel.decode_fusions import linear_tokens_chunks
    x = torch.randn(4, 2048, device=dev).to(BF)
    w = torch.randn(64, 2048, device=dev).to(BF)
    with pytest.raises(ValueError):
        linear_tokens_chunks(x, [w[:, :2048]], 2048)        # chunk wider than 1024
    with pytest.raises(ValueError):
        linear_tokens_chunks(x, [w[:, :1024]] * 3, 1024)     # x holds 2 chunks, not 3
    with pytest.raises(ValueError):
        linear_tokens_chunks(torch.randn(33, 1024, device=dev).to(BF), [w[:, :1024]], 1024)


# --------------------------------------------------------------------------- residual stream
@pytest.mark.parametrize("D", [256, 1024, 2048, 4096])
@pytest.mark.parametrize("M", [1, 5, 32, 300])
def test_residual_rms_norm_tensor_branch(dev, M, D):
    from atma_amd.kernel.decode_fusions import residual_rms_norm
    g = _g(dev, M * 3 + D)
    res = torch.randn(M, D, device=dev, generator=g).to(BF)
    br = torch.randn(M, D, device=dev, generator=g).to(BF)
    w = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(BF)
    out, s = residual_rms_norm(br, res, w, 1e-6)
    eager_s = res + br
    assert torch.equal(s, eager_s)
    ref = F.rms_norm(eager_s.float(), (D,), w.float(), 1e-6)
    assert _ulps(out, ref) <= 1.0
    out0, s0 = residual_rms_norm(br, None, w, 1e-6)         # the stream starts with the branch
    assert s0 is br and _ulps(out0, F.rms_norm(br.float(), (D,), w.float(), 1e-6)) <= 1.0


@pytest.mark.parametrize("with_res", [True, False])
@pytest.mark.parametrize("M", [1, 32])
def test_residual_rms_norm_partial_sums(dev, M, with_res):
    from atma_amd.kernel.decode_fusions import PartialSums, residual_rms_norm
    g = _g(dev, 77 + M)
    D, P, H = 1024, 2, 8
    parts = torch.randn(P, M, D, device=dev, generator=g)
    biases = [(torch.randn(D, device=dev, generator=g) * 0.1).to(BF) for _ in range(3)]
    mag = torch.rand(M, H, device=dev, generator=g).to(BF)
    mu_w = (torch.randn(D, H, device=dev, generator=g) * 0.3).to(BF)
    res = torch.randn(M, D, device=dev, generator=g).to(BF) if with_res else None
    w = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(BF)
    ps = PartialSums(parts, biases, mu_x=mag, mu_w=mu_w, dtype=BF)
    out, s = residual_rms_norm(ps, res, w, 1e-6)
    br64 = parts.double().sum(0) + sum(b.double() for b in biases) + mag.double() @ mu_w.double().t()
    if with_res:                                           # the eager add of the rounded branch
        assert _ulps(s, res + ps.materialize()) <= 1.0
    else:                                                  # the branch itself: one rounding
        assert _ulps(s, br64) <= 1.0
    assert _ulps(out, F.rms_norm(s.float(), (D,), w.float(), 1e-6)) <= 1.0


# --------------------------------------------------------------------------- mixers
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("K", [3, 4, 1])
def test_lfm2_conv_step_equals_eager_chain(dev, dtype, K):
    from atma_amd.kernel import causal_conv1d_decode_step
    from atma_amd.kernel.decode_fusions import lfm2_conv_step
    g = _g(dev, K)
    B, D, S = 9, 1024, 12
    bcx = torch.randn(B, 3 * D, device=dev, generator=g).to(dtype)
    w = (torch.randn(D, K, device=dev, generator=g) * 0.5).to(dtype)
    table = torch.randn(S, D, max(K - 1, 1), device=dev, generator=g).to(dtype)[:, :, :K - 1].contiguous()
    slots = torch.tensor([3, 0, 11, 5, 7, 1, 2, 4, 6], device=dev)
    t_fused, t_eager = table.clone(), table.clone()
    out = lfm2_conv_step(bcx, w, slots, t_fused)
    b, c, x = bcx.chunk(3, dim=-1)
    ref = c * causal_conv1d_decode_step(b * x, w, slots, t_eager)
    assert torch.equal(out, ref)
    assert torch.equal(t_fused, t_eager)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,Kt", [(32, 1024, 3), (7, 512, 4), (1, 2048, 3), (12, 256, 2)])
def test_linear_tokens_conv_equals_projection_then_conv_step(dev, dtype, M, K, Kt):
    from atma_amd.kernel import linear_tokens
    from atma_amd.kernel.decode_fusions import lfm2_conv_step, linear_tokens_conv
    g = _g(dev, M + K + Kt)
    H, S = 1024, 40
    x = torch.randn(M, K, device=dev, generator=g).to(dtype)
    w = (torch.randn(3 * H, K, device=dev, generator=g) * K ** -0.5).to(dtype)
    bias = (torch.randn(3 * H, device=dev, generator=g) * 0.1).to(dtype)
    taps = (torch.randn(H, Kt, device=dev, generator=g) * 0.5).to(dtype)
    table = torch.randn(S, H, Kt - 1, device=dev, generator=g).to(dtype)
    slots = torch.randperm(S - 1, device=dev, generator=g)[:M]
    if M > 1:
        slots[M // 2] = S                                  # no state row: NaN, table untouched
    t_fused, t_chain = table.clone(), table.clone()
    out = linear_tokens_conv(x, w, bias, taps, slots, t_fused)
    ref = lfm2_conv_step(linear_tokens(x, w, bias), taps, slots, t_chain)
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(out), nan)
    diff = (out.view(torch.int16) != ref.view(torch.int16)) & ~nan
    if diff.any():
        i, j = diff.nonzero()[0].tolist()
        raise AssertionError(f"{int(diff.sum())} outputs differ, first at {(i, j)}: {out[i, j].item()!r} against "
                             f"{ref[i, j].item()!r}")
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))     # NaN rows with the same bits
    assert torch.equal(t_fused, t_chain)
    if M > 1:
        assert nan[M // 2].all()
    assert torch.equal(t_fused[S - 1], table[S - 1])          # a row no token names


def test_linear_tokens_conv_rejects(dev):
    from atma_amd.kernel.decode_fusions import linear_tokens_conv
    x = torch.zeros(4, 1024, device=dev, dtype=BF)
    w = torch.zeros(3 * 1024, 1024, device=dev, dtype=BF)
    taps = torch.zeros(1024, 3, device=dev, dtype=BF)
    table = torch.zeros(4, 1024, 2, device=dev, dtype=BF)
    slots = torch.arange(4, device=dev)
    with pytest.raises(ValueError):
        linear_tokens_conv(torch.zeros(33, 1024, device=dev, dtype=BF), w, None, taps, torch.arange(33), table)
    with pytest.raises(ValueError):
        linear_tokens_conv(x, w[:3000], None, taps[:1000], slots, table)
    with pytest.raises(ValueError):
        linear_tokens_conv(x, w, None, taps, slots, table[:, :, :1])
    with pytest.raises(ValueError):                       # one tap: the two-launch chain serves it
        linear_tokens_conv(x, w, None, taps[:, :1].contiguous(), slots, table[:, :, :0])


def _prep_inputs(dev, B=6, H=8, Hkv=2, d=128, Kc=4, S=10, seed=0):
    g = _g(dev, seed)
    hd, kvd = H * d, Hkv * d
    W = 2 * hd + 2 * kvd + hd + 2 * H
    y = torch.randn(B, W, device=dev, generator=g).to(BF)
    taps = [(torch.randn(C, Kc, device=dev, generator=g) * 0.4).to(BF) for C in (hd, kvd, kvd)]
    tables = [torch.randn(S, C, Kc - 1, device=dev, generator=g).to(BF) for C in (hd, kvd, kvd)]
    slots = torch.randperm(S, device=dev, generator=g)[:B]
    return y, taps, tables, slots


@pytest.mark.parametrize("d,H,Hkv", [(128, 8, 2), (64, 4, 1)])
def test_global_decode_prep_vs_eager_chain(dev, d, H, Hkv):
    from atma_amd.kernel import causal_conv1d_decode_step, gated_delta_gates
    from atma_amd.kernel.decode_fusions import global_decode_prep
    y, taps, tables, slots = _prep_inputs(dev, H=H, Hkv=Hkv, d=d, seed=d + H)
    B = y.shape[0]
    hd, kvd = H * d, Hkv * d
    ck, cv = 2 * hd, 2 * hd + kvd
    cm = cv + kvd
    cg = cm + hd
    mine = [t.clone() for t in tables]
    q, k, v, gamma, beta = global_decode_prep(y, H, Hkv, d, (ck, cv, cg, cg + H), taps, mine, slots,
                                              torch.finfo(torch.float32).eps, gate_bias=(3.9, 0.0))
    eager = [t.clone() for t in tables]
    qg = y[:, :2 * hd].reshape(B, H, 2 * d)
    qn = F.rms_norm(qg[..., :d], (d,))
    kn = F.rms_norm(y[:, ck:cv].reshape(B, Hkv, d), (d,))
    rq = causal_conv1d_decode_step(qn.reshape(B, hd), taps[0], slots, eager[0], residual=True)
    rk = causal_conv1d_decode_step(kn.reshape(B, kvd), taps[1], slots, eager[1], residual=True)
    rv = causal_conv1d_decode_step(y[:, cv:cm].contiguous(), taps[2], slots, eager[2], residual=True)
    ga, be = gated_delta_gates(y[:, cg:cg + H].float(), y[:, cg + H:cg + 2 * H].float(), 3.9, 0.0,
                               decay_as_prob=True)
    assert rel_err(q.reshape(B, hd), rq) <= 1e-2 and rel_err(k.reshape(B, kvd), rk) <= 1e-2
    assert torch.equal(v.reshape(B, kvd), rv)
    assert torch.equal(gamma, ga) and torch.equal(beta, be)
    # the tables hold the normed inputs: equal where the norm rounded alike
    assert torch.equal(mine[2], eager[2])
    assert _ulps(mine[0], eager[0]) <= 1.0 and _ulps(mine[1], eager[1]) <= 1.0


def test_global_decode_gate_vs_eager(dev):
    from atma_amd.kernel.decode_fusions import global_decode_gate
    g = _g(dev, 9)
    B, H, d = 7, 8, 128
    hd = H * d
    y = torch.randn(B, 4 * hd, device=dev, generator=g).to(BF)
    cm = 3 * hd
    c = torch.randn(B, H, d, device=dev, generator=g).to(BF)
    r = torch.randn(B, H, d, device=dev, generator=g) * 1e-2
    x2 = global_decode_gate(c, r, y, cm, torch.finfo(torch.float32).eps)
    gate = y[:, :2 * hd].reshape(B, H, 2 * d)[..., d:].reshape(B, hd)
    ref1 = c.reshape(B, hd) * torch.sigmoid(gate)
    ref2 = F.rms_norm(r, (d,)).reshape(B, hd).to(BF) * torch.sigmoid(y[:, cm:cm + hd])
    assert rel_err(x2[:, :hd], ref1) <= 1e-2
    assert rel_err(x2[:, hd:], ref2) <= 1e-2
    only = global_decode_gate(c, None, y, cm, 0.0)
    assert only.shape == (B, hd) and torch.equal(only, x2[:, :hd])


@pytest.mark.parametrize("H", [4, 16])
def test_residual_rms_norm_low_rank_widths(dev, H):
    from atma_amd.kernel.decode_fusions import PartialSums, residual_rms_norm
    g = _g(dev, 300 + H)
    M, D = 5, 256
    parts = torch.randn(4, M, D, device=dev, generator=g)
    mag = torch.rand(M, H, device=dev, generator=g).to(BF)
    mu_w = (torch.randn(D, H, device=dev, generator=g) * 0.3).to(BF)
    w = torch.ones(D, device=dev).to(BF)
    out, s = residual_rms_norm(PartialSums(parts, [], mu_x=mag, mu_w=mu_w, dtype=BF), None, w, 1e-6)
    br64 = parts.double().sum(0) + mag.double() @ mu_w.double().t()
    assert _ulps(s, br64) <= 1.0


@pytest.mark.parametrize("H", [4, 8, 16])
def test_residual_rms_norm_low_rank_many_rows(dev, H):
    """The prefill's form (a 16-bit base, two biases, the low-rank term, a residual) over many
    rows equals the same rows in a few-row call bit for bit (whose roundings the tests above
    pin), and the new stream is within 1e-2 of its fp64 sum."""
    from atma_amd.kernel.decode_fusions import PartialSums, residual_rms_norm
    g = _g(dev, 400 + H)
    M, D = 8195, 1024
    base = torch.randn(M, D, device=dev, generator=g).to(BF)
    b1, b2 = [(torch.randn(D, device=dev, generator=g) * 0.1).to(BF) for _ in range(2)]
    mag = torch.rand(M, H, device=dev, generator=g).to(BF)
    mu_w = (torch.randn(D, H, device=dev, generator=g) * 0.3).to(BF)
    res = torch.randn(M, D, device=dev, generator=g).to(BF)
    w = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(BF)
    out, s = residual_rms_norm(PartialSums(None, [b1, b2], mu_x=mag, mu_w=mu_w, dtype=BF, base=base), res, w, 1e-6)
    few = slice(M - 7, M)
    out7, s7 = residual_rms_norm(PartialSums(None, [b1, b2], mu_x=mag[few].contiguous(), mu_w=mu_w, dtype=BF,
                                             base=base[few].contiguous()), res[few].contiguous(), w, 1e-6)
    assert torch.equal(out[few], out7) and torch.equal(s[few], s7)
    s64 = base.double() + b1.double() + b2.double() + mag.double() @ mu_w.double().t() + res.double()
    assert rel_err(s, s64) <= 1e-2


@pytest.mark.parametrize("V", [50304, 1000, 77, 131080, 200000])
def test_softcap_argmax_equals_softcap_then_argmax(dev, V):
    from atma_amd.kernel import softcap_argmax, softcap_logits
    g = _g(dev, V)
    rows = 32
    x = (torch.randn(rows, V, device=dev, generator=g) * 20).to(BF)
    x[3, 10] = x[3, 500 % V] = 1e4                       # equal after the cap: the first index wins
    x[5] = -float("inf")
    x[6, V // 2] = float("nan")                           # NaN ranks above every number
    capped, ids = softcap_argmax(x)
    ref = softcap_logits(x)
    assert torch.equal(capped.view(torch.int16), ref.view(torch.int16))   # bitwise (NaN rows included)
    assert torch.equal(ids, ref.float().argmax(-1))
    assert ids[3].item() == min(10, 500 % V) and ids[5].item() == 0 and ids[6].item() == V // 2

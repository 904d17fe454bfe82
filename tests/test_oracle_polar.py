"""Pins for the CPU Polar oracle (oracle/polar.py), fp64, no GPU.

The reference ships no golden tensors for this path, so every oracle function is
pinned by mathematics that a plausible slip would violate:
  * temperature-1, no-sink case == normalize(scaled_dot_product_attention)
    (a library routine) -- pins scores, scale, causal mask, value mixing, the norm;
  * constant-count non-causal case with temp = tau == SDPA with scale tau/sqrt(d),
    and n_eff == 1/sum(softmax^2) -- pins the length temperature and the count channel;
  * q = 0 closed form -- pins the null logit formula, the sink mixing with v_null,
    n_eff = n and m_eff = n (1 - w_null);
  * n_keys = 0 rows drain to the sink, T = 1 gives n_eff = 1;
  * window == recomputation on the last W keys with count W; GQA == expanded heads;
  * streaming == materialised; paged gather == explicit index math.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from helpers import polar_params
from oracle import polar as P



@pytest.fixture(autouse=True)
def _fp64_default():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _qkv(B, Hq, Hkv, T, d, seed=0, Tk=None):
    g = torch.Generator().manual_seed(seed)
    Tk = T if Tk is None else Tk
    q = torch.randn(B, Hq, T, d, generator=g)
    k = torch.randn(B, Hkv, Tk, d, generator=g)
    v = torch.randn(B, Hkv, Tk, d, generator=g)
    return q, k, v


def _p64(H, d, seed=0, **kw):
    return polar_params(H, d, seed=seed, dtype=torch.float64, **kw)


def test_temp_null_closed_form():
    lg, nb, ns = torch.tensor([0.3, -1.0]), torch.tensor([2.0, -0.5]), torch.tensor([0.5, 1.5])
    n = torch.tensor([0.0, 1.0, 7.0, 1000.0])
    temp, null = P.polar_temp_null(n, lg, nb, ns)
    sp = lambda x: math.log1p(math.exp(x))  # noqa: E731
    for h in range(2):
        for i, ni in enumerate([0.0, 1.0, 7.0, 1000.0]):
            nc = max(ni, 1.0)
            assert temp[h, i].item() == pytest.approx(1 + sp(lg[h].item()) * math.log(nc), rel=1e-14)
            assert null[h, i].item() == pytest.approx(
                nb[h].item() + sp(ns[h].item()) * math.sqrt(math.log(nc + 1)), rel=1e-14)


def _no_sink(params, temp_gain_raw=-30.0):
    p = dict(params)
    p["null_base"] = torch.full_like(p["null_base"], -1e4)
    p["len_gain_raw"] = torch.full_like(p["len_gain_raw"], temp_gain_raw)
    return p


@pytest.mark.parametrize("form", ["dense", "online"])
def test_reduces_to_sdpa_when_temp_one_and_no_sink(form):
    B, H, T, d = 2, 3, 37, 16
    q, k, v = _qkv(B, H, H, T, d, seed=1)
    p = _no_sink(_p64(H, d, seed=2))
    n = torch.arange(1, T + 1, dtype=torch.float64)
    if form == "dense":
        c, mag = P.polar_dense(q, k, v, n, params=p)
    else:
        c, mag = P.polar_online(q, k, v, n, params=p, k_block=8)
    ref = F.normalize(F.scaled_dot_product_attention(q, k, v, is_causal=True), dim=-1, eps=1e-6)
    assert (c - ref).abs().max() < 1e-10
    # count channel: n_eff = participation ratio of the causal softmax
    w = torch.softmax((q @ k.transpose(-1, -2) / math.sqrt(d)).masked_fill(
        torch.ones(T, T, dtype=torch.bool).triu(1), float("-inf")), dim=-1)
    n_eff = 1.0 / w.square().sum(-1)
    beta = F.softplus(p["mag_beta_raw"]).view(1, H, 1)
    assert (mag - torch.tanh(beta * torch.log1p(n_eff))).abs().max() < 1e-10


def test_length_temperature_scales_scores():
    B, H, Tq, Tk, d = 1, 2, 5, 29, 8
    q, k, v = _qkv(B, H, H, Tq, d, seed=3, Tk=Tk)
    lg = torch.tensor([0.4, -0.7])
    p = _no_sink(_p64(H, d, seed=4))
    p["len_gain_raw"] = lg
    n = torch.full((Tq,), float(Tk))
    c, mag = P.polar_dense(q, k, v, n, params=p)
    c2, _ = P.polar_online(q, k, v, n, params=p, k_block=7)
    for h in range(H):
        tau = 1 + F.softplus(lg[h]).item() * math.log(Tk)
        ref = F.normalize(F.scaled_dot_product_attention(q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1],
                                                         scale=tau / math.sqrt(d)), dim=-1)
        assert (c[:, h:h + 1] - ref).abs().max() < 1e-10
        assert (c2[:, h:h + 1] - ref).abs().max() < 1e-10


@pytest.mark.parametrize("form", ["dense", "online"])
def test_zero_query_closed_form(form):
    B, H, T, d = 1, 2, 11, 8
    _, k, v = _qkv(B, H, H, T, d, seed=5)
    q = torch.zeros(B, H, T, d)
    p = _p64(H, d, seed=6)
    n = torch.arange(1, T + 1, dtype=torch.float64)
    if form == "dense":
        c, mag = P.polar_dense(q, k, v, n, params=p)
    else:
        c, mag = P.polar_online(q, k, v, n, params=p, k_block=4)
    sp = F.softplus
    for h in range(H):
        for i in range(T):
            ni = i + 1
            temp = 1 + sp(p["len_gain_raw"][h]) * math.log(ni)
            null = p["null_base"][h] + sp(p["null_slope_raw"][h]) * math.sqrt(math.log(ni + 1))
            e_n = torch.exp(temp * null)
            w_null = e_n / (ni + e_n)
            s = (1 - w_null) * v[0, h, :ni].mean(0) + w_null * p["v_null"][h]
            assert (c[0, h, i] - s / s.norm()).abs().max() < 1e-10
            m_eff = ni * (1 - w_null)
            ref_mag = torch.tanh(sp(p["mag_beta_raw"][h]) * torch.log1p(m_eff))
            assert abs(mag[0, h, i] - ref_mag) < 1e-10


def test_zero_keys_drain_to_sink_and_single_key():
    B, H, Tq, Tk, d = 1, 2, 3, 6, 8
    q, k, v = _qkv(B, H, H, Tq, d, seed=7, Tk=Tk)
    p = _p64(H, d, seed=8)
    n = torch.tensor([0.0, 1.0, 0.0])
    for c, mag in (P.polar_dense(q, k, v, n, params=p), P.polar_online(q, k, v, n, params=p, k_block=2)):
        for i in (0, 2):
            assert mag[0, :, i].abs().max() < 1e-12
            assert (c[0, :, i] - F.normalize(p["v_null"], dim=-1)).abs().max() < 1e-10
        # one key: n_eff = 1 -> m_eff = 1 - w_null
        temp, null = P.polar_temp_null(torch.tensor([1.0]), p["len_gain_raw"], p["null_base"],
                                       p["null_slope_raw"])
        a = (q[0, :, 1] * k[0, :, 0]).sum(-1) / math.sqrt(d) * temp[:, 0]
        w_null = torch.exp(temp[:, 0] * null[:, 0]) / (torch.exp(a) + torch.exp(temp[:, 0] * null[:, 0]))
        ref = torch.tanh(F.softplus(p["mag_beta_raw"]) * torch.log1p(1 - w_null))
        assert (mag[0, :, 1] - ref).abs().max() < 1e-10


def test_window_equals_recompute_on_band():
    B, H, T, d, W = 1, 2, 40, 8, 9
    q, k, v = _qkv(B, H, H, T, d, seed=9)
    p = _p64(H, d, seed=10)
    n = torch.arange(1, T + 1, dtype=torch.float64)
    cw, mw = P.polar_online(q, k, v, n, params=p, window=W, k_block=16)
    cd, md = P.polar_dense(q, k, v, n, params=p, window=W)
    assert (cw - cd).abs().max() < 1e-10 and (mw - md).abs().max() < 1e-10
    for i in (0, 5, 8, 9, 25, 39):
        lo = max(0, i + 1 - W)
        cb, mb = P.polar_dense(q[:, :, i:i + 1], k[:, :, lo:i + 1], v[:, :, lo:i + 1],
                               torch.tensor([float(i + 1 - lo)]), params=p)
        assert (cw[:, :, i:i + 1] - cb).abs().max() < 1e-10
        assert (mw[:, :, i:i + 1] - mb).abs().max() < 1e-10


def test_preserve_length_calibrates_on_the_raw_count():
    """Under a window, preserve_length keeps the band mask but feeds temp/null the raw
    count n_i instead of min(n_i, W) (kernel/polar_triton.py:1049-1053)."""
    B, H, T, d, W = 1, 2, 30, 8, 7
    q, k, v = _qkv(B, H, H, T, d, seed=21)
    p = _p64(H, d, seed=22)
    n = torch.arange(1, T + 1, dtype=torch.float64)
    cp, mp = P.polar_dense(q, k, v, n, params=p, window=W, preserve_length=True)
    cw, mw = P.polar_dense(q, k, v, n, params=p, window=W)
    co, mo = P.polar_online(q, k, v, n, params=p, window=W, preserve_length=True, k_block=8)
    assert (cp - co).abs().max() < 1e-12 and (mp - mo).abs().max() < 1e-12
    assert (cp[:, :, :W] - cw[:, :, :W]).abs().max() < 1e-12       # n <= W: identical
    assert (mp[:, :, W:] - mw[:, :, W:]).abs().min() > 0           # n > W: the count matters
    for i in (0, 6, 7, 19, 29):
        lo = max(0, i + 1 - W)
        sig = torch.full((B, H, 1, T), float("-inf"), dtype=torch.float64)
        sig[..., lo:i + 1] = q[:, :, i:i + 1] @ k[:, :, lo:i + 1].transpose(-1, -2) / math.sqrt(d)
        cr, mr = P.polar_reduce(sig, v, torch.tensor([float(i + 1)], dtype=torch.float64), **p)
        assert (cp[:, :, i:i + 1] - cr).abs().max() < 1e-12 and (mp[:, :, i:i + 1] - mr).abs().max() < 1e-12


@pytest.mark.parametrize("form", ["dense", "online"])
@pytest.mark.parametrize("window,preserve", [(None, False), (3, False), (3, True)])
def test_autograd_matches_finite_differences(form, window, preserve):
    """The backward tests differentiate the streaming oracle in fp64; its autograd graph
    (the masking, the running-max shifts, the sink fold, the clamps) and the materialised
    form's agree with central differences for every input and parameter."""
    B, Hq, Hkv, T, d = 1, 2, 1, 6, 4
    q, k, v = (t.clone().requires_grad_() for t in _qkv(B, Hq, Hkv, T, d, seed=23))
    p = {a: b.clone().requires_grad_() for a, b in _p64(Hq, d, seed=24).items()}
    n = torch.arange(1, T + 1, dtype=torch.float64)
    names = list(p)

    def f(q, k, v, *ps):
        kw = dict(params=dict(zip(names, ps)), window=window, preserve_length=preserve)
        if form == "online":
            return P.polar_online(q, k, v, n, k_block=4, **kw)
        return P.polar_dense(q, k, v, n, **kw)

    assert torch.autograd.gradcheck(f, (q, k, v, *p.values()), eps=1e-6, atol=1e-7, rtol=1e-5)


def test_gqa_equals_expanded_and_online_equals_dense():
    B, Hq, Hkv, T, d = 2, 8, 2, 23, 16
    q, k, v = _qkv(B, Hq, Hkv, T, d, seed=11)
    p = _p64(Hq, d, seed=12)
    n = torch.arange(1, T + 1, dtype=torch.float64)
    c1, m1 = P.polar_online(q, k, v, n, params=p, k_block=5)
    c2, m2 = P.polar_online(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), n, params=p,
                            k_block=5)
    c3, m3 = P.polar_dense(q, k, v, n, params=p)
    assert torch.equal(c1, c2) and torch.equal(m1, m2)
    assert (c1 - c3).abs().max() < 1e-10 and (m1 - m3).abs().max() < 1e-10


def test_arbitrary_counts_equal_prefix_slices():
    """Non-causal rows with count m see exactly keys [0, m)."""
    B, H, Tq, Tk, d = 1, 2, 6, 30, 8
    q, k, v = _qkv(B, H, H, Tq, d, seed=13, Tk=Tk)
    p = _p64(H, d, seed=14)
    n = torch.tensor([30.0, 1.0, 17.0, 4.0, 29.0, 12.0])
    c, m = P.polar_online(q, k, v, n, params=p, k_block=8)
    for i, ni in enumerate(n.long().tolist()):
        cs, ms = P.polar_dense(q[:, :, i:i + 1], k[:, :, :ni], v[:, :, :ni], n[i:i + 1], params=p)
        assert (c[:, :, i:i + 1] - cs).abs().max() < 1e-10 and (m[:, :, i:i + 1] - ms).abs().max() < 1e-10


def test_invariants_and_rows_checker():
    B, H, T, d = 1, 4, 300, 32
    q, k, v = _qkv(B, H, H, T, d, seed=15)
    p = _p64(H, d, seed=16)
    n = torch.arange(1, T + 1, dtype=torch.float64)
    c, m = P.polar_online(q * 3, k, v, n, params=p, k_block=64)
    assert c.norm(dim=-1).max() <= 1 + 1e-9
    assert m.min() >= 0 and m.max() < 1
    rows = torch.tensor([0, 1, 63, 64, 200, 299])
    cr, mr = P.polar_rows(q * 3, k, v, n, rows, params=p, k_block=50)
    assert (cr - c[:, :, rows]).abs().max() < 1e-10 and (mr - m[:, :, rows]).abs().max() < 1e-10


def test_gather_paged_kv_index_math():
    pages, page, hkv, d = 7, 4, 2, 3
    cache = torch.arange(pages * page * hkv * d, dtype=torch.float64).view(pages, page, hkv, d)
    bt = torch.tensor([[5, 2, 6], [0, 3, -1]], dtype=torch.int32)
    ctx = torch.tensor([10, 6], dtype=torch.int32)
    g = P.gather_paged_kv(cache, bt, ctx)
    for b in range(2):
        for pos in range(int(ctx[b])):
            assert torch.equal(g[b, pos], cache[bt[b, pos // page], pos % page])
    assert g[1, 6:].abs().max() == 0


def test_decode_equals_last_prefill_row():
    B, Hq, Hkv, d, page = 3, 4, 2, 8, 4
    ctx = [9, 1, 12]
    g = torch.Generator().manual_seed(17)
    pool = 12
    kc = torch.randn(pool, page, Hkv, d, generator=g)
    vc = torch.randn(pool, page, Hkv, d, generator=g)
    perm = torch.randperm(pool, generator=g)
    bt = torch.full((B, 3), -1, dtype=torch.int32)
    used = 0
    for b, n in enumerate(ctx):
        npg = (n + page - 1) // page
        bt[b, :npg] = perm[used:used + npg].int()
        used += npg
    q = torch.randn(B, Hq, d, generator=g)
    p = _p64(Hq, d, seed=18)
    c, m = P.polar_decode_paged(q, kc, vc, bt, torch.tensor(ctx, dtype=torch.int32), params=p)
    kg = P.gather_paged_kv(kc, bt, torch.tensor(ctx))
    vg = P.gather_paged_kv(vc, bt, torch.tensor(ctx))
    for b, n in enumerate(ctx):
        cc, mm = P.polar_dense(q[b][None, :, None], kg[b, :n].permute(1, 0, 2)[None],
                               vg[b, :n].permute(1, 0, 2)[None], torch.tensor([float(n)]), params=p)
        assert (c[b] - cc[0, :, 0]).abs().max() < 1e-10 and (m[b] - mm[0, :, 0]).abs().max() < 1e-10

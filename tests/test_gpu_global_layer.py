"""The global-layer module on the GPU (HIP kernels + eager glue) against the CPU
oracle of ``PolarAttention.forward`` / ``Block.forward``, and the engine routes
(dense prefill into the paged cache + decode steps) against the full-sequence forward."""

import pytest
import torch

from oracle import block as OB
from tests.helpers import max_abs, rel_err

pytestmark = pytest.mark.gpu

DIM, DK = 256, 64          # 4 query heads, 1 KV head (GQA 4:1, as the 1024 / 128 model)
H, HKV = DIM // DK, DIM // DK // 4


def _block(window=None, seed=0, overlap=True):
    from atma_amd.layers.global_attention import GlobalBlock
    torch.manual_seed(seed)
    blk = GlobalBlock(DIM, head_dim=DK, window=window, overlap=overlap)
    with torch.no_grad():   # every parameter N(0, 0.02), the reference's test convention
        for n, p in blk.named_parameters():
            if not n.startswith("norm"):
                p.normal_(0.0, 0.02)
            if n in ("attn.null_base", "attn.mag_beta_raw"):
                p.normal_(0.0, 1.0)
    return blk


def _attn_sd(blk):
    return {k[5:]: v.detach().cpu().clone() for k, v in blk.state_dict().items() if k.startswith("attn.")}


@pytest.mark.parametrize("window", [None, 48])
def test_mixer_fp32_vs_oracle(dev, window):
    blk = _block(window=window)
    x = torch.randn(2, 150, DIM, generator=torch.Generator().manual_seed(1))
    ref = OB.polar_attention(_attn_sd(blk), x, H=H, Hkv=HKV, dk=DK, window=window)
    out = blk.attn.to(dev)(x.to(dev))
    assert max_abs(out, ref) <= 1e-4, max_abs(out, ref)


@pytest.mark.parametrize("grad", [True, False])
def test_block_fp32_vs_oracle(dev, grad):
    """With grad off the MLP runs the fused squared_relu_gate kernel (InferenceMLP)."""
    blk = _block()
    x = torch.randn(1, 200, DIM, generator=torch.Generator().manual_seed(2))
    sd = {k: v.detach().cpu().clone() for k, v in blk.state_dict().items()}
    ref = OB.global_block(sd, x, H=H, Hkv=HKV, dk=DK)
    with torch.set_grad_enabled(grad):
        out = blk.to(dev)(x.to(dev))
    assert max_abs(out, ref) <= 1e-4, max_abs(out, ref)


def test_mixer_bf16_vs_fp32_oracle(dev):
    blk = _block()
    x = torch.randn(2, 130, DIM, generator=torch.Generator().manual_seed(3))
    ref = OB.polar_attention(_attn_sd(blk), x, H=H, Hkv=HKV, dk=DK)
    out = blk.attn.to(dev, torch.bfloat16)(x.to(dev, torch.bfloat16))
    assert rel_err(out.float(), ref) <= 2e-2, rel_err(out.float(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_side_stream_overlap_is_bitwise_neutral(dev, dtype):
    a = _block(overlap=True).attn.to(dev, dtype)
    b = _block(overlap=False).attn.to(dev, dtype)
    c = _block(overlap="auto").attn.to(dev, dtype)
    x = torch.randn(2, 96, DIM, device=dev).to(dtype)
    ref = b(x)
    for _ in range(2):
        assert torch.equal(a(x), ref) and torch.equal(c(x), ref)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_prefill_then_decode_equals_full_forward(dev, dtype, tol):
    """Dense prefill of T0 tokens (paged KV + conv tails + memory table written), then
    n decode steps through the paged cache, reproduce rows T0..T0+n-1 of the causal
    full-sequence forward (inference/models/atma.py:397-437,546-618)."""
    from atma_amd.layers.global_attention import GlobalLayerCache
    attn = _block().attn.to(dev, dtype)
    B, T0, n, page = 3, 70, 6, 16
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, T0 + n, DIM, generator=g).to(dev, dtype)
    full = attn(x)

    max_pages = (T0 + n + page - 1) // page
    num_pages = B * max_pages + 5
    cache = GlobalLayerCache.allocate(attn, num_pages, page, max_seqs=B + 2, device=dev, dtype=dtype)
    perm = torch.randperm(num_pages, generator=g)[:B * max_pages].view(B, max_pages).int()
    bt = perm.to(dev)
    slots = torch.tensor([2, 0, 4], device=dev)   # table rows, deliberately not 0..B-1

    def slot_of(b, pos):
        return int(perm[b, pos // page]) * page + pos % page

    smap = torch.tensor([slot_of(b, t) for b in range(B) for t in range(T0)], dtype=torch.int32, device=dev)
    pre = attn.prefill(x[:, :T0], cache, slots, smap)
    assert rel_err(pre.float(), full[:, :T0].float()) <= tol
    for i in range(n):
        pos = T0 + i
        smap1 = torch.tensor([slot_of(b, pos) for b in range(B)], dtype=torch.int32, device=dev)
        ctx = torch.full((B,), pos + 1, dtype=torch.int32, device=dev)
        y = attn.decode(x[:, pos], cache, slots, bt, ctx, smap1)
        err = max_abs(y, full[:, pos]) if dtype == torch.float32 else rel_err(y.float(), full[:, pos].float())
        assert err <= tol, (i, err)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_chunked_prefill_continuation_equals_full_forward(dev, dtype, tol):
    """Fresh prefill of T0 tokens, two continuation chunks (gathered paged prefix +
    chunk with is_causal=False and absolute n_keys, conv tails as left context, memory
    from the table state; inference/models/atma.py:509-544), then a decode step, reproduce
    the causal full-sequence forward row for row."""
    from atma_amd.layers.global_attention import GlobalLayerCache
    attn = _block().attn.to(dev, dtype)
    B, T0, T1, T2, page = 2, 37, 29, 64, 16
    T = T0 + T1 + T2 + 1
    g = torch.Generator().manual_seed(6)
    x = torch.randn(B, T, DIM, generator=g).to(dev, dtype)
    full = attn(x)
    max_pages = (T + page - 1) // page
    num_pages = B * max_pages + 3
    cache = GlobalLayerCache.allocate(attn, num_pages, page, max_seqs=B + 2, device=dev, dtype=dtype)
    perm = torch.randperm(num_pages, generator=g)[:B * max_pages].view(B, max_pages).int()
    bt = perm.to(dev)
    slots = torch.tensor([3, 1], device=dev)

    def smap(lo, hi):
        return torch.tensor([int(perm[b, t // page]) * page + t % page for b in range(B) for t in range(lo, hi)],
                            dtype=torch.int32, device=dev)

    def check(y, lo, hi):
        ref = full[:, lo:hi]
        err = max_abs(y, ref) if dtype == torch.float32 else rel_err(y.float(), ref.float())
        assert err <= tol, (lo, hi, err)

    check(attn.prefill(x[:, :T0], cache, slots, smap(0, T0)), 0, T0)
    check(attn.prefill_continue(x[:, T0:T0 + T1], cache, slots, smap(T0, T0 + T1), bt, [T0] * B), T0, T0 + T1)
    lo = T0 + T1
    check(attn.prefill_continue(x[:, lo:lo + T2], cache, slots, smap(lo, lo + T2), bt, [lo] * B), lo, lo + T2)
    pos = T - 1
    ctx = torch.full((B,), pos + 1, dtype=torch.int32, device=dev)
    check(attn.decode(x[:, pos], cache, slots, bt, ctx, smap(pos, pos + 1)).unsqueeze(1), pos, pos + 1)


@pytest.mark.parametrize("overlap", [True, False])
def test_block_fp32_gradients_vs_fp64_oracle(dev, overlap):
    """Training through the layer: every parameter's gradient (and the input's) from
    loss.backward() on the GPU block against fp64 torch autograd through
    ``oracle/block.global_block`` (the reference forward is differentiable,
    model/reference.py:172).  The Polar branch must reach v_null, null_base,
    null_slope_raw, len_gain_raw, mag_beta_raw and, through c and mag, the projections
    and Canon convs; per-tensor bar max|a-b| / max|b| <= 1e-3 (the fp32 bar of the
    reference's Polar backward test, kernel/test_polar_kernel.py:81-117)."""
    blk = _block(overlap=overlap)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, 200, DIM, generator=g)
    w = torch.randn(1, 200, DIM, generator=g)
    sd = {k: v.detach().double().clone().requires_grad_(True) for k, v in blk.state_dict().items()}
    x64 = x.double().requires_grad_(True)
    ref_out = OB.global_block(sd, x64, H=H, Hkv=HKV, dk=DK)
    names = [n for n, _ in blk.named_parameters()]
    ref = torch.autograd.grad((ref_out * w.double()).sum(), [x64] + [sd[n] for n in names])

    blk = blk.to(dev)
    xd = x.to(dev).requires_grad_(True)
    out = blk(xd)
    got = torch.autograd.grad((out * w.to(dev)).sum(), [xd] + [p for _, p in blk.named_parameters()])
    assert max_abs(out.detach(), ref_out.detach()) <= 1e-4
    bad = {}
    for name, a, b in zip(["x"] + names, got, ref):
        e = rel_err(a, b)
        if not e <= 1e-3:
            bad[name] = e
    assert not bad, bad


def _token_sum_scales(monkeypatch, sd, x, w):
    """Per-head sums over tokens of |per-token contribution| to three gradients that
    are token sums: the memory's write- and retention-gate biases (d/d logit summed over
    (b, t)) and len_gain_raw (softplus'(len_gain) * sum_t d temp_t * ln n_t).  Obtained
    by adding a zero tensor at each token to the logit / temperature in the fp64 oracle
    and reading its gradient.  These sums cancel heavily (e.g. |sum| about 2.8 against
    sum |.| about 300 for one head's write-gate bias at T=333), so 16-bit rounding of the
    per-token terms is judged against the latter."""
    import oracle.polar as OP
    taps = {}
    lin, tn = OB.linear, OP.polar_temp_null

    def tap(name, y):
        taps[name] = torch.zeros_like(y, requires_grad=True)
        return y + taps[name]

    def linear(xx, sdd, name):
        y = lin(xx, sdd, name)
        return tap(name, y) if name in ("mem.w_beta", "mem.w_gamma") else y

    def temp_null(n, lg, nb, ns):
        t, nu = tn(n, lg, nb, ns)
        e = torch.zeros_like(t, requires_grad=True)
        taps["temp"] = e
        return t + e * torch.log(n.clamp_min(1.0))[None, :], nu

    monkeypatch.setattr(OB, "linear", linear)
    monkeypatch.setattr(OP, "polar_temp_null", temp_null)
    out = OB.global_block(sd, x, H=H, Hkv=HKV, dk=DK)
    names = ("mem.w_beta", "mem.w_gamma", "temp")
    gb, gg, gt = torch.autograd.grad((out * w).sum(), [taps[n] for n in names])
    monkeypatch.undo()
    lg = sd["attn.len_gain_raw"].detach()
    return {"attn.mem.w_beta.bias": gb.abs().sum((0, 1)), "attn.mem.w_gamma.bias": gg.abs().sum((0, 1)),
            "attn.len_gain_raw": gt.abs().sum(1) * torch.sigmoid(lg)}


@pytest.mark.parametrize("T", [200, 333])
def test_block_bf16_gradients_vs_fp64_oracle(dev, monkeypatch, T):
    """The 16-bit training route through the layer: the block in bfloat16 (its Polar
    backward on the MFMA loops with bf16 key/value shares, the memory branch on the
    chunked 16-bit gated-delta backward) against fp64 autograd through
    ``oracle/block.global_block`` evaluated on the same bf16-rounded parameters and
    input.  Per-tensor bar max|a-b| / max|b| <= 5e-2 (the reference's 16-bit backward
    bar, kernel/test_polar_kernel.py:119-128); for the three gradients that are
    cancelling token sums, max|a-b| <= 5e-3 * max_h sum_t |contribution| instead when
    that is the looser."""
    blk = _block(seed=3).to(torch.bfloat16)
    g = torch.Generator().manual_seed(13)
    x = torch.randn(2, T, DIM, generator=g).to(torch.bfloat16)
    w = torch.randn(2, T, DIM, generator=g)
    sd = {k: v.detach().double().clone().requires_grad_(True) for k, v in blk.state_dict().items()}
    x64 = x.double().requires_grad_(True)
    ref_out = OB.global_block(sd, x64, H=H, Hkv=HKV, dk=DK)
    names = [n for n, _ in blk.named_parameters()]
    ref = torch.autograd.grad((ref_out * w.double()).sum(), [x64] + [sd[n] for n in names])
    scales = _token_sum_scales(monkeypatch, sd, x.double(), w.double())

    print(f"bf16 block backward T={T}", flush=True)
    blk = blk.to(dev)
    xd = x.to(dev).requires_grad_(True)
    out = blk(xd)
    assert out.dtype == torch.bfloat16
    got = torch.autograd.grad((out.float() * w.to(dev)).sum(), [xd] + [p for _, p in blk.named_parameters()])
    assert rel_err(out.detach().float(), ref_out.detach()) <= 2e-2
    bad = {}
    for name, a, b in zip(["x"] + names, got, ref):
        assert a.dtype == torch.bfloat16, name
        e = rel_err(a.float(), b)
        if e <= 5e-2:
            continue
        if name in scales and max_abs(a.float(), b) <= 5e-3 * scales[name].max().item():
            continue
        bad[name] = e
    assert not bad, bad


def _packed_maps(lengths, slots, dev):
    """The engine's tile map (one entry per 128-row query tile) and token map."""
    ts, tq, tl, st, en, sl, packed = [], [], [], [], [], [], 0
    for n, s in zip(lengths, slots):
        for q0 in range(0, n, 128):
            ts.append(packed)
            tq.append(q0)
            tl.append(n)
        st += [packed] * n
        en += [packed + n] * n
        sl += [s] * n
        packed += n
    t = lambda v: torch.tensor(v, dtype=torch.int32, device=dev)  # noqa: E731
    return (t(ts), t(tq), t(tl)), (t(st), t(en), t(sl))


def _fresh_cache(attn, dev, dtype, pages=40, page=16, seqs=6):
    from atma_amd.layers.global_attention import GlobalLayerCache
    return GlobalLayerCache.allocate(attn, pages, page, max_seqs=seqs, device=dev, dtype=dtype)


def _cache_state(cache):
    return [cache.k_cache, cache.v_cache, cache.conv_q, cache.conv_k, cache.conv_v, cache.mem_table]


def test_grouped_route_equals_dense_route(dev):
    """Equal-length prompts through the grouped route (packed Canon convs, one tile-mapped
    Polar launch, memory per sequence) and the dense route: the KV pages and conv tails come
    from identical launches and agree bit for bit; the outputs and memory states agree to
    the bf16 bar (the grouped route runs the memory's projections per sequence, GEMMs of
    another row count whose library kernels may round differently)."""
    attn = _block(seed=5).attn.to(dev, torch.bfloat16)
    B, T, page = 3, 150, 16
    x = torch.randn(B, T, DIM, generator=torch.Generator().manual_seed(7)).to(dev, torch.bfloat16)
    slots = torch.tensor([4, 1, 2], device=dev)
    smap = torch.arange(B * T, dtype=torch.int32, device=dev) + 37           # any distinct slots
    with torch.no_grad():
        dense_cache = _fresh_cache(attn, dev, torch.bfloat16)
        ref = attn.prefill(x, dense_cache, slots, smap)
        grouped_cache = _fresh_cache(attn, dev, torch.bfloat16)
        tiles, tokens = _packed_maps([T] * B, slots.tolist(), dev)
        out = attn.prefill_packed(x.reshape(B * T, DIM), grouped_cache, [T] * B, slots, smap, tiles, tokens)
    assert rel_err(out.view(B, T, DIM).float(), ref.float()) <= 2e-2
    g, d = _cache_state(grouped_cache), _cache_state(dense_cache)
    for a, b in zip(g[:5], d[:5]):
        assert torch.equal(a, b)
    assert rel_err(g[5], d[5]) <= 2e-2


def test_grouped_route_matches_per_sequence_route(dev):
    """Ragged fresh prompts: the grouped route against the per-sequence route (each prompt
    alone, ``prefill_continue`` with nothing cached), outputs and every state within the
    bf16 bar, the KV pages within one bf16 rounding (the two routes' Canon convs round
    once each, in different kernels) -- the reference's
    tests/test_dense_prefill.py:148-204 pattern."""
    attn = _block(seed=6).attn.to(dev, torch.bfloat16)
    lengths = [3, 5, 130, 77]
    slots = [2, 0, 5, 3]
    total = sum(lengths)
    x = torch.randn(total, DIM, generator=torch.Generator().manual_seed(8)).to(dev, torch.bfloat16)
    smap = (torch.randperm(40 * 16, generator=torch.Generator().manual_seed(9))[:total]).int().to(dev)
    slots_t = torch.tensor(slots, device=dev)
    with torch.no_grad():
        per_cache = _fresh_cache(attn, dev, torch.bfloat16)
        parts, start = [], 0
        for i, n in enumerate(lengths):
            parts.append(attn.prefill_continue(x[start:start + n][None], per_cache, slots_t[i:i + 1],
                                               smap[start:start + n], None, [0])[0])
            start += n
        ref = torch.cat(parts, 0)
        grp_cache = _fresh_cache(attn, dev, torch.bfloat16)
        tiles, tokens = _packed_maps(lengths, slots, dev)
        out = attn.prefill_packed(x, grp_cache, lengths, slots_t, smap, tiles, tokens)
    assert rel_err(out.float(), ref.float()) <= 2e-2
    for a, b in zip(_cache_state(grp_cache)[2:], _cache_state(per_cache)[2:]):
        assert rel_err(a.float(), b.float()) <= 2e-2
    torch.testing.assert_close(grp_cache.k_cache, per_cache.k_cache)    # bf16 default: one rounding
    torch.testing.assert_close(grp_cache.v_cache, per_cache.v_cache)

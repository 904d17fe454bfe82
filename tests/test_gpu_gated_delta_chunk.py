"""GPU parity of the chunked gated-delta prefill (FLA chunk_gated_delta_rule contract)
against the fp64 oracle: fp32 inputs max-abs <= 1e-4, bf16 inputs max|a-b|/max|b| <= 2e-2;
state carry across a split; ragged tails; [K, V] initial/final state."""

import pytest
import torch
import torch.nn.functional as F

from helpers import max_abs, rel_err
from oracle import gated_delta as OG

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, d, generator=g).to(dtype)
    k = torch.randn(B, T, H, d, generator=g).to(dtype)
    v = torch.randn(B, T, H, d, generator=g).to(dtype)
    glog = F.logsigmoid(torch.randn(B, T, H, generator=g) + 3.9)   # the layer's own bias
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    S0 = torch.randn(B, H, d, d, generator=g) * 0.1
    return q, k, v, glog, beta, S0


def _run(dev, *args, **kw):
    from atma_amd.kernel import chunk_gated_delta_rule
    mv = lambda a: a.to(dev) if torch.is_tensor(a) else a  # noqa: E731
    o, S = chunk_gated_delta_rule(*map(mv, args), **{n: mv(a) for n, a in kw.items()})
    torch.cuda.synchronize()
    return o.cpu(), (S.cpu() if S is not None else None)


@pytest.mark.parametrize("T", [1, 63, 64, 65, 200, 1000])
@pytest.mark.parametrize("d", [128, 64])
def test_fp32_vs_oracle(dev, T, d):
    q, k, v, glog, beta, S0 = _inputs(2, T, 3, d, torch.float32, seed=T + d)
    o, S = _run(dev, q, k, v, glog, beta, scale=1.0, initial_state=S0, output_final_state=True,
                use_qk_l2norm_in_kernel=True)
    o_ref, S_ref = OG.chunk_gated_delta_rule(q.double(), k.double(), v.double(), glog.double(),
                                             beta.double(), scale=1.0, initial_state=S0.double(),
                                             output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert max_abs(o, o_ref) <= 1e-4
    assert max_abs(S, S_ref) <= 1e-4


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_half_vs_fp32_oracle(dev, dtype):
    q, k, v, glog, beta, S0 = _inputs(2, 700, 8, 128, dtype, seed=5)
    o, S = _run(dev, q, k, v, glog, beta, scale=1.0, initial_state=None, output_final_state=True,
                use_qk_l2norm_in_kernel=True)
    assert o.dtype == dtype and S.dtype == torch.float32
    o_ref, S_ref = OG.chunk_gated_delta_rule(q.float(), k.float(), v.float(), glog, beta, scale=1.0,
                                             output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert rel_err(o, o_ref) <= 2e-2 and rel_err(S, S_ref) <= 2e-2


def test_state_carry_across_split(dev):
    q, k, v, glog, beta, S0 = _inputs(1, 333, 4, 128, torch.float32, seed=6)
    kw = dict(scale=1.0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    o, S = _run(dev, q, k, v, glog, beta, initial_state=S0, **kw)
    o1, S1 = _run(dev, q[:, :130], k[:, :130], v[:, :130], glog[:, :130], beta[:, :130],
                  initial_state=S0, **kw)
    o2, S2 = _run(dev, q[:, 130:], k[:, 130:], v[:, 130:], glog[:, 130:], beta[:, 130:],
                  initial_state=S1, **kw)
    assert max_abs(torch.cat([o1, o2], 1), o) <= 2e-5 and max_abs(S2, S) <= 2e-5


def test_no_l2norm_and_scale(dev):
    q, k, v, glog, beta, S0 = _inputs(1, 130, 2, 64, torch.float32, seed=7)
    k = F.normalize(k, dim=-1)                                     # unit keys (stable rule)
    o, _ = _run(dev, q, k, v, glog, beta, scale=0.25, initial_state=S0, use_qk_l2norm_in_kernel=False)
    o_ref, _ = OG.chunk_gated_delta_rule(q.double(), k.double(), v.double(), glog.double(),
                                         beta.double(), scale=0.25, initial_state=S0.double(),
                                         use_qk_l2norm_in_kernel=False)
    assert max_abs(o, o_ref) <= 1e-4


@pytest.mark.parametrize("T", [1, 63, 65, 200])
@pytest.mark.parametrize("d", [64, 128])
def test_half_ragged_with_state(dev, T, d):
    """16-bit path: ragged chunk tails, both head dims, a carried-in fp32 state."""
    q, k, v, glog, beta, S0 = _inputs(2, T, 3, d, torch.bfloat16, seed=11 + T + d)
    o, S = _run(dev, q, k, v, glog, beta, scale=1.0, initial_state=S0, output_final_state=True,
                use_qk_l2norm_in_kernel=True)
    o_ref, S_ref = OG.chunk_gated_delta_rule(q.float(), k.float(), v.float(), glog, beta, scale=1.0,
                                             initial_state=S0, output_final_state=True,
                                             use_qk_l2norm_in_kernel=True)
    assert rel_err(o, o_ref) <= 2e-2 and rel_err(S, S_ref) <= 2e-2


@pytest.mark.parametrize("d", [64, 128])
def test_half_no_l2norm_and_scale(dev, d):
    """16-bit path without in-kernel normalisation: the raw query rows carry `scale`
    alone and the raw key rows no norm."""
    q, k, v, glog, beta, S0 = _inputs(1, 190, 2, d, torch.float32, seed=12)
    k = F.normalize(k, dim=-1)
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    o, _ = _run(dev, q, k, v, glog, beta, scale=0.25, initial_state=S0, use_qk_l2norm_in_kernel=False)
    o_ref, _ = OG.chunk_gated_delta_rule(q.float(), k.float(), v.float(), glog, beta, scale=0.25,
                                         initial_state=S0, use_qk_l2norm_in_kernel=False)
    assert rel_err(o, o_ref) <= 2e-2


def test_half_strided_inputs_bitwise(dev):
    """q / k / v as (B, T, H, d) views of head-major tensors (the layer's and the
    bench's layout) give bit-identical results to contiguous copies."""
    B, T, H, d = 2, 300, 4, 128
    g = torch.Generator().manual_seed(13)
    qh, kh, vh = (torch.randn(B, H, T, d, generator=g).to(torch.bfloat16) for _ in range(3))
    glog = F.logsigmoid(torch.randn(B, T, H, generator=g) + 3.9)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    kw = dict(scale=1.0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    views = [t.to(dev).transpose(1, 2) for t in (qh, kh, vh)]
    o1, S1 = _run(dev, *views, glog, beta, **kw)
    o2, S2 = _run(dev, *[t.contiguous() for t in views], glog, beta, **kw)
    assert torch.equal(o1, o2) and torch.equal(S1, S2)


def test_half_long_sequence(dev):
    """configs[2] length, 16-bit: against the fp32 oracle (whole output), and one call ==
    two calls split at a chunk boundary with the fp32 state carried.  A sequence this long
    with two heads takes the segmented recurrence (segment summaries combined in fp32), so
    the split run agrees to rounding, not bit for bit; the plain scan's bitwise split is
    pinned by test_split_bitwise_plain."""
    B, T, H, d = 1, 65536, 2, 128
    q, k, v, glog, beta, _ = _inputs(B, T, H, d, torch.bfloat16, seed=14)
    kw = dict(scale=1.0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    o, S = _run(dev, q, k, v, glog, beta, initial_state=None, **kw)
    h = T // 2
    o1, S1 = _run(dev, q[:, :h], k[:, :h], v[:, :h], glog[:, :h], beta[:, :h], initial_state=None, **kw)
    o2, S2 = _run(dev, q[:, h:], k[:, h:], v[:, h:], glog[:, h:], beta[:, h:], initial_state=S1, **kw)
    assert rel_err(torch.cat([o1, o2], 1), o) <= 5e-3 and rel_err(S2, S) <= 5e-3
    o_ref, S_ref = OG.chunk_gated_delta_rule(q.float(), k.float(), v.float(), glog, beta, scale=1.0,
                                             output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert rel_err(o, o_ref) <= 2e-2 and rel_err(S, S_ref) <= 2e-2


@pytest.mark.parametrize("dtype,d,T", [(torch.float32, 128, 200), (torch.float32, 64, 65),
                                       (torch.bfloat16, 128, 300), (torch.float16, 64, 129)])
def test_grouped_kv_heads_equal_expanded(dev, dtype, d, T):
    """k / v with Hkv < H heads (query head h reads KV head h // (H // Hkv)) give
    bit-identical results to the reference's repeat_interleave-expanded call, for
    head-major views (the layer's layout), with a carried initial state."""
    B, H, Hkv = 2, 8, 2
    g = torch.Generator().manual_seed(17 + d + T)
    qh = torch.randn(B, H, T, d, generator=g).to(dtype)
    kh, vh = (torch.randn(B, Hkv, T, d, generator=g).to(dtype) for _ in range(2))
    glog = F.logsigmoid(torch.randn(B, T, H, generator=g) + 3.9)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    S0 = torch.randn(B, H, d, d, generator=g) * 0.1
    kw = dict(scale=1.0, initial_state=S0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    q, k, v = (t.to(dev).transpose(1, 2) for t in (qh, kh, vh))
    o1, S1 = _run(dev, q, k, v, glog, beta, **kw)
    kx, vx = (t.repeat_interleave(H // Hkv, 2) for t in (k, v))
    o2, S2 = _run(dev, q, kx, vx, glog, beta, **kw)
    assert torch.equal(o1, o2) and torch.equal(S1, S2)


@pytest.mark.parametrize("dtype,d", [(torch.float32, 128), (torch.bfloat16, 128), (torch.float16, 64)])
def test_raw_gate_logits_equal_gate_kernel_then_call(dev, dtype, d):
    """g / beta as raw logits with gate_bias (activations fused into the prefill's load)
    == the stand-alone gate kernel followed by the plain call, bitwise; and the fused
    form against the oracle fed torch's logsigmoid / sigmoid."""
    from atma_amd.kernel import gated_delta_gates
    B, T, H, Hkv = 2, 200, 4, 2
    g = torch.Generator().manual_seed(31 + d)
    q = torch.randn(B, T, H, d, generator=g).to(dtype)
    k, v = (torch.randn(B, T, Hkv, d, generator=g).to(dtype) for _ in range(2))
    zg = torch.randn(B, T, H, generator=g) * 3
    zb = torch.randn(B, T, H, generator=g) * 3
    S0 = torch.randn(B, H, d, d, generator=g) * 0.1
    kw = dict(scale=1.0, initial_state=S0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    o1, S1 = _run(dev, q, k, v, zg, zb, gate_bias=(3.9, 0.5), **kw)
    glog, beta = gated_delta_gates(zg.to(dev), zb.to(dev), 3.9, 0.5)
    o2, S2 = _run(dev, q, k, v, glog, beta, **kw)
    assert torch.equal(o1, o2) and torch.equal(S1, S2)
    kx, vx = (t.repeat_interleave(H // Hkv, 2) for t in (k, v))
    o_ref, S_ref = OG.chunk_gated_delta_rule(q.double(), kx.double(), vx.double(),
                                             F.logsigmoid(zg.double() + 3.9),
                                             torch.sigmoid(zb.double() + 0.5), scale=1.0,
                                             initial_state=S0.double(), output_final_state=True,
                                             use_qk_l2norm_in_kernel=True)
    if dtype == torch.float32:
        assert max_abs(o1, o_ref) <= 1e-4 and max_abs(S1, S_ref) <= 1e-4
    else:
        assert rel_err(o1, o_ref) <= 2e-2 and rel_err(S1, S_ref) <= 2e-2


def test_split_bitwise_plain(dev):
    """Enough sequence-heads to fill the device take the plain (unsegmented) scan: one call
    == two calls split at a chunk boundary with the fp32 state carried, bit for bit."""
    B, T, H, d = 3, 1024, 8, 128
    q, k, v, glog, beta, _ = _inputs(B, T, H, d, torch.bfloat16, seed=15)
    kw = dict(scale=1.0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    o, S = _run(dev, q, k, v, glog, beta, initial_state=None, **kw)
    h = 576  # a chunk boundary
    o1, S1 = _run(dev, q[:, :h], k[:, :h], v[:, :h], glog[:, :h], beta[:, :h], initial_state=None, **kw)
    o2, S2 = _run(dev, q[:, h:], k[:, h:], v[:, h:], glog[:, h:], beta[:, h:], initial_state=S1, **kw)
    assert torch.equal(torch.cat([o1, o2], 1), o) and torch.equal(S2, S)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_segmented_recurrence(dev, dtype):
    """A long sequence with few heads (two heads, 4,096 tokens: 8 segments of 8 chunks)
    against the fp32 oracle, from an initial state, with its final state."""
    B, T, H, d = 1, 4096, 2, 128
    q, k, v, glog, beta, S0 = _inputs(B, T, H, d, dtype, seed=16)
    kw = dict(scale=1.0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    o, S = _run(dev, q, k, v, glog, beta, initial_state=S0, **kw)
    o_ref, S_ref = OG.chunk_gated_delta_rule(q.float(), k.float(), v.float(), glog, beta, scale=1.0,
                                             initial_state=S0, output_final_state=True,
                                             use_qk_l2norm_in_kernel=True)
    assert rel_err(o, o_ref) <= 2e-2 and rel_err(S, S_ref) <= 2e-2

"""Pins of the global-block oracle's glue (oracle/block.py): parameter naming, conv
direction, causality and the zero-init identities the reference relies on.  The Polar
and gated-delta pieces it composes are pinned in the other oracle tests."""

import pytest
import torch

from oracle import block as OB
from oracle import gated_delta as OG


def _layer(dim=256, dk=64, window=None, seed=0, std=0.02, zero_mem_proj=False):
    from atma_amd.layers.global_attention import GlobalBlock
    torch.manual_seed(seed)
    blk = GlobalBlock(dim, head_dim=dk, window=window)
    with torch.no_grad():
        for n, p in blk.named_parameters():
            if n.startswith("norm"):
                continue
            p.normal_(0.0, std)
        if zero_mem_proj:
            blk.attn.mem.proj.weight.zero_()
            blk.attn.mem.proj.bias.zero_()
    return blk


def _sd(mod):
    return {k: v.detach().clone() for k, v in mod.state_dict().items()}


def test_parameter_names_follow_reference_registration_order():
    from atma_amd.layers.global_attention import PolarAttention
    names = [n for n, _ in PolarAttention(256, head_dim=64).named_parameters()]
    # torch lists a module's own parameters first (model/reference.py:119-123), then its
    # children in registration order: model/blocks.py:520-529 (AtmaAttnBase), mu_proj
    # (model/reference.py:118), then TitansMemory (model/blocks.py:455-461)
    expect = ["v_null", "null_base", "null_slope_raw", "len_gain_raw", "mag_beta_raw",
              "q.weight", "q.bias", "k.weight", "k.bias", "v.weight", "v.bias", "canon_q.weight",
              "canon_k.weight", "canon_v.weight", "proj.weight", "proj.bias", "mu_proj.weight",
              "mu_proj.bias", "mem.w_gamma.weight", "mem.w_gamma.bias", "mem.w_beta.weight", "mem.w_beta.bias",
              "mem.gate.weight", "mem.gate.bias", "mem.proj.weight", "mem.proj.bias"]
    assert names == expect


def test_causal_depthwise_direction():
    torch.manual_seed(0)
    x = torch.randn(2, 3, 10, dtype=torch.float64)
    w = torch.zeros(3, 1, 4, dtype=torch.float64)
    w[:, 0, 3] = 1.0                       # newest tap: identity
    assert torch.equal(OB.causal_depthwise(x, w), x)
    w.zero_()
    w[:, 0, 2] = 1.0                       # one step back: shift right, zero at t=0
    out = OB.causal_depthwise(x, w)
    assert torch.equal(out[..., 1:], x[..., :-1]) and torch.all(out[..., 0] == 0)


def test_mixer_is_causal():
    blk = _layer()
    sd = {k[5:]: v for k, v in _sd(blk).items() if k.startswith("attn.")}
    torch.manual_seed(1)
    x = torch.randn(1, 40, 256)
    y = OB.polar_attention(sd, x, H=4, Hkv=1, dk=64)
    x2 = x.clone()
    x2[:, 25:] += torch.randn(1, 15, 256)
    y2 = OB.polar_attention(sd, x2, H=4, Hkv=1, dk=64)
    assert torch.allclose(y[:, :25], y2[:, :25], atol=1e-6, rtol=0)
    assert (y[:, 25:] - y2[:, 25:]).abs().max() > 1e-3


def test_zero_initialised_memory_projection_is_a_no_op():
    blk = _layer(zero_mem_proj=True)
    sd = {k[5:]: v for k, v in _sd(blk).items() if k.startswith("attn.")}
    x = torch.randn(2, 30, 256)
    a = OB.polar_attention(sd, x, H=4, Hkv=1, dk=64, mem=True)
    b = OB.polar_attention(sd, x, H=4, Hkv=1, dk=64, mem=False)
    assert torch.equal(a, b)


def test_block_reduces_to_identity_with_zero_output_projections():
    blk = _layer()
    with torch.no_grad():
        for m in (blk.attn.proj, blk.attn.mu_proj, blk.attn.mem.proj, blk.mlp.proj):
            m.weight.zero_()
            m.bias.zero_()
    x = torch.randn(2, 17, 256)
    assert torch.equal(OB.global_block(_sd(blk), x, H=4, Hkv=1, dk=64), x)


def test_memory_branch_readout_equals_sequential_definition():
    blk = _layer()
    sd = {k[5:]: v.double() for k, v in _sd(blk).items() if k.startswith("attn.")}
    torch.manual_seed(2)
    x = torch.randn(1, 70, 256, dtype=torch.float64)
    q, k, v, _ = OB.attention_qkv(sd, x, 4, 1, 64)
    km, vm = k.repeat_interleave(4, 1), v.repeat_interleave(4, 1)
    out, S = OB.memory_branch(sd, x, q, km, vm)
    # the same readout from the token-by-token definition (scripts/titans_proto.py:53-76)
    g_logit = OB.linear(x, sd, "mem.w_gamma") + OB.MEM_GAMMA_BIAS
    b_logit = OB.linear(x, sd, "mem.w_beta") + OB.MEM_BETA_BIAS
    r, S_seq = OG.gated_delta_sequential(OG.l2_normalize(q), OG.l2_normalize(km), vm,
                                         torch.sigmoid(g_logit).transpose(1, 2),
                                         torch.sigmoid(b_logit).transpose(1, 2))
    # per-head RMSNorm with the fp32 model's default epsilon (the fp64 oracle's convention)
    r = torch.nn.functional.rms_norm(r.transpose(1, 2), (64,), eps=torch.finfo(torch.float32).eps)
    r = r.reshape(1, 70, 256)
    ref = OB.linear(r * torch.sigmoid(OB.linear(x, sd, "mem.gate")), sd, "mem.proj")
    assert (out - ref).abs().max() < 1e-10
    assert (S - S_seq.transpose(-1, -2)).abs().max() < 1e-10


@pytest.mark.parametrize("window", [None, 8])
def test_window_only_changes_rows_past_the_window(window):
    blk = _layer()
    sd = {k[5:]: v for k, v in _sd(blk).items() if k.startswith("attn.")}
    x = torch.randn(1, 20, 256)
    a = OB.polar_attention(sd, x, H=4, Hkv=1, dk=64, window=window, mem=False)
    b = OB.polar_attention(sd, x, H=4, Hkv=1, dk=64, window=None, mem=False)
    w = window or 20
    assert torch.allclose(a[:, :w], b[:, :w], atol=1e-6)


def test_fp64_oracle_is_the_fp32_function():
    """The fp64 block oracle (the gradient reference of the GPU training tests) computes
    the fp32 model's function at higher precision: per-head RMSNorm keeps fp32's default
    epsilon, so the memory's first rows (tiny readout) agree too."""
    from atma_amd.layers.global_attention import GlobalBlock
    torch.manual_seed(0)
    dim, dk = 256, 64
    blk = GlobalBlock(dim, head_dim=dk)
    with torch.no_grad():
        for n, p in blk.named_parameters():
            if not n.startswith("norm"):
                p.normal_(0.0, 0.02)
            if n in ("attn.null_base", "attn.mag_beta_raw"):
                p.normal_(0.0, 1.0)
    sd = {k: v.detach().clone() for k, v in blk.state_dict().items()}
    x = torch.randn(1, 200, dim, generator=torch.Generator().manual_seed(11))
    o32 = OB.global_block(sd, x, H=dim // dk, Hkv=dim // dk // 4, dk=dk)
    o64 = OB.global_block({k: v.double() for k, v in sd.items()}, x.double(), H=dim // dk,
                          Hkv=dim // dk // 4, dk=dk)
    assert (o32.double() - o64).abs().max().item() <= 5e-6

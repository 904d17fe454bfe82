"""Pins of the whole-model CPU oracle (``oracle/model.py``): the LFM2 conv block against
an explicit per-token restatement of its convolution, causality of the whole model, and
the soft cap's closed-form properties."""

import torch

from oracle import model as OM


def _conv_sd(dim, K, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64) * 0.3  # noqa: E731
    return {"in_proj.weight": r(3 * dim, dim), "in_proj.bias": r(3 * dim), "conv.weight": r(dim, 1, K),
            "out_proj.weight": r(dim, dim), "out_proj.bias": r(dim)}


def test_lfm2_conv_equals_explicit_taps():
    """out_t = out_proj(C_t * sum_j w[:, j] * (B*x)_{t-K+1+j}), zero before the start."""
    dim, K, T = 8, 3, 11
    sd = _conv_sd(dim, K, 0)
    x = torch.randn(2, T, dim, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    got = OM.lfm2_conv(sd, x)
    proj = x @ sd["in_proj.weight"].T + sd["in_proj.bias"]
    b, c, xp = proj[..., :dim], proj[..., dim:2 * dim], proj[..., 2 * dim:]
    xg = b * xp
    w = sd["conv.weight"][:, 0, :]
    want = torch.zeros_like(xg)
    for t in range(T):
        for j in range(K):
            s = t - (K - 1) + j
            if s >= 0:
                want[:, t] += w[:, j] * xg[:, s]
    want = (c * want) @ sd["out_proj.weight"].T + sd["out_proj.bias"]
    assert (got - want).abs().max() < 1e-12


def _model_sd(vocab=64, L=4, dim=64, dk=16, seed=0):
    from atma_amd.engine import Atma, AtmaConfig
    cfg = AtmaConfig(vocab_size=vocab, num_hidden_layers=L, hidden_size=dim, head_dim=dk, dtype=torch.float32)
    m = Atma(cfg).init_weights(0.05, seed)
    sd = {k: v.detach().double() for k, v in m.state_dict().items()}
    for k in sd:
        if k.endswith("norm1.weight") or k.endswith("norm2.weight") or k == "norm.weight":
            sd[k] = torch.ones_like(sd[k])
    return sd, cfg


def test_whole_model_is_causal_and_composed_of_blocks():
    sd, cfg = _model_sd()
    kw = dict(num_layers=cfg.num_hidden_layers, H=cfg.num_attention_heads, Hkv=cfg.num_key_value_heads,
              dk=cfg.head_dim)
    ids = torch.randint(0, cfg.vocab_size, (1, 20), generator=torch.Generator().manual_seed(2))
    full = OM.atma_logits(sd, ids, **kw)
    pre = OM.atma_logits(sd, ids[:, :13], **kw)
    assert full.shape == (1, 20, cfg.vocab_size)
    assert (full[:, :13] - pre).abs().max() < 1e-10           # a token never sees the future
    changed = ids.clone()
    changed[0, 15] = (changed[0, 15] + 1) % cfg.vocab_size
    other = OM.atma_logits(sd, changed, **kw)
    assert (other[:, :15] - full[:, :15]).abs().max() < 1e-10 and (other[:, 15:] - full[:, 15:]).abs().max() > 0


def test_softcap_closed_form():
    x = torch.linspace(-1e4, 1e4, 20001, dtype=torch.float64)
    y = OM.softcap(x)
    assert (y.abs() < 15).all() and torch.equal(OM.softcap(-x), -y)
    assert (y[1:] > y[:-1]).all()                               # strictly increasing
    small = torch.tensor([1e-6, -3e-5], dtype=torch.float64)
    assert torch.allclose(OM.softcap(small), small, rtol=1e-9)  # ~x near 0

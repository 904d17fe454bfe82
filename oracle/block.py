"""CPU oracle of one ATMA global block -- TEST INFRASTRUCTURE ONLY.

A functional restatement, over a plain ``{name: tensor}`` parameter dict whose keys
follow the reference's module registration order, of:

* ``PolarAttention.forward`` (``model/reference.py:127-195``): q/gate, k, v
  projections, per-head RMSNorm of q and k, the Canon causal depthwise conv on q/k/v
  (residual), GQA expansion, the materialised Polar reduction, ``proj(c *
  sigmoid(gate)) + mu_proj(mag)``;
* the Titans memory branch, torch path (``model/blocks.py:463-490``): retention /
  write logits with biases +3.9 / +0.0, unit-normalised q/k, the chunked gated-delta
  scan, per-head RMSNorm of the readout, ``proj(r * sigmoid(gate(x)))``;
* ``Block.forward`` (``model/reference.py:226-229``): pre-norm residual mixer + the
  squared-ReLU MLP (``model/layers.py:6-31``).

The layer routes are built from the pinned oracle functions (``polar_dense``,
``gated_delta_chunked``); the glue (linear layers, RMSNorm, depthwise conv, gating)
is restated here and pinned against the reference's own modules by the golden tensors
of ``tests/golden/block_glue.pt`` (``tests/test_oracle_golden.py``: fp64 bit for bit, fp32
within 5e-6), and in ``tests/test_oracle_block.py`` by causality, the zero-init identities
the reference relies on, and prefill/decode consistency.
"""

import torch
import torch.nn.functional as F

from .gated_delta import gated_delta_chunked, l2_normalize
from .polar import polar_dense

MEM_GAMMA_BIAS = 3.9   # model/config.py:43, model/blocks.py:466
MEM_BETA_BIAS = 0.0    # model/config.py:44, model/blocks.py:467


def linear(x, sd, name):
    """``Linear.forward`` (``model/reference.py:22-28``): weight/bias cast to x's dtype."""
    b = sd.get(name + ".bias")
    return F.linear(x, sd[name + ".weight"].to(x.dtype), None if b is None else b.to(x.dtype))


def head_rms_norm(x, dk, native_eps=False):
    """Per-head ``F.rms_norm(x, (dk,))`` with torch's default epsilon of the model's
    compute dtype (``model/reference.py:136-137``, ``model/blocks.py:488``).  Left to
    itself torch uses ``finfo(x.dtype).eps``, so an fp64 oracle would compute a
    different function (eps 2.2e-16 instead of fp32's 1.2e-7), visible on rows whose
    readout is tiny (the memory's first token); the fp64 form therefore keeps fp32's
    epsilon and differs from the fp32 model only by rounding.  ``native_eps=True`` keeps
    torch's default instead: what the reference module computes when it is itself run
    in fp64 (the golden fixtures)."""
    eps = torch.finfo(torch.float32).eps if x.dtype == torch.float64 and not native_eps else None
    return F.rms_norm(x, (dk,), eps=eps)


def causal_depthwise(x_in, weight):
    """Causal depthwise conv over time: x_in (B, C, T), weight (C, 1, K), left zero pad
    K-1 (``model/reference.py:143-145``)."""
    K = weight.shape[-1]
    return F.conv1d(F.pad(x_in, (K - 1, 0)), weight.to(x_in.dtype), groups=x_in.shape[1])


def attention_qkv(sd, x, H, Hkv, dk, native_eps=False):
    """Projections, RMSNorm, Canon conv (``model/reference.py:131-155``).
    Returns q (B,H,T,dk), k, v (B,Hkv,T,dk) unexpanded, gate (B,T,H*dk)."""
    B, T, _ = x.shape
    qg = linear(x, sd, "q").view(B, T, H, 2 * dk)
    q, gate = torch.chunk(qg, 2, dim=-1)
    k = linear(x, sd, "k").view(B, T, Hkv, dk)
    v = linear(x, sd, "v").view(B, T, Hkv, dk)
    q = head_rms_norm(q, dk, native_eps)
    k = head_rms_norm(k, dk, native_eps)
    outs = []
    for t, name, h in ((q, "canon_q", H), (k, "canon_k", Hkv), (v, "canon_v", Hkv)):
        t_in = t.reshape(B, T, h * dk).transpose(1, 2)
        t_out = t_in + causal_depthwise(t_in, sd[name + ".weight"])
        outs.append(t_out.transpose(1, 2).reshape(B, T, h, dk).transpose(1, 2))
    return outs[0], outs[1], outs[2], gate.reshape(B, T, H * dk)


def polar_params(sd):
    return {n: sd[n] for n in ("v_null", "null_base", "null_slope_raw", "len_gain_raw", "mag_beta_raw")}


def memory_branch(sd, x, q_t, k_t, v_t, S0=None, chunk=64):
    """TitansMemory torch path (``model/blocks.py:463-490``).  q_t, k_t, v_t: (B,H,T,dk)
    with KV expanded.  S0: optional ``[K,V]`` (B,H,dk,dv) initial state (the engine's
    table layout).  Returns (out (B,T,dim), final state ``[K,V]``)."""
    B, H, T, dk = q_t.shape
    wd = torch.float64 if x.dtype == torch.float64 else torch.float32
    g_logit = linear(x, sd, "mem.w_gamma").to(wd) + MEM_GAMMA_BIAS
    b_logit = linear(x, sd, "mem.w_beta").to(wd) + MEM_BETA_BIAS
    gamma = torch.sigmoid(g_logit).transpose(1, 2)
    beta = torch.sigmoid(b_logit).transpose(1, 2)
    qn = l2_normalize(q_t.to(wd))
    kn = l2_normalize(k_t.to(wd))
    S0t = None if S0 is None else S0.to(wd).transpose(-1, -2)
    r, S = gated_delta_chunked(qn, kn, v_t.to(wd), gamma, beta, chunk=chunk, S0=S0t)
    r = head_rms_norm(r.transpose(1, 2), dk)
    r_flat = r.reshape(B, T, H * dk).to(x.dtype)
    out = linear(r_flat * torch.sigmoid(linear(x, sd, "mem.gate")), sd, "mem.proj")
    return out, S.transpose(-1, -2)


def polar_attention(sd, x, *, H, Hkv, dk, window=None, mem=True, native_eps=False):
    """``PolarAttention.forward`` (``model/reference.py:127-195``), causal over x (B,T,dim).
    ``native_eps``: see ``head_rms_norm``."""
    B, T, _ = x.shape
    q, k, v, gate = attention_qkv(sd, x, H, Hkv, dk, native_eps)
    n_keys = torch.arange(1, T + 1, dtype=torch.float32)
    c, mag = polar_dense(q, k, v, n_keys, params=polar_params(sd), window=window)
    c_flat = c.transpose(1, 2).reshape(B, T, H * dk)
    out = linear(c_flat * torch.sigmoid(gate), sd, "proj") + linear(mag.transpose(1, 2), sd, "mu_proj")
    if mem:
        g = H // Hkv
        out = out + memory_branch(sd, x, q, k.repeat_interleave(g, 1), v.repeat_interleave(g, 1))[0]
    return out


def rms_norm_weighted(x, w, eps=1e-6):
    """``RMSNorm.forward`` (``model/layers.py:6-16``)."""
    return F.rms_norm(x, (x.shape[-1],), weight=w.to(x.dtype), eps=eps)


def mlp(sd, x, prefix="mlp"):
    """Squared-ReLU gated MLP (``model/layers.py:19-31``)."""
    xg = linear(x, sd, prefix + ".fc")
    a, gate = torch.chunk(xg, 2, dim=-1)
    return linear(gate * a.relu().square(), sd, prefix + ".proj")


def global_block(sd, x, *, H, Hkv, dk, window=None, mem=True, native_eps=False):
    """``Block.forward`` (``model/reference.py:226-229``) for an attention block; the
    mixer's parameters live under ``attn.``."""
    attn_sd = {k[5:]: t for k, t in sd.items() if k.startswith("attn.")}
    x = x + polar_attention(attn_sd, rms_norm_weighted(x, sd["norm1.weight"]), H=H, Hkv=Hkv, dk=dk,
                            window=window, mem=mem, native_eps=native_eps)
    return x + mlp(sd, rms_norm_weighted(x, sd["norm2.weight"]))

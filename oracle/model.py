"""CPU oracle of the whole ATMA model -- TEST INFRASTRUCTURE ONLY (see ``oracle/__init__``).

``ReferenceModel.forward`` (``model/reference.py:236-269``) over a ``{name: tensor}``
state dict with the reference's keys: token embedding, blocks in Local-Local-Global-Local
order (``i % 4 == 2`` global, ``:245``), final RMSNorm, LM head, then the fp32 soft cap
``15 x / sqrt(x^2 + 225)`` (``:265-266``).  The LFM2 conv block restates
``LFM2Conv.forward`` (``model/reference.py:31-48``); the global block is
``oracle/block.global_block``.  Pinned against the reference's ``LFM2Conv``, conv ``Block``
and a 4-block ``ReferenceModel`` by the golden tensors of ``tests/golden/block_glue.pt``
(``tests/test_oracle_golden.py``), and in ``tests/test_oracle_model.py`` (conv block == an
explicit per-token loop, causality, composition).
"""

import torch
import torch.nn.functional as F

from .block import causal_depthwise, global_block, linear, mlp, rms_norm_weighted


def lfm2_conv(sd, x):
    """``LFM2Conv.forward`` (``model/reference.py:37-48``): ``B, C, x = in_proj(x)``,
    causal depthwise conv (left zero pad K-1) of ``B * x``, then ``out_proj(C * conv)``.
    x: (B, T, dim); sd keys ``in_proj.*``, ``conv.weight``, ``out_proj.*``."""
    b_gate, c_gate, x_proj = linear(x, sd, "in_proj").chunk(3, dim=-1)
    xg = (b_gate * x_proj).transpose(1, 2)
    return linear(c_gate * causal_depthwise(xg, sd["conv.weight"]).transpose(1, 2), sd, "out_proj")


def conv_block(sd, x):
    """``Block.forward`` (``model/reference.py:226-229``) for a conv block."""
    attn_sd = {k[5:]: t for k, t in sd.items() if k.startswith("attn.")}
    x = x + lfm2_conv(attn_sd, rms_norm_weighted(x, sd["norm1.weight"]))
    return x + mlp(sd, rms_norm_weighted(x, sd["norm2.weight"]))


def softcap(logits):
    """``model/reference.py:265-266``, in the logits' dtype (fp32 there)."""
    return 15.0 * logits * (logits.square() + 225.0).rsqrt()


def atma_logits(sd, input_ids, *, num_layers, H, Hkv, dk, window=None, mem=True):
    """Logits (B, T, vocab) fp32 (fp64 for an fp64 state dict) of every position.
    input_ids: (B, T) int64."""
    emb = sd["embed.weight"]
    x = F.embedding(input_ids, emb)
    for i in range(num_layers):
        pre = f"blocks.{i}."
        bsd = {k[len(pre):]: t for k, t in sd.items() if k.startswith(pre)}
        if i % 4 == 2:
            x = global_block(bsd, x, H=H, Hkv=Hkv, dk=dk, window=window, mem=mem)
        else:
            x = conv_block(bsd, x)
    logits = linear(rms_norm_weighted(x, sd["norm.weight"]), sd, "proj")
    return softcap(logits.to(torch.promote_types(logits.dtype, torch.float32)))

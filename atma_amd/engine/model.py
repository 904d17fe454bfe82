"""The paged-engine ATMA model (``inference/models/atma.py:195-754``): 16 pre-norm blocks in
Local-Local-Global-Local order -- LFM2 gated depthwise-conv blocks and global blocks
(Polar attention + gated-delta memory) -- between a token embedding and a soft-capped LM
head.  Parameter names follow the reference (``embed``, ``blocks.{i}.attn.*``,
``blocks.{i}.mlp.*``, ``blocks.{i}.norm{1,2}``, ``norm``, ``proj``), so its checkpoints load.

Every layer reads the engine's thread-local ``Context`` to pick its route:

* dense prefill (fresh, equal-length prompts): the global layer's batched route, the
  LFM2 conv as one packed HIP launch;
* grouped prefill (fresh ragged prompts, 16-bit): one tile-mapped Polar launch
  (``PolarAttention.prefill_packed``), packed convs;
* per-sequence prefill (fp32 ragged prompts, chunked continuations): gathered paged
  prefix + chunk (``PolarAttention.prefill_continue``), convs from the stored tails;
* decode: one token per sequence, graph capturable (paged Polar decode, in-place conv
  and memory steps).
"""

import torch
import torch.nn.functional as F
from torch import nn

from ..kernel import causal_conv1d_decode_step, packed_causal_conv1d, softcap_argmax, softcap_logits
from ..kernel.decode_fusions import (PartialSums, lfm2_conv_step, linear_tokens_conv, linear_tokens_conv_supported,
                                     residual_rms_norm_supported)
from ..kernel.layer_fusions import lfm2_conv_packed
from ..layers.attention import Attention
from ..layers.global_attention import MLP, GlobalLayerCache, Linear, PolarAttention, RMSNorm, decode_rows
from .config import AtmaConfig
from .context import get_context


class AtmaAttention(PolarAttention):
    """The global layer inside the engine (``AtmaAttention``, ``inference/models/atma.py:195-618``):
    the mixer of ``PolarAttention`` plus the paged-cache holder ``attn`` and the layer's
    state-table keys ``attn_{i}_{q,k,v}`` / ``mem_{i}``."""

    def __init__(self, layer_idx, dim, head_dim=128, num_kv_heads=None, kernel_size=4, window=None,
                 mem_enabled=True, mem_chunk=64, mem_gamma_bias=3.9, mem_beta_bias=0.0):
        super().__init__(dim, head_dim=head_dim, num_kv_heads=num_kv_heads, kernel_size=kernel_size,
                         window=window, mem_enabled=mem_enabled, mem_chunk=mem_chunk,
                         mem_gamma_bias=mem_gamma_bias, mem_beta_bias=mem_beta_bias)
        self.layer_idx = layer_idx
        self.attn = Attention(self.num_heads, self.head_dim, self.head_dim ** -0.5, self.num_kv_heads)

    def _cache(self, ctx) -> GlobalLayerCache:
        t, i = ctx.conv_state_tables, self.layer_idx
        return GlobalLayerCache(k_cache=self.attn.k_cache, v_cache=self.attn.v_cache, conv_q=t[f"attn_{i}_q"],
                                conv_k=t[f"attn_{i}_k"], conv_v=t[f"attn_{i}_v"], mem_table=t.get(f"mem_{i}"))

    def forward(self, x, defer=False):
        """x: (tokens, dim) -- the packed prefill tokens or one token per decoding sequence.
        ``defer``: a fused decode step may return its output projections unsummed
        (``PartialSums``, finished by the next residual norm)."""
        ctx = get_context()
        cache = self._cache(ctx)
        if not ctx.is_prefill:
            return self.decode(x, cache, ctx.seq_slots, ctx.block_tables, ctx.context_lens, ctx.slot_mapping,
                               defer=defer)
        if ctx.dense_prefill:
            B, T = ctx.dense_batch_size, ctx.dense_seq_len
            out = self.prefill(x.view(B, T, -1), cache, ctx.seq_slots, ctx.slot_mapping, defer=defer)
            return out if isinstance(out, PartialSums) else out.reshape(B * T, -1)
        if ctx.grouped_polar_prefill:
            return self.prefill_packed(
                x, cache, ctx.seqlens_q, ctx.seq_slots, ctx.slot_mapping,
                (ctx.polar_tile_seq_starts, ctx.polar_tile_q_starts, ctx.polar_tile_seq_lens),
                (ctx.token_seq_starts, ctx.token_seq_ends, ctx.token_seq_slots), defer=defer)
        outs, start = [], 0
        for i, n in enumerate(ctx.seqlens_q):
            seq = ctx.seqs[i]
            bt = None if ctx.block_tables is None else ctx.block_tables[i:i + 1]
            outs.append(self.prefill_continue(x[start:start + n][None], cache, ctx.seq_slots[i:i + 1],
                                              ctx.slot_mapping[start:start + n], bt,
                                              [seq.num_cached_tokens])[0])
            start += n
        return torch.cat(outs, 0)


class AtmaLFM2Conv(nn.Module):
    """LFM2 gated depthwise-conv block (``AtmaLFM2Conv``, ``inference/models/atma.py:625-673``;
    math ``model/reference.py:31-48``): ``B, C, x = in_proj(x)``, ``out_proj(C * conv(B * x))``
    with a causal depthwise conv of ``kernel_size`` taps whose last inputs per sequence live
    in the state table ``conv_{i}_gated``."""

    def __init__(self, layer_idx, dim, kernel_size=3):
        super().__init__()
        self.hidden_size = dim
        self.kernel_size = kernel_size
        self.in_proj = Linear(dim, 3 * dim)
        self.conv = nn.Conv1d(dim, dim, kernel_size=kernel_size, padding=kernel_size - 1, groups=dim, bias=False)
        self.out_proj = Linear(dim, dim)
        self.layer_idx = layer_idx

    def forward(self, x, defer=False):
        ctx = get_context()
        table = ctx.conv_state_tables[f"conv_{self.layer_idx}_gated"]
        if not ctx.is_prefill and decode_rows(x):
            taps = self.conv.weight.squeeze(1)
            w = self.in_proj.weight
            if x.is_contiguous() and w.dtype == x.dtype and linear_tokens_conv_supported(x, w, taps):
                # in_proj, b * x, the conv step and c * (.) in one launch (linear_tokens_conv)
                return self.out_proj(linear_tokens_conv(x, w, self.in_proj.bias, taps, ctx.seq_slots, table))
            # one launch for b * x, the conv step and c * (.) (lfm2_conv_step)
            return self.out_proj(lfm2_conv_step(self.in_proj(x), taps, ctx.seq_slots, table))
        if (ctx.is_prefill and ctx.token_seq_starts is not None and x.is_cuda and not torch.is_grad_enabled()
                and x.dtype in (torch.bfloat16, torch.float16) and x.shape[-1] % 8 == 0 and self.kernel_size in (3, 4)):
            # fresh prompts: b * x, the packed conv and c * (.) in one launch (lfm2_conv_packed)
            return self.out_proj(lfm2_conv_packed(self.in_proj(x), self.conv.weight.squeeze(1), table,
                                                  ctx.token_seq_starts, ctx.token_seq_ends, ctx.token_seq_slots))
        b_gate, c_gate, x_proj = self.in_proj(x).chunk(3, dim=-1)
        xg = b_gate * x_proj
        w = self.conv.weight.squeeze(1)
        if not ctx.is_prefill:
            xc = causal_conv1d_decode_step(xg, w, ctx.seq_slots, table)
        elif ctx.token_seq_starts is not None:        # fresh prompts: one packed launch, tails written
            xc = packed_causal_conv1d(xg, w, table, ctx.token_seq_starts, ctx.token_seq_ends, ctx.token_seq_slots)
        else:
            xc = self._conv_per_sequence(xg, w, table, ctx)
        return self.out_proj(c_gate * xc)

    def _conv_per_sequence(self, xg, w, table, ctx):
        """``prefill_causal_conv1d`` (``inference/models/atma.py:102-139``): a fresh
        sequence pads with zeros, a continuation with its stored tail; the new tail is the
        last K-1 columns of the padded stream."""
        K = self.kernel_size
        outs, start = [], 0
        for i, n in enumerate(ctx.seqlens_q):
            seq = ctx.seqs[i]
            xi = xg[start:start + n].t()[None]                               # (1, C, n)
            left = (table[seq.seq_slot].to(xi.dtype)[None] if seq.num_cached_tokens > 0
                    else xi.new_zeros(1, xi.shape[1], K - 1))
            padded = torch.cat([left, xi], dim=2)
            outs.append(F.conv1d(padded, w.to(xi.dtype).unsqueeze(1), groups=xi.shape[1])[0].t())
            table[seq.seq_slot] = padded[0, :, padded.shape[2] - (K - 1):].to(table.dtype)
            start += n
        return torch.cat(outs, 0)


class AtmaDecoderBlock(nn.Module):
    """Pre-norm block (``inference/models/atma.py:680-713``): ``x + attn(norm1 x)``, then
    ``x + mlp(norm2 x)``; the mixer is global for ``i % 4 == 2``, LFM2 conv otherwise."""

    def __init__(self, layer_idx, config: AtmaConfig):
        super().__init__()
        dim = config.hidden_size
        if config.is_attention_layer(layer_idx):
            self.attn = AtmaAttention(layer_idx, dim, head_dim=config.head_dim,
                                      num_kv_heads=config.num_key_value_heads,
                                      kernel_size=config.attn_kernel_size, window=config.attn_window,
                                      mem_enabled=config.mem_enabled, mem_chunk=config.mem_chunk,
                                      mem_gamma_bias=config.mem_gamma_bias, mem_beta_bias=config.mem_beta_bias)
        else:
            self.attn = AtmaLFM2Conv(layer_idx, dim, kernel_size=config.conv_kernel_size)
        self.mlp = MLP(dim)
        self.norm1 = RMSNorm(dim, config.rms_norm_eps)
        self.norm2 = RMSNorm(dim, config.rms_norm_eps)

    def forward(self, x):
        x = x + self.attn(self.norm1(x))
        return x + self.mlp(self.norm2(x))

    def forward_stream(self, branch, residual):
        """The same block over the residual stream: the previous block's branch output
        and the stream before it go in, each add is fused with the norm after it
        (``RMSNorm.add_norm``), and this block's MLP output comes out unadded -- the
        additions are the eager block's, in the same dtype, so the stream's values are
        unchanged.  Returns (mlp branch, stream)."""
        h, residual = self.norm1.add_norm(branch, residual)
        h, residual = self.norm2.add_norm(self.attn(h, defer=True), residual)
        return self.mlp(h, defer=True), residual


class Atma(nn.Module):
    """The served model (``Atma``, ``inference/models/atma.py:716-754``)."""

    def __init__(self, config: AtmaConfig):
        super().__init__()
        self.config = config
        self.embed = nn.Embedding(config.vocab_size, config.hidden_size)
        self.blocks = nn.ModuleList([AtmaDecoderBlock(i, config) for i in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.proj = Linear(config.hidden_size, config.vocab_size)     # LM head, with bias

    def forward(self, input_ids, positions=None):
        """Hidden states of every scheduled token (no positions: the model has none).
        16-bit inference runs the blocks over the residual stream (``forward_stream``:
        every residual add fused with the norm that follows it)."""
        x = self.embed(input_ids)
        if torch.is_grad_enabled() or not residual_rms_norm_supported(x):
            for block in self.blocks:
                x = block(x)
            return self.norm(x)
        branch, residual = x, None
        for block in self.blocks:
            branch, residual = block.forward_stream(branch, residual)
        return self.norm.add_norm(branch, residual)[0]

    def compute_logits(self, hidden):
        """LM head + soft cap ``15 x / sqrt(x^2 + 225)`` (HIP ``softcap_logits``); at prefill
        only each sequence's last token (``inference/layers/embed_head.py:64-74``)."""
        ctx = get_context()
        if ctx.is_prefill and ctx.cu_seqlens_q is not None:
            hidden = hidden[ctx.cu_seqlens_q[1:].long() - 1]
        return softcap_logits(self.proj(hidden))

    def decode_head(self, hidden, ids_out=None):
        """Logits of one token per decoding sequence and, for 16-bit models, their greedy
        ids from the same pass over the logits (``softcap_argmax``, into ``ids_out`` when
        given); graph capturable.  Returns (logits, ids or None)."""
        logits = self.proj(hidden)
        if logits.dtype in (torch.bfloat16, torch.float16):
            return softcap_argmax(logits, ids_out)
        return softcap_logits(logits), None

    def init_weights(self, std=0.02, seed=0):
        """Every parameter N(0, std) from ``seed`` (the random-init convention of the
        reference's tests and of BASELINE configs[4]), drawn on the CPU in registration
        order so the values do not depend on the device."""
        g = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=g, dtype=torch.float32) * std)
        return self


class Sampler(nn.Module):
    """Next-token sampler (``inference/layers/sampler.py:5-10``) with a greedy mode: rows
    whose temperature is 0 take the argmax; the others sample by the reference's
    exponential race over ``softmax(logits / t)``."""

    def forward(self, logits, temperatures, all_greedy=False):
        logits = logits.float()
        greedy = logits.argmax(dim=-1)
        if all_greedy:
            return greedy
        t = temperatures.unsqueeze(1)
        probs = torch.softmax(logits / torch.where(t > 0, t, torch.ones_like(t)), dim=-1)
        race = probs / torch.empty_like(probs).exponential_(1).clamp_min_(1e-10)
        return torch.where(temperatures > 0, race.argmax(dim=-1), greedy)

"""The global-layer mixer as a PyTorch module: Polar attention + the Titans
gated-delta memory, with the reference's parameter names and three routes.

* ``forward(x)`` -- the causal full-sequence form of ``PolarAttention.forward``
  (``model/reference.py:127-195``, memory ``model/blocks.py:463-490``).
* ``prefill(x, cache, ...)`` -- the engine's dense fresh-prefill route
  (``inference/models/atma.py:397-437``): writes the paged KV cache, the Canon conv
  states and the memory state table.
* ``decode(x, cache, ...)`` -- the engine's decode route
  (``inference/models/atma.py:546-618``): one token per sequence against the paged
  cache; conv / memory states advance in place.  Fixed shapes, no host sync:
  graph capturable.

The Polar and gated-delta arithmetic runs in the HIP kernels (``atma_amd.kernel``);
projections, RMSNorm and the depthwise Canon conv stay eager, as in the reference.
Unlike the reference, K/V reach the Polar and gated-delta kernels unexpanded (GQA is
resolved in-kernel).
Prefill schedule (``overlap``): the memory branch may run on a second HIP stream beside
Polar attention (the two only share their inputs).  The gated-delta recurrence is
latency-bound with one workgroup per CU, so this pays only when its grid is small (a
quarter of the CUs or less: long sequences, small batches), and only if its workgroups
start before Polar's fill the GPU; Polar's launch therefore waits on the recurrence's
start signal (``StartSignal``).  ``overlap="auto"`` (default) takes the overlapped
schedule exactly when ``recurrence_pays_to_overlap`` says so, ``True`` always, ``False``
never.  Results are bitwise the same in every schedule.
Training: when autograd must see the call (grad mode on and an input or parameter
requiring grad), the full-sequence route runs the differentiable ops -- ``polar_attention``
(HIP forward with saved statistics + HIP backward) and the autograd form of
``chunk_gated_delta_rule`` -- back to back on one stream, as the reference's training
layer is differentiable (``model/reference.py:172``, ``train/model.py:747-754``).
"""

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn

from ..kernel import (StartSignal, causal_conv1d_decode_step, chunk_gated_delta_rule,
                      gated_delta_decode_step, gated_delta_gates, global_decode_step, polar_attention,
                      polar_attention_decode, polar_attention_fwd, polar_attention_packed_fwd,
                      recurrence_pays_to_overlap)
from ..kernel.decode_fusions import (PartialSums, chunk_width, global_decode_gate, global_decode_prep,
                                     linear_tokens_chunks, linear_tokens_gated, linear_tokens_multi,
                                     linear_tokens_multi_supported,
                                     residual_rms_norm, residual_rms_norm_supported)
from ..kernel.inference_ops import (linear_tokens, linear_tokens_supported, packed_causal_conv1d,
                                     squared_relu_gate)
from ..kernel.layer_fusions import global_gate, head_rms_norm, linear_gated, linear_gated_supported
from ..kernel.polar import global_decode_step_supported_shape
from .attention import store_kvcache

# torch's rms_norm without eps uses its compute type's epsilon: fp32's for 16-bit and fp32 rows
F32_EPS = torch.finfo(torch.float32).eps


def decode_rows(x):
    """True for the decode step's activations: a few token rows (<= 32, one per
    sequence) in 16 bits on the GPU, outside autograd -- the shapes the decode fusions
    (linear_tokens and kernel/decode_fusions) serve."""
    return (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and x.dim() == 2 and x.shape[0] <= 32
            and x.is_contiguous() and not torch.is_grad_enabled())


# Polar structural priors (model/reference.py:17-20)
LEN_GAIN_INIT = -1.0
NULL_SLOPE_INIT = 0.5
NULL_BASE_INIT = 2.0
MAG_BETA_INIT = -1.5


class Linear(nn.Linear):
    """``F.linear`` with weights cast to the input dtype (``model/reference.py:22-28``).

    Inference calls on a few token rows (a decode step: one row per sequence) at the shapes
    ``linear_tokens`` serves run that HIP kernel, which streams the weights once; every
    other call (training, prefill, other shapes) is ``F.linear``."""

    def forward(self, x):
        w = self.weight.type_as(x)
        b = None if self.bias is None else self.bias.type_as(x)
        if x.is_cuda and not torch.is_grad_enabled() and x.dim() >= 1 and x.stride(-1) == 1:
            K = x.shape[-1]
            rows = x.numel() // K if K else 0
            if linear_tokens_supported(rows, w.shape[0], K, x.dtype) and x.is_contiguous():
                return linear_tokens(x.reshape(rows, K), w, b).view(*x.shape[:-1], w.shape[0])
        return F.linear(x, w, b)


class TitansMemory(nn.Module):
    """Gated-delta compression memory (``model/blocks.py:426-490``): retention
    ``gamma = sigmoid(w_gamma x + 3.9)``, write strength ``beta = sigmoid(w_beta x + 0)``,
    unit-normalised q/k in-kernel, readout RMS-normed per head, output-gated and
    projected (``proj`` zero-initialised, so the branch starts as a no-op)."""

    def __init__(self, dim, num_heads, head_dim, chunk=64, gamma_bias=3.9, beta_bias=0.0):
        super().__init__()
        self.H, self.dk, self.chunk = num_heads, head_dim, chunk
        self.gamma_bias, self.beta_bias = gamma_bias, beta_bias
        self.w_gamma = Linear(dim, num_heads)
        self.w_beta = Linear(dim, num_heads)
        self.gate = Linear(dim, num_heads * head_dim)
        self.proj = Linear(num_heads * head_dim, dim)
        nn.init.zeros_(self.proj.weight)
        nn.init.zeros_(self.proj.bias)

    def raw_logits(self, x):
        """Gate logits before the biases (fp32); the biases are added by the fused
        gate kernel together with the activations."""
        return self.w_gamma(x).float(), self.w_beta(x).float()

    def _out(self, x, r):
        lead = r.shape[:-2]
        r = F.rms_norm(r, (self.dk,)).reshape(*lead, self.H * self.dk).to(x.dtype)
        return self.proj(r * torch.sigmoid(self.gate(x)))

    def forward(self, x, q, k, v, initial_state=None, output_final_state=False, start_signal=None):
        """x: (B, T, dim); q: (B, T, H, dk); k, v: (B, T, Hkv, dk) with H % Hkv == 0
        (the kernel maps query head h to KV head h // (H // Hkv), so the reference's
        repeat_interleave expansion is not materialised).  initial_state:
        ``[K, V]`` (B, H, dk, dv) fp32 or None.  ``start_signal``: raised as the recurrence
        kernel starts (the overlapped prefill schedule).  Returns (out (B, T, dim), final
        state or None) -- ``_mem_prefill_dense`` (``inference/models/atma.py:305-339``)."""
        r, S = self.readout(x, q, k, v, initial_state, output_final_state, start_signal)
        return self._out(x, r), S

    def readout(self, x, q, k, v, initial_state=None, output_final_state=False, start_signal=None):
        """The recurrence alone: (r (B, T, H, dk) fp32 readout before its norm and gate,
        final state or None) -- what ``forward`` feeds ``_out``."""
        zg, zb = self.raw_logits(x)   # activations applied inside the prefill's load
        return chunk_gated_delta_rule(q, k, v, zg, zb, scale=1.0, initial_state=initial_state,
                                      output_final_state=output_final_state, use_qk_l2norm_in_kernel=True,
                                      gate_bias=(self.gamma_bias, self.beta_bias), start_signal=start_signal)

    def decode_gates(self, x):
        """(gamma, beta) of one decode step: retention sigmoid(w_gamma x + gamma_bias) and
        write strength sigmoid(w_beta x + beta_bias), fp32 (B, H)."""
        return gated_delta_gates(*self.raw_logits(x), self.gamma_bias, self.beta_bias,
                                 decay_as_prob=True)

    def step(self, x, q, k, v, state_table, slots):
        """One decode step, state table advanced in place (``_mem_decode``,
        ``inference/models/atma.py:341-375``).  x: (B, dim); q: (B, H, dk); k, v:
        (B, Hkv, dk), grouped heads read in-kernel."""
        gamma, beta = self.decode_gates(x)
        r = gated_delta_decode_step(q, k, v, gamma, beta, state_table, slots)
        return self._out(x, r)


@dataclass
class GlobalLayerCache:
    """Per-layer engine state (``inference/engine/model_runner.py:176-193``):
    paged K/V ``(num_pages, page_size, Hkv, d)``, Canon conv tails
    ``(max_seqs, channels, kernel_size - 1)`` for q / k / v, and the memory table
    ``(max_seqs, H, dk, dv)`` fp32 ``[K, V]``."""
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    conv_q: torch.Tensor
    conv_k: torch.Tensor
    conv_v: torch.Tensor
    mem_table: Optional[torch.Tensor] = None

    @staticmethod
    def allocate(layer, num_pages, page_size, max_seqs, device, dtype):
        H, Hkv, dk, K = layer.num_heads, layer.num_kv_heads, layer.head_dim, layer.kernel_size
        z = lambda *s, dt=dtype: torch.zeros(*s, device=device, dtype=dt)  # noqa: E731
        return GlobalLayerCache(
            k_cache=z(num_pages, page_size, Hkv, dk), v_cache=z(num_pages, page_size, Hkv, dk),
            conv_q=z(max_seqs, H * dk, K - 1), conv_k=z(max_seqs, Hkv * dk, K - 1),
            conv_v=z(max_seqs, Hkv * dk, K - 1),
            mem_table=z(max_seqs, H, dk, dk, dt=torch.float32) if layer.mem is not None else None)


class PolarAttention(nn.Module):
    """ATMA's global-layer mixer.  Parameters are registered in the reference's order
    (``model/blocks.py:511-529``, then ``model/reference.py:113-125``) so state dicts
    line up: q, k, v, canon_q, canon_k, canon_v, proj, mu_proj, v_null, null_base,
    null_slope_raw, len_gain_raw, mag_beta_raw, mem.*"""

    def __init__(self, dim, head_dim=128, num_kv_heads=None, kernel_size=4, window=None,
                 mem_enabled=True, mem_chunk=64, mem_gamma_bias=3.9, mem_beta_bias=0.0,
                 num_heads=None, overlap="auto"):
        super().__init__()
        self.num_heads = num_heads if num_heads is not None else dim // head_dim
        self.num_kv_heads = num_kv_heads if num_kv_heads is not None else self.num_heads // 4
        self.head_dim = head_dim
        self.kernel_size = kernel_size
        H, Hkv, dk = self.num_heads, self.num_kv_heads, head_dim
        hd, kvd = H * dk, Hkv * dk
        self.q = Linear(dim, 2 * hd)
        self.k = Linear(dim, kvd)
        self.v = Linear(dim, kvd)
        self.canon_q = nn.Conv1d(hd, hd, kernel_size, padding=kernel_size - 1, groups=hd, bias=False)
        self.canon_k = nn.Conv1d(kvd, kvd, kernel_size, padding=kernel_size - 1, groups=kvd, bias=False)
        self.canon_v = nn.Conv1d(kvd, kvd, kernel_size, padding=kernel_size - 1, groups=kvd, bias=False)
        self.proj = Linear(hd, dim)
        self.window = window
        self.mu_proj = Linear(H, dim)
        self.v_null = nn.Parameter(torch.zeros(H, dk))
        self.null_base = nn.Parameter(torch.full((H,), NULL_BASE_INIT))
        self.null_slope_raw = nn.Parameter(torch.full((H,), NULL_SLOPE_INIT))
        self.len_gain_raw = nn.Parameter(torch.full((H,), LEN_GAIN_INIT))
        self.mag_beta_raw = nn.Parameter(torch.full((H,), MAG_BETA_INIT))
        self.mem = (TitansMemory(dim, H, dk, chunk=mem_chunk, gamma_bias=mem_gamma_bias,
                                 beta_bias=mem_beta_bias) if mem_enabled else None)
        if overlap not in (True, False, "auto"):
            raise ValueError(f"overlap must be True, False or 'auto' (got {overlap!r})")
        self.overlap = overlap
        self._side = {}
        self._signal = {}

    # ------------------------------------------------------------------ pieces
    def polar_params(self):
        return dict(v_null=self.v_null, null_base=self.null_base, null_slope_raw=self.null_slope_raw,
                    len_gain_raw=self.len_gain_raw, mag_beta_raw=self.mag_beta_raw)

    def polar_params_f32(self):
        """``polar_params`` as the fp32 tensors the kernels read, converted once and kept
        until a parameter changes (its version counter or storage), so that a decode step
        -- and a graph captured from one -- does not convert them per call."""
        ps = self.polar_params()
        key = tuple((p.data_ptr(), p._version, p.dtype) for p in ps.values())
        if getattr(self, "_pf32_key", None) != key:
            self._pf32 = {n: p.detach().to(torch.float32).contiguous() for n, p in ps.items()}
            self._pf32_key = key
        return self._pf32

    def _glue_fusable(self, x):
        """16-bit GPU inference with the memory branch: the per-head glue runs as the
        layer-fusion kernels (``head_rms_norm``, ``global_gate``)."""
        return (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and not torch.is_grad_enabled()
                and self.head_dim in (64, 128) and self.mem is not None)

    def _project(self, x):
        """q/gate, k, v projections and per-head RMSNorm of q, k (``model/reference.py:131-139``).
        x: (..., dim) -> q (..., H, dk), gate (..., H, dk) (a view of the q|gate projection),
        k, v (..., Hkv, dk).  16-bit inference normalises q and k in one pass each, reading
        q in place (``head_rms_norm``; torch's default eps of the compute type, fp32's)."""
        lead = x.shape[:-1]
        H, Hkv, dk = self.num_heads, self.num_kv_heads, self.head_dim
        q, gate = torch.chunk(self.q(x).view(*lead, H, 2 * dk), 2, dim=-1)
        k = self.k(x).view(*lead, Hkv, dk)
        v = self.v(x).view(*lead, Hkv, dk)
        if self._glue_fusable(x):
            return head_rms_norm(q, F32_EPS), gate, head_rms_norm(k, F32_EPS), v
        return F.rms_norm(q, (dk,)), gate, F.rms_norm(k, (dk,)), v

    @staticmethod
    def _conv_prefill(t, conv, tails=None, slots=None, continuing=False):
        """Residual causal depthwise conv over (B, T, C); optionally stores the last K-1
        inputs per sequence (``prefill_causal_conv1d_dense``, ``inference/models/atma.py:148-162``).
        ``continuing``: the left context is the stored tail of each sequence instead of
        zeros (a chunked-prefill continuation, ``inference/models/atma.py:128-130``)."""
        w = conv.weight
        K = w.shape[-1]
        x_in = t.transpose(1, 2)
        if continuing:
            padded = torch.cat([tails[slots].to(t.dtype), x_in], dim=2)
        else:
            padded = F.pad(x_in, (K - 1, 0))
        out = F.conv1d(padded, w.to(t.dtype), groups=x_in.shape[1])
        if tails is not None:
            tails[slots] = padded[:, :, padded.shape[2] - (K - 1):].to(tails.dtype)
        return t + out.transpose(1, 2)

    @staticmethod
    def _conv_packed(t, conv, tails, token_maps):
        """Residual Canon conv over packed fresh sequences in one HIP launch
        (``packed_causal_conv1d``, ``inference/models/atma.py:431-442``): t (tokens, C);
        each sequence's last K-1 inputs go to its row of ``tails``."""
        return t + packed_causal_conv1d(t, conv.weight.squeeze(1), tails, *token_maps)

    @staticmethod
    def dense_token_maps(B, T, slots):
        """Per-token (sequence start, sequence end, table row) of B equal-length fresh
        sequences packed along tokens (the engine's token map, ``inference/engine/
        model_runner.py:390-404``, for the dense batch)."""
        dev = slots.device
        start = torch.arange(B, device=dev, dtype=torch.int32).repeat_interleave(T) * T
        return start, start + T, slots.to(torch.int32).repeat_interleave(T)

    @staticmethod
    def _conv_step(t, conv, tails, slots):
        """Residual conv for one new token per sequence, tails advanced in place
        (``_gpu_conv_step``, ``inference/models/atma.py:165-192``): one fused launch of
        ``causal_conv1d_decode_step`` with the residual add.  t: (B, C)."""
        return causal_conv1d_decode_step(t, conv.weight.squeeze(1), slots, tails, residual=True)

    def _combine(self, c, mag, gate):
        """``proj(c * sigmoid(gate)) + mu_proj(mag)`` (``inference/models/atma.py:246-252``).
        c, gate: (..., H, dk), mag: (..., H)."""
        lead = c.shape[:-2]
        gated = (c * torch.sigmoid(gate)).reshape(*lead, self.num_heads * self.head_dim)
        return self.proj(gated) + self.mu_proj(mag.to(c.dtype))

    def _fused_out(self, x, c, mag, gate, r):
        """The layer's output for 16-bit inference rows, unsummed: ``global_gate`` forms both
        projection inputs in one pass, one GEMM and one GEMM-accumulate give
        ``proj(xa) + mem.proj(xm)`` without biases, and the biases and ``mu_proj(mag)`` ride
        along as a ``PartialSums`` for the residual norm (or ``materialize``).
        x (rows, dim); c (B, T, H, dk) view with rows = B T; mag (rows, H); gate (rows, H, dk)
        view; r (rows, H, dk) fp32."""
        m = self.mem
        xa, xm = global_gate(c, gate, r, m.gate(x), F32_EPS)
        y = F.linear(xa, self.proj.weight.type_as(xa)).addmm_(xm, m.proj.weight.type_as(xm).t())
        return PartialSums(None, [self.proj.bias.type_as(y), m.proj.bias.type_as(y), self.mu_proj.bias.type_as(y)],
                           mu_x=mag.contiguous().to(y.dtype), mu_w=self.mu_proj.weight.type_as(y), dtype=y.dtype,
                           base=y)

    def _side_stream(self, device):
        s = self._side.get(device)
        if s is None:
            s = self._side[device] = torch.cuda.Stream(device=device)  # default priority
            self._signal[device] = StartSignal(device)
        return s

    def _training(self, *inputs):
        """True when autograd must see this call: grad mode is on and an input or a
        parameter of the layer requires grad."""
        return torch.is_grad_enabled() and (any(t.requires_grad for t in inputs)
                                            or any(p.requires_grad for p in self.parameters()))

    def _overlapped(self, B, dtype, device, training=False):
        if self.mem is None or self.overlap is False or device.type != "cuda" or training \
                or torch.cuda.is_current_stream_capturing():
            return False
        return self.overlap is True or recurrence_pays_to_overlap(B, self.num_heads, self.head_dim,
                                                                  dtype, device)

    def _with_memory(self, polar_fn, mem_fn, inputs):
        """Run the Polar part on the current stream and the memory branch (``mem_fn(signal)``)
        in the layer's schedule; return (polar result, memory result)."""
        if self.mem is None:
            return polar_fn(), None
        x = inputs[0]
        if not self._overlapped(x.shape[0], x.dtype, x.device, self._training(*inputs)):
            return polar_fn(), mem_fn(None)
        main = torch.cuda.current_stream(x.device)
        side = self._side_stream(x.device)
        signal = self._signal[x.device]
        signal.arm()
        side.wait_stream(main)
        with torch.cuda.stream(side):
            m = mem_fn(signal)
        signal.wait()          # Polar is dispatched once the recurrence holds its CUs
        p = polar_fn()
        main.wait_stream(side)
        for t in inputs:
            t.record_stream(side)
        for t in (m if isinstance(m, tuple) else (m,)):
            if isinstance(t, torch.Tensor):
                t.record_stream(main)
        return p, m

    # ------------------------------------------------------------------ routes
    def forward(self, x):
        """Causal full-sequence mixer (``model/reference.py:127-195``): x (B, T, dim)."""
        B, T, _ = x.shape
        H, Hkv, dk = self.num_heads, self.num_kv_heads, self.head_dim
        q, gate, k, v = self._project(x)
        q = self._conv_prefill(q.reshape(B, T, H * dk), self.canon_q).view(B, T, H, dk)
        k = self._conv_prefill(k.reshape(B, T, Hkv * dk), self.canon_k).view(B, T, Hkv, dk)
        v = self._conv_prefill(v.reshape(B, T, Hkv * dk), self.canon_v).view(B, T, Hkv, dk)
        return self._attend_prefill(x, q, gate, k, v, None, None)

    def _attend_prefill(self, x, q, gate, k, v, S0, final_sink, defer=False):
        """``defer`` (16-bit inference): return the output as a ``PartialSums`` over B T rows."""
        B, T = q.shape[:2]
        H, dk = self.num_heads, self.head_dim
        n_keys = torch.arange(1, T + 1, device=x.device, dtype=torch.float32)
        qh, kh, vh = (t.transpose(1, 2) for t in (q, k, v))   # (B, heads, T, dk) views
        fused = self._glue_fusable(x)

        # under autograd the differentiable op (HIP forward with saved statistics, HIP
        # backward loops); otherwise the forward-only kernel
        attend = polar_attention if self._training(x, q, k, v) else polar_attention_fwd

        def polar():
            c, mag = attend(qh, kh, vh, n_keys, is_causal=True, window=self.window, **self.polar_params())
            if fused:
                return c, mag
            return self._combine(c.transpose(1, 2), mag.transpose(1, 2), gate)

        def memory(signal):
            fn = self.mem.readout if fused else self.mem
            return fn(x, q, k, v, initial_state=S0, output_final_state=final_sink is not None, start_signal=signal)

        out, m = self._with_memory(polar, memory, (x, q, k, v))
        if m is not None and final_sink is not None:
            final_sink(m[1])
        if fused:
            c, mag = out
            res = self._fused_out(x.reshape(B * T, -1), c.transpose(1, 2), mag.transpose(1, 2).reshape(B * T, H),
                                  gate.reshape(B * T, H, dk), m[0].reshape(B * T, H, dk))
            return res if defer else res.materialize().view(B, T, -1)
        if m is not None:
            out = out + m[0]
        return out

    def prefill(self, x, cache: GlobalLayerCache, slots, slot_mapping, defer=False):
        """Dense fresh prefill of B equal-length sequences (``inference/models/atma.py:397-437``).

        x: (B, T, dim); slots: (B,) int64 rows of the conv / memory tables;
        slot_mapping: (B*T,) int32 cache slots of every token (-1 = skip)."""
        B, T, _ = x.shape
        H, Hkv, dk = self.num_heads, self.num_kv_heads, self.head_dim
        q, gate, k, v = self._project(x)
        maps = self.dense_token_maps(B, T, slots)
        q = self._conv_packed(q.reshape(B * T, H * dk), self.canon_q, cache.conv_q, maps).view(B, T, H, dk)
        k = self._conv_packed(k.reshape(B * T, Hkv * dk), self.canon_k, cache.conv_k, maps).view(B, T, Hkv, dk)
        v = self._conv_packed(v.reshape(B * T, Hkv * dk), self.canon_v, cache.conv_v, maps).view(B, T, Hkv, dk)
        store_kvcache(k.reshape(B * T, Hkv, dk), v.reshape(B * T, Hkv, dk), cache.k_cache, cache.v_cache,
                      slot_mapping)
        S0 = cache.mem_table[slots] if self.mem is not None else None

        def sink(S):
            cache.mem_table[slots] = S

        return self._attend_prefill(x, q, gate, k, v, S0, sink, defer)

    def prefill_packed(self, x, cache: GlobalLayerCache, seq_lens, slots, slot_mapping, tile_maps, token_maps,
                       defer=False):
        """Grouped fresh prefill of ragged prompts packed along tokens
        (``inference/models/atma.py:431-507``): the Canon convs as one packed launch each
        (tails written per sequence), the K/V rows to the pages, ONE tile-mapped Polar
        launch over every sequence (``polar_attention_packed_fwd``, 16-bit inputs), and the
        memory per sequence from its table state.

        x: (tokens, dim) packed in sequence order; seq_lens: the B prompt lengths; slots: (B,)
        int64 table rows; slot_mapping: (tokens,) int32 cache slots; tile_maps: (tile_seq_starts,
        tile_q_starts, tile_seq_lens) int32 (one entry per 128-row query tile); token_maps:
        (token_seq_starts, token_seq_ends, token_seq_slots) int32 (one entry per token)."""
        total = x.shape[0]
        H, Hkv, dk = self.num_heads, self.num_kv_heads, self.head_dim
        q, gate, k, v = self._project(x)
        q = self._conv_packed(q.reshape(total, H * dk), self.canon_q, cache.conv_q, token_maps).view(total, H, dk)
        k = self._conv_packed(k.reshape(total, Hkv * dk), self.canon_k, cache.conv_k, token_maps).view(
            total, Hkv, dk)
        v = self._conv_packed(v.reshape(total, Hkv * dk), self.canon_v, cache.conv_v, token_maps).view(
            total, Hkv, dk)
        store_kvcache(k, v, cache.k_cache, cache.v_cache, slot_mapping)
        c, mag = polar_attention_packed_fwd(q, k, v, *tile_maps, window=self.window, **self.polar_params())
        if self._glue_fusable(x):
            rs, start = [], 0
            for i, n in enumerate(int(t) for t in seq_lens):
                sl = slots[i:i + 1]
                seg = slice(start, start + n)
                r, S = self.mem.readout(x[seg][None], q[seg][None], k[seg][None], v[seg][None],
                                        initial_state=cache.mem_table[sl], output_final_state=True)
                cache.mem_table[sl] = S
                rs.append(r[0])
                start += n
            res = self._fused_out(x, c.view(1, total, H, dk), mag, gate, torch.cat(rs, 0))
            return res if defer else res.materialize()
        out = self._combine(c, mag, gate)
        if self.mem is not None:
            parts, start = [], 0
            for i, n in enumerate(int(t) for t in seq_lens):
                sl = slots[i:i + 1]
                seg = slice(start, start + n)
                r, S = self.mem(x[seg][None], q[seg][None], k[seg][None], v[seg][None],
                                initial_state=cache.mem_table[sl], output_final_state=True)
                cache.mem_table[sl] = S
                parts.append(r[0])
                start += n
            out = out + torch.cat(parts, 0)
        return out

    def prefill_continue(self, x, cache: GlobalLayerCache, slots, slot_mapping, block_tables, cached):
        """Chunked-prefill continuation of B sequences by T tokens each
        (``inference/models/atma.py:509-544``): the Canon convs continue from the stored
        tails, the chunk's K/V go to the pages, each sequence attends over its gathered
        prefix plus the chunk with ``is_causal=False`` and absolute ``n_keys =
        cached + 1 .. cached + T``, and the memory continues from its table state.

        x: (B, T, dim); slots: (B,) int64 table rows; slot_mapping: (B*T,) int32 cache slots
        of the chunk; block_tables: (B, max_pages) int32; cached: B ints (tokens already in
        the pages; 0 makes that sequence a fresh prefill)."""
        B, T, _ = x.shape
        H, Hkv, dk = self.num_heads, self.num_kv_heads, self.head_dim
        cached = [int(c) for c in cached]
        q, gate, k, v = self._project(x)
        q = self._conv_prefill(q.reshape(B, T, H * dk), self.canon_q, cache.conv_q, slots, True).view(B, T, H, dk)
        k = self._conv_prefill(k.reshape(B, T, Hkv * dk), self.canon_k, cache.conv_k, slots, True).view(
            B, T, Hkv, dk)
        v = self._conv_prefill(v.reshape(B, T, Hkv * dk), self.canon_v, cache.conv_v, slots, True).view(
            B, T, Hkv, dk)
        store_kvcache(k.reshape(B * T, Hkv, dk), v.reshape(B * T, Hkv, dk), cache.k_cache, cache.v_cache,
                      slot_mapping)
        page = cache.k_cache.shape[1]
        cs, ms = [], []
        for b in range(B):
            n = cached[b]
            if n > 0:
                pages = block_tables[b, :(n + page - 1) // page].long()
                kp = cache.k_cache[pages].reshape(-1, Hkv, dk)[:n]
                vp = cache.v_cache[pages].reshape(-1, Hkv, dk)[:n]
                kb, vb = torch.cat([kp, k[b]], 0), torch.cat([vp, v[b]], 0)
            else:
                kb, vb = k[b], v[b]
            n_keys = torch.arange(n + 1, n + T + 1, device=x.device, dtype=torch.float32)
            c, mag = polar_attention_fwd(q[b].transpose(0, 1).unsqueeze(0), kb.transpose(0, 1).unsqueeze(0),
                                         vb.transpose(0, 1).unsqueeze(0), n_keys, is_causal=n == 0,
                                         window=self.window, **self.polar_params())
            cs.append(c[0].transpose(0, 1))
            ms.append(mag[0].transpose(0, 1))
        out = self._combine(torch.stack(cs), torch.stack(ms), gate)
        if self.mem is not None:
            r, S = self.mem(x, q, k, v, initial_state=cache.mem_table[slots], output_final_state=True)
            cache.mem_table[slots] = S
            out = out + r
        return out

    def _decode_fusable(self, x, cache, block_tables):
        H, Hkv, dk = self.num_heads, self.num_kv_heads, self.head_dim
        m = self.mem
        if m is None or not decode_rows(x) or dk not in (64, 128) or self.kernel_size > 16 \
                or H * dk not in (256, 512, 1024):
            return False
        outs = [2 * H * dk, Hkv * dk, Hkv * dk, H * dk, H, H]
        if not linear_tokens_multi_supported(x.shape[0], x.shape[1], outs, x.dtype):
            return False
        kc = cache.k_cache
        return bool(kc.dtype == x.dtype and cache.conv_q.dtype == x.dtype and global_decode_step_supported_shape(
            x.shape[0], H, kc.shape[2], block_tables.shape[1], kc.shape[1], dk, x.dtype))

    def _decode_fused(self, x, cache, slots, block_tables, context_lens, slot_mapping):
        """The decode step in seven launches: one projection launch for q|gate, k, v, the
        memory gate and gate logits (``linear_tokens_multi``), the norms / Canon convs /
        gates (``global_decode_prep``), the attention + KV write + memory step
        (``global_decode_step``, two), the gated projection inputs
        (``global_decode_gate``), and both output projections as fp32 partial sums
        (``linear_tokens_chunks``), returned with their biases and ``mu_proj(mag)`` as a
        ``PartialSums`` for the residual norm to add."""
        H, Hkv, dk = self.num_heads, self.num_kv_heads, self.head_dim
        m = self.mem
        hd, kvd = H * dk, Hkv * dk
        lin = (self.q, self.k, self.v, m.gate, m.w_gamma, m.w_beta)
        y = linear_tokens_multi(x, [l.weight for l in lin], [l.bias for l in lin])
        ck, cv = 2 * hd, 2 * hd + kvd
        cm = cv + kvd
        cg = cm + hd
        taps = tuple(c.weight.squeeze(1) for c in (self.canon_q, self.canon_k, self.canon_v))
        q, k, v, gamma, beta = global_decode_prep(y, H, Hkv, dk, (ck, cv, cg, cg + H), taps,
                                                  (cache.conv_q, cache.conv_k, cache.conv_v), slots, F32_EPS,
                                                  gate_bias=(m.gamma_bias, m.beta_bias))
        c, mag, r = global_decode_step(q, k, v, cache.k_cache, cache.v_cache, slot_mapping, block_tables,
                                       context_lens, gamma, beta, cache.mem_table, slots, window=self.window,
                                       **self.polar_params_f32())
        x2 = global_decode_gate(c, r, y, cm, F32_EPS)
        parts = linear_tokens_chunks(x2, [self.proj.weight, m.proj.weight], hd)
        return PartialSums(parts, [self.proj.bias, m.proj.bias, self.mu_proj.bias], mu_x=mag,
                           mu_w=self.mu_proj.weight, dtype=x.dtype)

    def decode(self, x, cache: GlobalLayerCache, slots, block_tables, context_lens, slot_mapping, defer=False):
        """One token per sequence (``inference/models/atma.py:546-618``).

        x: (B, dim); slots: (B,) int64 table rows; block_tables: (B, max_pages) int32;
        context_lens: (B,) int32 including this token; slot_mapping: (B,) int32.
        16-bit decode rows with the memory branch run fused (``_decode_fused``); ``defer``
        then returns its ``PartialSums`` unsummed."""
        if self._decode_fusable(x, cache, block_tables):
            out = self._decode_fused(x, cache, slots, block_tables, context_lens, slot_mapping)
            return out if defer else out.materialize()
        H, Hkv, dk = self.num_heads, self.num_kv_heads, self.head_dim
        Bn = x.shape[0]
        q, gate, k, v = self._project(x)
        q = self._conv_step(q.reshape(Bn, H * dk), self.canon_q, cache.conv_q, slots).view(Bn, H, dk)
        k = self._conv_step(k.reshape(Bn, Hkv * dk), self.canon_k, cache.conv_k, slots).view(Bn, Hkv, dk)
        v = self._conv_step(v.reshape(Bn, Hkv * dk), self.canon_v, cache.conv_v, slots).view(Bn, Hkv, dk)
        if self.mem is not None:
            # the KV write, the attention and the memory step as one fused call (two
            # launches where the shapes allow it: the memory step runs in the attention's
            # merge launch, and the newest key joins from k / v)
            gamma, beta = self.mem.decode_gates(x)
            c, mag, r = global_decode_step(q, k, v, cache.k_cache, cache.v_cache, slot_mapping,
                                           block_tables, context_lens, gamma, beta, cache.mem_table,
                                           slots, window=self.window, **self.polar_params_f32())
            return self._combine(c, mag, gate) + self.mem._out(x, r)
        store_kvcache(k, v, cache.k_cache, cache.v_cache, slot_mapping)
        c, mag = polar_attention_decode(q, cache.k_cache, cache.v_cache, block_tables, context_lens,
                                        window=self.window, **self.polar_params_f32())
        return self._combine(c, mag, gate)


class RMSNorm(nn.Module):
    """``model/layers.py:6-16``."""

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        return F.rms_norm(x, (x.size(-1),), weight=self.weight.type_as(x), eps=self.eps)

    def add_norm(self, branch, residual):
        """The pre-norm block's residual step: ``s = residual + branch`` (``residual`` None:
        the branch starts the stream), returns ``(self(s), s)``.  On 16-bit GPU rows outside
        autograd one HIP launch (``residual_rms_norm``), which also takes a branch still in
        fp32 partial sums (``PartialSums``); otherwise the eager add and norm."""
        w = self.weight.to(branch.dtype)
        if not torch.is_grad_enabled() and residual_rms_norm_supported(w):
            return residual_rms_norm(branch, residual, w, self.eps)
        if isinstance(branch, PartialSums):
            branch = branch.materialize()
        s = branch if residual is None else residual + branch
        return self(s), s


class MLP(nn.Module):
    """Squared-ReLU gated MLP (``model/layers.py:19-31``)."""

    def __init__(self, dim):
        super().__init__()
        self.fc = Linear(dim, 8 * dim)
        self.proj = Linear(4 * dim, dim)

    def forward(self, x, defer=False):
        """``defer`` (decode rows only): the activation is formed in the first projection's
        epilogue (``linear_tokens_gated``) and the down projection returned as fp32 partial
        sums (``PartialSums``, K split over 4x the workgroups) for the next
        ``RMSNorm.add_norm`` to finish."""
        if defer and decode_rows(x):
            dim, hidden = self.proj.weight.shape
            ck = chunk_width(hidden)
            if ck is not None and linear_tokens_supported(x.shape[0], self.fc.weight.shape[0], x.shape[1], x.dtype):
                h = linear_tokens_gated(x, self.fc.weight, self.fc.bias)
                w = self.proj.weight
                parts = linear_tokens_chunks(h, [w[:, c * ck:(c + 1) * ck] for c in range(hidden // ck)], ck)
                return PartialSums(parts, [self.proj.bias], dtype=x.dtype)
        if x.is_cuda and not torch.is_grad_enabled() and x.is_contiguous() and self.fc.weight.dtype == x.dtype:
            rows, K = x.numel() // x.shape[-1], x.shape[-1]
            if linear_gated_supported(rows, K, self.fc.weight.shape[0], x.dtype):
                # many rows (a prefill): the projection and its activation in one MFMA kernel
                # that never writes the 8 dim-wide projection (linear_gated)
                h = linear_gated(x.view(rows, K), self.fc.weight, self.fc.bias)
                return self.proj(h.view(*x.shape[:-1], -1))
        a, gate = torch.chunk(self.fc(x), 2, dim=-1)
        if x.is_cuda and not torch.is_grad_enabled():
            # InferenceMLP (inference/models/atma.py:87-96): the fused HIP activation,
            # equal to the eager form bit for bit (bf16 rounds the square as eager does)
            lead = a.shape[:-1]
            h = squared_relu_gate(a.reshape(-1, a.shape[-1]), gate.reshape(-1, gate.shape[-1]))
            return self.proj(h.view(*lead, -1))
        return self.proj(gate * a.relu().square())


class GlobalBlock(nn.Module):
    """Pre-norm global block (``model/reference.py:198-229`` with attention=True):
    ``x + attn(norm1 x)``, then ``x + mlp(norm2 x)``."""

    def __init__(self, dim, head_dim=128, num_kv_heads=None, attn_kernel_size=4, window=None,
                 mem_enabled=True, mem_chunk=64, overlap="auto"):
        super().__init__()
        self.attn = PolarAttention(dim, head_dim=head_dim, num_kv_heads=num_kv_heads,
                                   kernel_size=attn_kernel_size, window=window, mem_enabled=mem_enabled,
                                   mem_chunk=mem_chunk, overlap=overlap)
        self.mlp = MLP(dim)
        self.norm1 = RMSNorm(dim)
        self.norm2 = RMSNorm(dim)

    def forward(self, x):
        x = x + self.attn(self.norm1(x))
        return x + self.mlp(self.norm2(x))

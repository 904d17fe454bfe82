"""Benchmark of ATMA's global-layer mixer on one MI355X.

Default workload (the `value`): BASELINE.json configs[2] at T=65,536 -- the north-star
long-context prefill, bf16, B=1, 8 query / 2 KV heads, d=128: Polar attention forward
(GQA in-kernel) plus the gated-delta chunked prefill (C=64, fp32 state from zero, memory
gate / beta logits activated inside the prefill kernel's load as the layer does:
logsigmoid(z + 3.9), sigmoid(z)).  One step = both ops over the resident sequence in the
global layer's schedule for the shape: back to back on one stream, or -- when the
recurrence kernel's grid takes at most a quarter of the CUs, as at B=1, T=65,536 -- the
memory branch on a second stream with Polar launched once the recurrence has started
(both schedules are reported: ms_sequential, ms_overlap).
value = (Polar + gated-delta algorithmic FLOPs) / step time; `roofline` is the Polar
kernel alone at that shape (HIP events on its stream).

Also reported in the same JSON line: configs[1] (B=8, T=2,048, `breakdown_c2`),
configs[2] at T=262,144 (`prefill_long`), configs[3] (paged decode step: 64 sequences,
ctx ~ U[1024, 32768], 256-token pages in a shuffled pool: the layer's fused decode route
-- KV write + Polar decode + gated-delta step in two launches -- replayed as a HIP
graph; the three separate calls timed beside it), each with its roofline fraction;
configs[4] (the 378M model served through the paged engine, 32 x 2,048-token prompts ->
256 greedy tokens: prefill / decode tok/s and wall time); configs[0] (one global block
in fp32 on the GPU); the training steps of the layer's two branches at the configs[1]
shape (Polar and the gated-delta memory, forward + backward); plus the CPU oracle timed
on this host (configs[2] extrapolated from a row / token sample, and configs[0] exact).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c1|c2|c3|c4|c5|ops|train|copy|cpu] [--no-cpu]
"""

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
METRIC = "Polar+GDN prefill TFLOP/s & MFMA%; paged decode tok/s & HBM GB/s (1 GPU)"
HQ, HKV, D, CHUNK = 8, 2, 128, 64


def polar_flops(B, T):
    return float(B) * HQ * 2 * D * T * (T + 1)


def gdn_flops(B, T):
    return float(B) * T * HQ * (6 * D * D + 4 * CHUNK * D)


def _params(torch, dev, seed=0):
    """Polar parameters at the reference priors (model/reference.py:17-20)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    return dict(v_null=(torch.randn(HQ, D, generator=g) * 0.02).to(dev),
                null_base=torch.full((HQ,), 2.0, device=dev),
                null_slope_raw=torch.full((HQ,), 0.5, device=dev),
                len_gain_raw=torch.full((HQ,), -1.0, device=dev),
                mag_beta_raw=torch.full((HQ,), -1.5, device=dev))


class Prefill:
    """Resident inputs and one step of the prefill hot path."""

    def __init__(self, torch, dev, B, T, seed=0):
        from atma_amd.kernel import (StartSignal, chunk_gated_delta_rule, polar_attention_fwd,
                                     recurrence_pays_to_overlap)
        self.torch, self.B, self.T = torch, B, T
        self.fwd, self.gdn = polar_attention_fwd, chunk_gated_delta_rule
        g = torch.Generator(device=dev).manual_seed(seed)
        bf = torch.bfloat16
        self.q = torch.randn(B, HQ, T, D, device=dev, generator=g, dtype=bf)
        self.k = torch.randn(B, HKV, T, D, device=dev, generator=g, dtype=bf)
        self.v = torch.randn(B, HKV, T, D, device=dev, generator=g, dtype=bf)
        # the memory branch takes (B, T, heads, d) views of the same tensors; its kernels
        # map query head h to KV head h // (HQ // HKV), so nothing is expanded
        self.qm = self.q.transpose(1, 2)
        self.km = self.k.transpose(1, 2)
        self.vm = self.v.transpose(1, 2)
        self.zg = torch.randn(B, T, HQ, device=dev, generator=g)
        self.zb = torch.randn(B, T, HQ, device=dev, generator=g)
        self.s0 = torch.zeros(B, HQ, D, D, device=dev)
        self.n_keys = torch.arange(1, T + 1, device=dev, dtype=torch.float32)
        self.p = _params(torch, dev, seed)
        self.side = torch.cuda.Stream(device=dev)  # default priority
        self.signal = StartSignal(dev)
        # the global layer's schedule for this shape (PolarAttention(overlap="auto"))
        self.overlap = recurrence_pays_to_overlap(B, HQ, D, torch.bfloat16, dev)

    def polar(self):
        return self.fwd(self.q, self.k, self.v, self.n_keys, **self.p)

    def memory(self, signal=None):
        # raw gate logits: the layer's activations (logsigmoid(z + 3.9), sigmoid(z)) are
        # applied inside the prefill kernel's load, as TitansMemory does
        return self.gdn(self.qm, self.km, self.vm, self.zg, self.zb, scale=1.0, initial_state=self.s0,
                        output_final_state=True, use_qk_l2norm_in_kernel=True, gate_bias=(3.9, 0.0),
                        start_signal=signal)

    def step(self):
        """One mixer step in the global layer's schedule for this shape."""
        return self.step_overlap() if self.overlap else self.step_sequential()

    def step_sequential(self):
        """Both ops back to back on one stream.  Returns (c, mag), (o, final state)."""
        return self.polar(), self.memory()

    def step_overlap(self):
        """The memory branch on a second stream; Polar's launch waits (one-wave kernel) until
        the recurrence's workgroups have started, then runs beside it."""
        torch = self.torch
        main = torch.cuda.current_stream()
        self.signal.arm()
        self.side.wait_stream(main)
        with torch.cuda.stream(self.side):
            mem = self.memory(self.signal)
        self.signal.wait()
        out = self.polar()
        main.wait_stream(self.side)
        for t in mem:                      # made on the side stream, read on this one
            t.record_stream(main)
        return out, mem

    def flops(self):
        return polar_flops(self.B, self.T), gdn_flops(self.B, self.T)


def _time(torch, fn, steps, warmup):
    """Average ms per call of fn over `steps` calls, HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def bench_prefill(torch, dev, B, T, steps, warmup):
    w = Prefill(torch, dev, B, T)
    fp, fg = w.flops()
    # about 60 ms of steps first, so every timed leg runs at the GPU's steady clocks;
    # then the component legs, then the step in the layer's schedule: `warmup` untimed
    # steps and `steps` timed ones
    one = _time(torch, w.step, 1, 1)
    _time(torch, w.step, max(1, int(60.0 / max(one, 1e-3))), 0)
    ms_polar = _time(torch, w.polar, steps, max(1, warmup // 2))
    ms_gdn = _time(torch, w.memory, steps, max(1, warmup // 2))
    ms_seq = _time(torch, w.step_sequential, steps, max(1, warmup // 2))
    ms_ovl = _time(torch, w.step_overlap, steps, max(1, warmup // 2))
    ms_step = _time(torch, w.step, steps, warmup)
    res = dict(B=B, T=T, ms_per_step=ms_step, tflops=(fp + fg) / (ms_step * 1e-3) / 1e12,
               schedule="overlap" if w.overlap else "sequential",
               ms_sequential=ms_seq, ms_overlap=ms_ovl,
               polar_ms=ms_polar, polar_tflops=fp / (ms_polar * 1e-3) / 1e12,
               gdn_ms=ms_gdn, gdn_tflops=fg / (ms_gdn * 1e-3) / 1e12,
               polar_flops=fp, gdn_flops=fg)
    res["mfma_frac"] = res["tflops"] / PEAK_BF16_TFLOPS
    res["polar_mfma_frac"] = res["polar_tflops"] / PEAK_BF16_TFLOPS
    del w
    torch.cuda.empty_cache()
    return res


class Decode:
    """one paged decode step for 64 sequences."""

    def __init__(self, torch, dev, seed=0, B=64, ctx_lo=1024, ctx_hi=32768, page=256, full=False):
        from atma_amd.kernel import gated_delta_decode_step, global_decode_step, polar_attention_decode
        from atma_amd.layers.attention import store_kvcache
        self.torch = torch
        self.dec, self.step_mem, self.store = polar_attention_decode, gated_delta_decode_step, store_kvcache
        self.fused = global_decode_step
        gc = torch.Generator().manual_seed(seed)
        ctx = (torch.full((B,), ctx_hi) if full else torch.randint(ctx_lo, ctx_hi + 1, (B,), generator=gc))
        npg = (ctx + page - 1) // page
        pool = int(npg.sum())
        perm = torch.randperm(pool, generator=gc).int()
        maxp = (ctx_hi + page - 1) // page
        bt = torch.zeros((B, maxp), dtype=torch.int32)
        used = 0
        for b in range(B):
            bt[b, :npg[b]] = perm[used:used + npg[b]]
            used += int(npg[b])
        slot_map = torch.tensor([int(bt[b, (int(ctx[b]) - 1) // page]) * page + (int(ctx[b]) - 1) % page
                                 for b in range(B)], dtype=torch.int32)
        g = torch.Generator(device=dev).manual_seed(seed)
        bf = torch.bfloat16
        self.kc = torch.randn(pool, page, HKV, D, device=dev, generator=g, dtype=bf)
        self.vc = torch.randn(pool, page, HKV, D, device=dev, generator=g, dtype=bf)
        self.q = torch.randn(B, HQ, D, device=dev, generator=g, dtype=bf)
        self.knew = torch.randn(B, HKV, D, device=dev, generator=g, dtype=bf)
        self.vnew = torch.randn(B, HKV, D, device=dev, generator=g, dtype=bf)
        self.gamma = torch.sigmoid(torch.randn(B, HQ, device=dev, generator=g) + 3.9)
        self.beta = torch.sigmoid(torch.randn(B, HQ, device=dev, generator=g))
        max_seqs = 2 * B
        self.table = torch.randn(max_seqs, HQ, D, D, device=dev, generator=g) * 0.1
        self.slots = torch.randperm(max_seqs, generator=gc)[:B].to(dev)
        self.bt, self.ctx, self.slot_map = bt.to(dev), ctx.int().to(dev), slot_map.to(dev)
        self.p = _params(torch, dev, seed)
        self.B, self.pages = B, pool
        self.ctx_sum = int(ctx.sum())
        self.graph = None

    def step(self):
        """The global layer's decode route: KV write + attention + memory step, fused
        (two launches)."""
        return self.fused(self.q, self.knew, self.vnew, self.kc, self.vc, self.slot_map, self.bt, self.ctx,
                          self.gamma, self.beta, self.table, self.slots, **self.p)

    def step_separate(self):
        """The same step as the reference's three calls."""
        self.store(self.knew, self.vnew, self.kc, self.vc, self.slot_map)
        c, mag = self.dec(self.q, self.kc, self.vc, self.bt, self.ctx, **self.p)
        r = self.step_mem(self.q, self.knew, self.vnew, self.gamma, self.beta, self.table, self.slots)
        return c, mag, r

    def attention(self):
        return self.dec(self.q, self.kc, self.vc, self.bt, self.ctx, **self.p)

    def capture(self):
        torch = self.torch
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                self.step()
        torch.cuda.current_stream().wait_stream(s)
        # two captures of the same step, replayed in turn: relaunching one graph exec
        # right behind itself waits for its previous launch to retire (about 8 us per
        # step on this runtime); alternating two execs keeps the queue fed, as the
        # engine's graph runner does
        self.graphs, self.outs = [], []
        for _ in range(2):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.outs.append(self.step())   # (c, mag, r) of this exec: rewritten by its replays
            self.graphs.append(g)
        self.graph = self.graphs[0]
        self.graph_out = self.outs[0]
        self.flip = 0

    def replay(self):
        """Replay the next exec; graph_out is then its (c, mag, r)."""
        self.graphs[self.flip].replay()
        self.graph_out = self.outs[self.flip]
        self.flip ^= 1

    def replay_one(self):
        self.graph.replay()
        self.graph_out = self.outs[0]

    def bytes(self):
        kv = self.ctx_sum * HKV * D * 2 * 2
        state = self.B * HQ * D * D * 4 * 2
        small = (self.B * HQ * D * 2 * 2            # q read by attention and memory
                 + self.B * HQ * D * 2 + self.B * HQ * 2 + self.B * HQ * D * 4   # c, mag, r
                 + self.B * HKV * D * 2 * 2 * 3     # new k/v: store read + write, memory read
                 + 4 * self.pages + 4 * self.B * 3)  # page table, ctx, slots
        return kv, state, small


def bench_decode(torch, dev, steps, warmup, full=False):
    w = Decode(torch, dev, full=full)
    w.capture()
    # bring the GPU to its steady clocks before the first timed leg: about 60 ms of steps
    # (with 8 ms, the first timed leg still ran 3-5% slow while the clocks ramped)
    one = _time(torch, w.replay, 1, 1)
    _time(torch, w.replay, max(40, int(60.0 / max(one, 1e-3))), 0)
    ms_graph = _time(torch, w.replay, steps, warmup)
    ms_one = _time(torch, w.replay_one, steps, warmup)
    ms_eager = _time(torch, w.step, steps, warmup)
    ms_sep = _time(torch, w.step_separate, steps, warmup)
    ms_attn = _time(torch, w.attention, steps, warmup)
    kv, state, small = w.bytes()
    total = kv + state + small
    res = dict(B=w.B, ctx_sum=w.ctx_sum, pages=w.pages, ms_per_step=ms_graph, ms_eager=ms_eager,
               ms_one_graph_exec=ms_one, ms_separate_calls_eager=ms_sep,
               tok_per_s=w.B / (ms_graph * 1e-3), bytes=total, gbs=total / (ms_graph * 1e-3) / 1e9,
               attn_ms=ms_attn, attn_bytes=kv, attn_gbs=kv / (ms_attn * 1e-3) / 1e9)
    res["hbm_frac"] = res["gbs"] / PEAK_HBM_GBS
    res["attn_hbm_frac"] = res["attn_gbs"] / PEAK_HBM_GBS
    del w
    torch.cuda.empty_cache()
    return res


def bench_inference_ops(torch, dev, steps, warmup):
    """The inference fusions at configs[4] shapes (hidden 1024, MLP 4x, vocab 50,304,
    32 prompts x 2,048 tokens), bf16, each as achieved HBM GB/s of its compulsory bytes:
    squared_relu_gate over one prefill step's MLP activations (65,536 x 4,096: read x and
    gate, write out), softcap_logits over one decode step's logits (32 x 50,304 read +
    written), packed_causal_conv1d over the packed prefill's q projection (65,536 tokens x
    1,024 channels, K = 4: read x, write out)."""
    from atma_amd.kernel import packed_causal_conv1d, softcap_logits, squared_relu_gate
    g = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    res = {}
    fc = torch.randn(65536, 8192, device=dev, generator=g, dtype=bf)
    a, gate = fc.chunk(2, dim=-1)
    ms = _time(torch, lambda: squared_relu_gate(a, gate), steps, warmup)
    res["squared_relu_gate"] = dict(shape=[65536, 4096], ms=ms, gbs=3 * a.numel() * 2 / (ms * 1e-3) / 1e9)
    del fc, a, gate
    logits = torch.randn(32, 50304, device=dev, generator=g, dtype=bf)
    ms = _time(torch, lambda: softcap_logits(logits), steps, warmup)
    res["softcap_logits"] = dict(shape=[32, 50304], ms=ms, gbs=2 * logits.numel() * 2 / (ms * 1e-3) / 1e9)
    T, C, S = 65536, 1024, 32
    x = torch.randn(T, C, device=dev, generator=g, dtype=bf)
    w = torch.randn(C, 4, device=dev, generator=g, dtype=bf)
    table = torch.zeros(S, C, 3, device=dev, dtype=bf)
    seq = torch.arange(T, device=dev, dtype=torch.int32) // (T // S)
    starts, ends = seq * (T // S), (seq + 1) * (T // S)
    ms = _time(torch, lambda: packed_causal_conv1d(x, w, table, starts, ends, seq), steps, warmup)
    res["packed_causal_conv1d"] = dict(shape=[T, C], ms=ms, gbs=(2 * x.numel() * 2 + 3 * T * 4) / (ms * 1e-3) / 1e9)
    for r in res.values():
        r["hbm_frac"] = r["gbs"] / PEAK_HBM_GBS
    del x, table
    torch.cuda.empty_cache()
    return res


def bench_train(torch, dev, steps, warmup):
    """Training steps of the global layer's two branches at the configs[1] shape (B=8,
    T=2048, 8 / 2 heads, d=128, bf16), each forward + backward (the gradients of every
    input and parameter), timed with HIP events.

    Memory branch: chunk_gated_delta_rule on raw q / k (l2 norm in-kernel), log decay and
    beta leaves: the 16-bit chunked forward, then the chunked (WY) backward's three
    launches.  Polar: polar_attention forward with saved statistics, then the backward
    (preamble, dq and dk / dv loops, parameter sums); its matmul FLOPs are the forward's
    plus the backward's 7 products of 2 d per causal pair (polar_bwd_flops), and the
    backward alone is the step minus the forward with statistics."""
    from atma_amd.kernel import chunk_gated_delta_rule
    from atma_amd.kernel.polar_train import polar_attention, polar_bwd_flops
    B, T = 8, 2048
    g = torch.Generator(device=dev).manual_seed(0)
    bf = dict(device=dev, dtype=torch.bfloat16)
    q, k, v = (torch.randn(B, T, HQ, D, generator=g, **bf).requires_grad_(True) for _ in range(3))
    gl = torch.nn.functional.logsigmoid(torch.randn(B, T, HQ, device=dev, generator=g) + 3.9).requires_grad_(True)
    beta = torch.sigmoid(torch.randn(B, T, HQ, device=dev, generator=g)).requires_grad_(True)
    dO = torch.randn(B, T, HQ, D, generator=g, **bf)

    def mem_step():
        o, _ = chunk_gated_delta_rule(q, k, v, gl, beta, scale=1.0, use_qk_l2norm_in_kernel=True)
        torch.autograd.grad(o, (q, k, v, gl, beta), dO)

    pq = torch.randn(B, HQ, T, D, generator=g, **bf).requires_grad_(True)
    pk, pv = (torch.randn(B, HKV, T, D, generator=g, **bf).requires_grad_(True) for _ in range(2))
    prm = {n: t.clone().requires_grad_(True) for n, t in _params(torch, dev).items()}
    n_keys = torch.arange(1, T + 1, device=dev, dtype=torch.float32)
    dc = torch.randn(B, HQ, T, D, generator=g, **bf)
    dm = torch.randn(B, HQ, T, generator=g, **bf)

    def polar_step():
        c, mag = polar_attention(pq, pk, pv, n_keys, is_causal=True, **prm)
        torch.autograd.grad((c, mag), (pq, pk, pv, *prm.values()), (dc, dm))

    def polar_fwd():
        with torch.no_grad():
            p = [t.detach() for t in prm.values()]
            torch.ops.atma_hip.polar_attention_fwd_train(pq.detach(), pk.detach(), pv.detach(), n_keys, *p,
                                                         1e-6, True, 0, False)

    _time(torch, mem_step, 10, 2)
    ms_mem = _time(torch, mem_step, steps, warmup)
    _time(torch, polar_step, 5, 1)
    ms_polar = _time(torch, polar_step, steps, warmup)
    ms_pfwd = _time(torch, polar_fwd, steps, warmup)
    f_fwd = 4.0 * B * HQ * D * T * (T + 1) / 2.0
    f_bwd = float(polar_bwd_flops(B, HQ, T, D))
    ms_pbwd = ms_polar - ms_pfwd
    return dict(B=B, T=T, memory_ms_fwd_bwd=ms_mem, polar_ms_fwd_bwd=ms_polar, polar_ms_fwd=ms_pfwd,
                polar_ms_bwd=ms_pbwd, polar_bwd_tflops=f_bwd / ms_pbwd / 1e9,
                polar_bwd_mfma_frac=f_bwd / ms_pbwd / 1e9 / PEAK_BF16_TFLOPS,
                polar_step_tflops=(f_fwd + f_bwd) / ms_polar / 1e9)


def c1_state(torch, seed=0):
    """one global block, hidden 1,024, 8 / 2 heads, d = 128, no window, memory
    chunk 64; every parameter N(0, 0.02) from seed 0 (the reference's test convention,
    tests/test_dense_prefill.py:105-106); input (1, 2048, 1024) N(0, 1) from seed 0.
    Returns (the block module on the CPU, x)."""
    from atma_amd.layers.global_attention import GlobalBlock
    torch.manual_seed(seed)
    blk = GlobalBlock(1024, head_dim=128, mem_chunk=CHUNK)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0.0, 0.02)
    x = torch.randn(1, 2048, 1024, generator=torch.Generator().manual_seed(seed))
    return blk, x


def _median_runs(fn, budget_s, min_runs=3, max_runs=10):
    """1 warm-up, then timed runs until min_runs and the time budget are both spent."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_c1(torch):
    """BASELINE configs[0] on the host CPU: the oracle's global block (oracle/block.py, the
    restatement of model/reference.py:127-233) in fp32 -- the mixer alone (Polar +
    memory) and the whole block (+ norms, MLP) -- as tokens/s (median of >= 3 runs)."""
    from oracle import block as OB
    blk, x = c1_state(torch)
    sd = {k: v.detach().clone() for k, v in blk.state_dict().items()}
    attn_sd = {k[5:]: v for k, v in sd.items() if k.startswith("attn.")}
    xn = OB.rms_norm_weighted(x, sd["norm1.weight"])
    T = x.shape[1]
    with torch.no_grad():
        s_mix, n_mix = _median_runs(lambda: OB.polar_attention(attn_sd, xn, H=HQ, Hkv=HKV, dk=D), 8.0)
        s_blk, n_blk = _median_runs(lambda: OB.global_block(sd, x, H=HQ, Hkv=HKV, dk=D), 8.0)
    return {"mixer_tok_s": T / s_mix, "mixer_ms": s_mix * 1e3, "mixer_runs": n_mix,
            "block_tok_s": T / s_blk, "block_ms": s_blk * 1e3, "block_runs": n_blk}


def bench_c1_gpu(torch, dev, steps, warmup):
    """configs[0] on the GPU, fp32 (the 1e-4 parity mode): the same block and input as
    cpu_c1, forward only (the HIP kernels for Polar and the memory, eager glue), as
    tokens/s for the mixer and the block."""
    blk, x = c1_state(torch)
    blk = blk.to(dev)
    x = x.to(dev)
    xn = blk.norm1(x)
    T = x.shape[1]
    with torch.no_grad():
        ms_mix = _time(torch, lambda: blk.attn(xn), steps, warmup)
        ms_blk = _time(torch, lambda: blk(x), steps, warmup)
    return {"mixer_tok_s": T / (ms_mix * 1e-3), "mixer_ms": ms_mix, "block_tok_s": T / (ms_blk * 1e-3),
            "block_ms": ms_blk, "dtype": "fp32"}


def bench_c5(torch, dev, n_prompts=32, prompt_len=2048, new_tokens=256, seed=0):
    """the 378M ATMA (16 blocks, hidden 1,024, vocab 50,304; every
    parameter N(0, 0.02) from seed 0; bf16) served through the paged engine: 32 prompts of
    2,048 uniform random token ids (seed 0) -> 256 greedy tokens each, ignore_eos.  The
    prompts prefill as one dense batch; decode replays the captured HIP graph.  Prefill and
    decode tok/s are the engine's own (HIP events around each step, as the reference's
    LLMEngine.generate); wall_s is the whole timed generate.  A short untimed generate on
    the same prompts runs first (kernel and library warm-up at the full prefill shape).
    decode_ms_per_step is the served step (host scheduling, input staging, the graph, the
    token sync); decode_graph_ms the graph alone; decode_hbm_frac each over 8 TB/s for the
    step's algorithmic bytes (``_c5_decode_bytes`` at the run's mean context)."""
    from atma_amd.engine import AtmaConfig, Config, LLMEngine, SamplingParams
    pages = (prompt_len + new_tokens + 255) // 256
    cfg = Config(kvcache_block_size=256, max_num_seqs=n_prompts, max_num_batched_tokens=n_prompts * prompt_len,
                 max_model_len=prompt_len + new_tokens, num_kvcache_blocks=n_prompts * pages + 8,
                 init_std=0.02, seed=seed, hf_config=AtmaConfig())
    t0 = time.perf_counter()
    engine = LLMEngine(cfg)
    t_init = time.perf_counter() - t0
    g = torch.Generator().manual_seed(seed)
    prompts = torch.randint(0, cfg.hf_config.vocab_size, (n_prompts, prompt_len), generator=g).tolist()
    engine.generate(prompts, SamplingParams(temperature=0.0, max_tokens=2, ignore_eos=True))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    res = engine.generate(prompts, SamplingParams(temperature=0.0, max_tokens=new_tokens, ignore_eos=True))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    m = engine.last_metrics
    mr = engine.model_runner
    n_params = sum(p.numel() for p in mr.model.parameters())
    assert all(len(r["token_ids"]) == new_tokens for r in res)
    # the device time of one decode step alone: the bucket-32 graph (model, LM head,
    # greedy pick) replayed back to back on the last step's inputs (every request has
    # finished: the replays write only into freed pages and table rows)
    graph = mr.graphs[n_prompts][0]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    graph.replay()
    e0.record()
    for _ in range(20):
        graph.replay()
    e1.record()
    e1.synchronize()
    graph_ms = e0.elapsed_time(e1) / 20
    engine.exit()
    del engine
    torch.cuda.empty_cache()
    step_ms = m["decode_time"] * 1e3 / max(1, m["decode_tokens"] // n_prompts)
    step_bytes = _c5_decode_bytes(cfg.hf_config, n_params, n_prompts, prompt_len + (new_tokens + 1) / 2)
    return {"model_params": n_params, "requests": n_prompts, "prompt_len": prompt_len, "new_tokens": new_tokens,
            "prefill_tok_s": m["prefill_throughput"], "decode_tok_s": m["decode_throughput"],
            "prefill_ms": m["prefill_time"] * 1e3, "decode_ms_per_step": step_ms,
            "decode_graph_ms": graph_ms, "decode_bytes_per_step": step_bytes,
            "decode_hbm_frac": step_bytes / (step_ms * 1e-3) / 8e12,
            "decode_graph_hbm_frac": step_bytes / (graph_ms * 1e-3) / 8e12,
            "wall_s": wall, "init_s": t_init,
            "prefill_tokens": m["prefill_tokens"], "decode_tokens": m["decode_tokens"]}


def _c5_decode_bytes(hf, n_params, n_seqs, avg_context):
    """Algorithmic HBM bytes of one decode step of the served model: every weight but the
    embedding table once (16-bit), each sequence's KV cache over its context once in every
    global layer, and the memory state read and written (fp32) -- the conv tails, token
    rows and activations are below 0.1% of it and left out."""
    item = 2
    n_global = sum(hf.is_attention_layer(i) for i in range(hf.num_hidden_layers))
    weights = (n_params - hf.vocab_size * hf.hidden_size) * item
    kv = n_seqs * avg_context * hf.num_key_value_heads * hf.head_dim * 2 * item * n_global
    mem = n_seqs * hf.num_attention_heads * hf.head_dim * hf.head_dim * 4 * 2 * n_global if hf.mem_enabled else 0
    return int(weights + kv + mem)


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline(torch, T=65536, row_stride=256, gdn_tokens=8192):
    """The CPU oracle (oracle/, fp32 torch on this host's cores) on the headline workload,
    configs[2] (B=1, T=65,536, 8/2 heads, d=128), timed on a bounded sample and
    EXTRAPOLATED to the full step (the full step would take tens of minutes on the CPU):

    * Polar: the exact row oracle (oracle/polar.polar_rows, the streaming form) on the query
      rows row_stride - 1, 2 row_stride - 1, ..., T - 1 of all 8 heads, each against all of
      its causal keys; scaled by the causal (query, key) pairs of the full sequence,
      T (T + 1) / 2, over the sampled rows' counts (the cost is linear in those pairs);
    * gated delta: oracle chunk_gated_delta_rule (the chunked UT form) over the first
      gdn_tokens tokens, scaled by T / gdn_tokens (the chunked scan is linear in T).

    value = (Polar + gated-delta algorithmic FLOPs at T) / the extrapolated time.  Inputs are
    seeded N(0, 1) like the GPU workload; median of up to 5 runs within about 20 s.  Also
    reports configs[0] (one global block, exact, no extrapolation) under "c1"."""
    from oracle import gated_delta as OG
    from oracle import polar as OP
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, HQ, T, D, generator=g)
    k = torch.randn(1, HKV, T, D, generator=g)
    v = torch.randn(1, HKV, T, D, generator=g)
    zg, zb = torch.randn(1, gdn_tokens, HQ, generator=g), torch.randn(1, gdn_tokens, HQ, generator=g)
    p = {n: t.cpu() for n, t in _params(torch, "cpu").items()}
    n = torch.arange(1, T + 1, dtype=torch.float32)
    rows = torch.arange(row_stride - 1, T, row_stride)
    pair_scale = (T * (T + 1) / 2) / float((rows + 1).sum())
    tok_scale = T / gdn_tokens
    qg = q[:, :, :gdn_tokens].transpose(1, 2)
    kx = k[:, :, :gdn_tokens].repeat_interleave(HQ // HKV, 1).transpose(1, 2)
    vx = v[:, :, :gdn_tokens].repeat_interleave(HQ // HKV, 1).transpose(1, 2)
    gl, bt = torch.nn.functional.logsigmoid(zg + 3.9), torch.sigmoid(zb)

    def polar_sample():
        with torch.no_grad():
            OP.polar_rows(q, k, v, n, rows, params=p, k_block=4096)

    def gdn_sample():
        with torch.no_grad():
            OG.chunk_gated_delta_rule(qg, kx, vx, gl, bt, scale=1.0, output_final_state=True,
                                      use_qk_l2norm_in_kernel=True)

    s_polar, r_polar = _median_runs(polar_sample, 10.0, min_runs=3, max_runs=5)
    s_gdn, r_gdn = _median_runs(gdn_sample, 6.0, min_runs=3, max_runs=5)
    sec = s_polar * pair_scale + s_gdn * tok_scale
    flops = polar_flops(1, T) + gdn_flops(1, T)
    return {"value": flops / sec / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "extrapolated": True,
            "sample": (f"configs[2] B=1 T={T}, 8/2 heads, d=128, fp32 torch CPU oracle: Polar exact rows "
                       f"every {row_stride} ({len(rows)} rows x 8 heads, all causal keys; median of "
                       f"{r_polar} runs {s_polar:.3f} s) x {pair_scale:.1f} (causal pairs), plus the chunked "
                       f"gated delta over the first {gdn_tokens} tokens (median of {r_gdn} runs {s_gdn:.3f} s) "
                       f"x {tok_scale:.0f}; extrapolated step {sec:.1f} s"),
            "ms_per_step_extrapolated": sec * 1e3, "polar_s_extrapolated": s_polar * pair_scale,
            "gdn_s_extrapolated": s_gdn * tok_scale,
            "torch_threads": torch.get_num_threads(), "cpu_model": _cpu_model(),
            "c1": dict(cpu_c1(torch), workload="configs[0]: one global block (Polar + gated-delta "
                                                "memory + MLP), B=1, T=2048, hidden 1024, 8/2 heads, "
                                                "d=128, fp32, params N(0,0.02) seed 0 (exact, not extrapolated)")}


def copy_calibration(torch, dev, steps):
    """A plain copy of known size (512 MiB read + 512 MiB written per launch): what
    rocprofv3's FETCH_SIZE / WRITE_SIZE report for it, divided by the true byte counts,
    gives the factors that turn those counters into HBM bytes for the kernels here."""
    n = 512 << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 255)
    dst = torch.empty_like(src)
    ms = _time(torch, lambda: dst.copy_(src), max(3, steps), 1)
    return {"bytes_read": n, "bytes_written": n, "ms": ms, "gbs": 2 * n / (ms * 1e-3) / 1e9}


def _traffic(name):
    """HBM bytes per Polar prefill launch measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by a copy-kernel calibration), committed under profiles/."""
    f = ROOT / "profiles" / name
    try:
        return json.loads(f.read_text()).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=["c1", "c2", "c3", "c4", "c5", "ops", "train", "copy", "cpu"], default=None,
                    help="one workload; 'copy' runs a plain 512 MiB device copy, the "
                         "reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-long", action="store_true", help="skip T=262,144")

    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build targets a single MI355X "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        return 2
    import torch
    from atma_amd import _lib
    _lib.load()
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False

    out = {}
    if args.only == "copy":
        out["copy"] = copy_calibration(torch, dev, args.steps)
        print(json.dumps(out))
        return 0
    if args.only == "cpu":
        print(json.dumps({"cpu_baseline": cpu_baseline(torch)}))
        return 0
    if args.only in (None, "c3"):
        # the headline: configs[2] at T = 65,536, `warmup` untimed and `steps` timed steps
        c3 = [bench_prefill(torch, dev, 1, 65536, args.steps, args.warmup)]
        print(f"# c3 prefill T=65536: {json.dumps(c3[0])}", file=sys.stderr, flush=True)
        if not args.no_long:
            c3.append(bench_prefill(torch, dev, 1, 262144, 2, 1))
            print(f"# c3 prefill T=262144: {json.dumps(c3[1])}", file=sys.stderr, flush=True)
        out["c3"] = c3
    if args.only in (None, "c2"):
        c2 = bench_prefill(torch, dev, 8, 2048, args.steps, args.warmup)
        print(f"# c2 prefill: {json.dumps(c2)}", file=sys.stderr, flush=True)
        out["c2"] = c2
    if args.only in (None, "c4"):
        c4 = bench_decode(torch, dev, args.steps, args.warmup)
        print(f"# c4 decode: {json.dumps(c4)}", file=sys.stderr, flush=True)
        c4w = bench_decode(torch, dev, max(5, args.steps // 2), 2, full=True)
        print(f"# c4 decode 64x32768: {json.dumps(c4w)}", file=sys.stderr, flush=True)
        out["c4"] = [c4, c4w]
    if args.only in (None, "train"):
        tr = bench_train(torch, dev, max(5, args.steps // 2), 2)
        print(f"# train c2: {json.dumps(tr)}", file=sys.stderr, flush=True)
        out["train"] = tr
    if args.only in (None, "c5"):
        c5 = bench_c5(torch, dev)
        print(f"# c5 served 378M: {json.dumps(c5)}", file=sys.stderr, flush=True)
        out["c5"] = c5
    if args.only in (None, "c1"):
        c1 = bench_c1_gpu(torch, dev, max(3, args.steps // 2), 2)
        print(f"# c1 block fp32 (GPU): {json.dumps(c1)}", file=sys.stderr, flush=True)
        out["c1"] = c1
    if args.only in (None, "ops"):
        ops = bench_inference_ops(torch, dev, args.steps, args.warmup)
        print(f"# inference ops: {json.dumps(ops)}", file=sys.stderr, flush=True)
        out["ops"] = ops
    if args.only is not None:
        print(json.dumps(out))
        return 0

    c3, c2 = out["c3"][0], out["c2"]
    rnd = lambda d: {k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}  # noqa: E731
    line = {
        "metric": METRIC,
        "value": round(c3["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c3["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v and gate logits; Polar params at the reference priors)",
        "config": {"workload": "configs[2]: long-context single-sequence global-layer prefill, Polar fwd + "
                               "gated-delta chunked (C=64, fp32 state from 0), B=1, T=65536, in the layer's "
                               f"schedule ({c3['schedule']})", "B": 1, "T": 65536, "q_heads": HQ,
                   "kv_heads": HKV, "head_dim": D, "mfma_frac_of_bf16_peak": round(c3["mfma_frac"], 4)},
        "roofline": {"bound": "mfma", "kernel": "polar_fwd16_pp_kernel<bf16,128>",
                     "achieved": round(c3["polar_tflops"], 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(c3["polar_mfma_frac"], 4),
                     "traffic": _traffic("polar_prefill_c3_t65536_traffic.json"),
                     "launch_ms": round(c3["polar_ms"], 4), "flops_per_launch": c3["polar_flops"]},
        "breakdown_c3": rnd(c3),
        "breakdown_c2": dict(rnd(c2), roofline_traffic=_traffic("polar_prefill_c2_traffic.json")),
        "prefill_long": [rnd(r) for r in out["c3"][1:]],
        "decode": [rnd(r) for r in out["c4"]],
        "inference_ops": {n: rnd(r) for n, r in out["ops"].items()},
        "block_c1_gpu": rnd(out["c1"]),
        "serve_c5": rnd(out["c5"]),
        "train_c2": rnd(out["train"]),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())

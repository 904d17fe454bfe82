"""Model runner of the paged engine (``inference/engine/model_runner.py:13-533``).

It owns the device state of a serving process: the model, the per-sequence state
tables (keys ``attn_{i}_{q,k,v}``, ``conv_{i}_gated``, ``mem_{i}``, as the reference,
``:161-211``), one paged KV tensor ``(2, n_global, num_pages, page_size, Hkv, d)``
(``:73-155``), and the decode step captured as HIP graphs per batch-size bucket
(``:254-310``).  ``prepare_prefill`` / ``prepare_decode`` turn scheduled sequences into
the device tensors and routing flags of the ``Context`` (``:316-480``); ``run`` runs the
model and samples (``:491-533``).

Differences from the reference, each deliberate:

* The state tables carry one extra row (index ``max_num_seqs``) that no sequence owns.
  Graph rows beyond the live batch point there, so a padded replay advances no real
  sequence's conv / memory state (the reference leaves those rows' slots stale).
* The tables are zeroed after warm-up and capture, whose dummy steps write into them.
* The KV page count comes from ``Config.num_kvcache_blocks`` or, when -1, from
  ``max_num_seqs x max_model_len`` within ``gpu_memory_utilization`` of free memory,
  instead of a profiling prefill at the full batch budget.
* The grouped (tile-mapped) Polar route is taken for 16-bit models only, the dtype its
  kernel serves (``kernel/polar_triton.py:625-627``); fp32 ragged prompts take the
  per-sequence route.
"""

from collections import deque

import numpy as np
import torch

from ..layers.attention import Attention
from .config import Config
from .context import get_context, reset_context, set_context
from .model import Atma, Sampler
from .sequence import Sequence

POLAR_TILE_ROWS = 128    # query rows per tile of the packed Polar launch


class ModelRunner:

    def __init__(self, config: Config, model: Atma = None):
        self.config = config
        hf = config.hf_config
        self.block_size = config.kvcache_block_size
        Sequence.block_size = config.kvcache_block_size
        self.enforce_eager = config.enforce_eager
        if not torch.cuda.is_available():
            raise RuntimeError("ModelRunner serves on the GPU only (HIP kernels); no GPU is visible")
        self.device = torch.device("cuda", torch.cuda.current_device())
        if model is None:
            model = Atma(hf)
            if config.model:
                from ..layers.loader import load_model
                load_model(model, config.model, strict=config.strict_weights)
            else:
                model.init_weights(config.init_std, config.seed)
        self.model = model.to(self.device, hf.dtype).eval()
        self.sampler = Sampler()
        self.last_logits = None
        self.allocate_conv_state_tables()
        self.allocate_kv_cache()
        self.warmup_model()
        if not self.enforce_eager:
            self.capture_cudagraph()
        self._zero_state_tables()

    def exit(self):
        for name in ("graphs", "graph_out", "graph_pool", "graph_vars"):
            if hasattr(self, name):
                delattr(self, name)
        torch.cuda.synchronize(self.device)

    # ------------------------------------------------------------------ state
    def allocate_conv_state_tables(self):
        hf = self.config.hf_config
        rows = self.config.max_num_seqs + 1          # + the padding row no sequence owns
        dev, dt = self.device, hf.dtype
        kv_hidden = hf.num_key_value_heads * hf.head_dim
        self.conv_state_tables = {}
        for i in range(hf.num_hidden_layers):
            if hf.is_attention_layer(i):
                for s, dim in (("q", hf.hidden_size), ("k", kv_hidden), ("v", kv_hidden)):
                    self.conv_state_tables[f"attn_{i}_{s}"] = torch.zeros(
                        rows, dim, hf.attn_kernel_size - 1, device=dev, dtype=dt)
                if hf.mem_enabled:
                    self.conv_state_tables[f"mem_{i}"] = torch.zeros(
                        rows, hf.num_attention_heads, hf.head_dim, hf.head_dim, device=dev, dtype=torch.float32)
            else:
                self.conv_state_tables[f"conv_{i}_gated"] = torch.zeros(
                    rows, hf.hidden_size, hf.conv_kernel_size - 1, device=dev, dtype=dt)
        self.pad_slot = self.config.max_num_seqs
        self._free_slots = deque(range(self.config.max_num_seqs))

    def _zero_state_tables(self):
        for t in self.conv_state_tables.values():
            t.zero_()

    def allocate_kv_cache(self):
        hf, cfg = self.config.hf_config, self.config
        self.attn_modules = [m for m in self.model.modules() if isinstance(m, Attention)]
        n_attn = len(self.attn_modules)
        if n_attn == 0:
            return
        item = torch.empty((), dtype=hf.dtype).element_size()
        page_bytes = 2 * n_attn * self.block_size * hf.num_key_value_heads * hf.head_dim * item
        if cfg.num_kvcache_blocks <= 0:
            want = cfg.max_num_seqs * ((cfg.max_model_len + self.block_size - 1) // self.block_size)
            free, _ = torch.cuda.mem_get_info(self.device)
            cap = int(free * cfg.gpu_memory_utilization) // page_bytes
            cfg.num_kvcache_blocks = max(16, min(want, cap))
        self.kv_cache = torch.zeros(2, n_attn, cfg.num_kvcache_blocks, self.block_size, hf.num_key_value_heads,
                                    hf.head_dim, device=self.device, dtype=hf.dtype)
        for idx, m in enumerate(self.attn_modules):
            m.k_cache = self.kv_cache[0, idx]
            m.v_cache = self.kv_cache[1, idx]

    def alloc_seq_slot(self, seq: Sequence) -> int:
        seq.seq_slot = self._free_slots.popleft()
        return seq.seq_slot

    def free_seq_slot(self, seq: Sequence):
        """Release a sequence's table rows, zeroed for the next owner (``:205-211``)."""
        self.free_seq_slots([seq])

    def free_seq_slots(self, seqs):
        """``free_seq_slot`` for several sequences at once: one zeroing launch per state table
        for all their rows (a batch that finishes together, 32 requests x 28 tables, would
        otherwise make 896 launches)."""
        slots = [s.seq_slot for s in seqs if s.seq_slot >= 0]
        if not slots:
            return
        if len(slots) == 1:
            for t in self.conv_state_tables.values():
                t[slots[0]].zero_()
        else:
            idx = torch.tensor(slots, dtype=torch.int64).to(self.device)
            for t in self.conv_state_tables.values():
                t.index_fill_(0, idx, 0)
        for s in seqs:
            if s.seq_slot >= 0:
                self._free_slots.append(s.seq_slot)
                s.seq_slot = -1

    # ------------------------------------------------------------------ warm-up / graphs
    def warmup_model(self):
        """One short prefill and one decode step through every kernel (``:229-248``)."""
        n = min(64, self.config.max_num_batched_tokens, self.config.max_model_len)
        pre = Sequence([0] * n)
        pre.num_scheduled_tokens = n
        pre.block_table = list(range(min((n + self.block_size - 1) // self.block_size,
                                         self.config.num_kvcache_blocks)))
        dec = Sequence([0])
        dec.num_scheduled_tokens = 1
        dec.block_table = [0]
        try:
            self.run([pre], is_prefill=True)
            self.free_seq_slot(pre)
            self.run([dec], is_prefill=False)
        finally:
            for s in (pre, dec):
                self.free_seq_slot(s)
        torch.cuda.synchronize(self.device)

    def _decode_stage(self, max_bs, max_blocks):
        """One buffer for every decode-step input the graphs read: token ids and table
        rows (int64), cache slots, context lengths and block tables (int32).  Each step
        fills a pinned host copy (two, used in turn) and sends it with one H2D copy."""
        n64, n32 = 2 * max_bs, 2 * max_bs + max_bs * max_blocks
        nbytes = 8 * n64 + 4 * n32
        dev = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        hosts = [torch.empty(nbytes, dtype=torch.uint8).pin_memory() for _ in range(2)]

        def views(buf):
            i64 = buf[:8 * n64].view(torch.int64)
            i32 = buf[8 * n64:].view(torch.int32)
            return dict(input_ids=i64[:max_bs], seq_slots=i64[max_bs:], slot_mapping=i32[:max_bs],
                        context_lens=i32[max_bs:2 * max_bs],
                        block_tables=i32[2 * max_bs:].view(max_bs, max_blocks))
        self._stage_dev, self._stage_hosts = dev, hosts
        self._stage_np = [{k: v.numpy() for k, v in views(h).items()} for h in hosts]
        self._stage_key = [None, None]   # the batch whose table rows and slots each host copy holds
        self._stage_flip = 0
        self._stage_ids_bytes = 8 * max_bs  # the token ids lead the buffer
        # greedy ids of a launched step come back through these (pinned, used in turn)
        self._ids_host = [torch.empty(max_bs, dtype=torch.int64).pin_memory() for _ in range(2)]
        self._ids_done = [torch.cuda.Event(), torch.cuda.Event()]
        self._ids_flip = 0
        return views(dev)

    @torch.inference_mode()
    def capture_cudagraph(self):
        """The decode forward captured once per batch-size bucket (``:254-310``), LM head
        included; 16-bit models also take the greedy ids inside the graph
        (``Atma.decode_head``), written over the step's own input ids: a step that feeds the
        same batch again finds its tokens in place (``launch_decode``)."""
        cfg = self.config
        max_bs = cfg.max_num_seqs
        max_blocks = (cfg.max_model_len + self.block_size - 1) // self.block_size
        gv = self._decode_stage(max_bs, max_blocks)
        gv["slot_mapping"].fill_(-1)
        gv["context_lens"].zero_()
        gv["block_tables"].zero_()
        gv["input_ids"].zero_()
        gv["seq_slots"].fill_(self.pad_slot)
        self.graph_bs = sorted({b for b in [1, 2, 4, 8] + list(range(16, max_bs + 1, 16)) + [max_bs]
                                if b <= max_bs})
        self.graphs, self.graph_out, self.graph_pool = {}, {}, None
        # two execs per bucket, replayed in turn: a graph exec relaunched right behind
        # itself waits for its previous launch to retire, two alternating ones do not
        self.graph_flip = 0
        for bs in reversed(self.graph_bs):
            set_context(False, slot_mapping=gv["slot_mapping"][:bs], context_lens=gv["context_lens"][:bs],
                        block_tables=gv["block_tables"][:bs], seq_slots=gv["seq_slots"][:bs],
                        conv_state_tables=self.conv_state_tables)
            ids_out = gv["input_ids"][:bs]
            self.model.decode_head(self.model(gv["input_ids"][:bs]), ids_out)    # warm-up
            pair, outs = [], []
            for _ in range(2):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, self.graph_pool):
                    out = self.model.decode_head(self.model(gv["input_ids"][:bs]), ids_out)
                if self.graph_pool is None:
                    self.graph_pool = graph.pool()
                pair.append(graph)
                outs.append(out)
            self.graphs[bs], self.graph_out[bs] = pair, outs
            torch.cuda.synchronize(self.device)
            reset_context()
        self.graph_vars = gv

    def _uses_graph(self, bs):
        return not self.enforce_eager and hasattr(self, "graphs") and bs <= self.config.max_num_seqs

    def can_pipeline(self, seqs):
        """True when decode steps of this batch can be launched ahead of reading back the
        previous step's tokens: captured graphs that take the greedy ids themselves (16-bit
        models), every request greedy, the batch within the largest bucket."""
        return (self._uses_graph(len(seqs)) and self.graph_out[self.graph_bs[-1]][0][1] is not None
                and all(s.temperature == 0 for s in seqs))

    @torch.inference_mode()
    def launch_decode(self, seqs, ahead):
        """Enqueue one decode step of ``seqs`` without waiting for it; ``collect`` returns its
        tokens.  ahead 0: every request's newest token is known on the host.  ahead 1: the
        step right after a launched, not yet collected step of the same batch in the same
        order -- its input tokens are that step's greedy ids, already in place on the device
        (the graph writes them over its input ids), and each request is one token longer
        than its host record.  The step's ids are copied back into pinned memory behind the
        graph."""
        bs = len(seqs)
        bucket = self._stage(seqs, ahead)
        off = self._stage_ids_bytes if ahead else 0
        self._stage_dev[off:].copy_(self._stage_hosts[self._stage_flip ^ 1][off:], non_blocking=True)
        g = self.graph_flip
        self.graph_flip ^= 1
        self.graphs[bucket][g].replay()
        logits, ids = self.graph_out[bucket][g]
        host, done = self._ids_host[self._ids_flip], self._ids_done[self._ids_flip]
        self._ids_flip ^= 1
        host[:bs].copy_(ids[:bs], non_blocking=True)
        done.record()
        self.last_logits = logits[:bs]
        return done, host, bs

    @staticmethod
    def collect(launch):
        """The token ids of a ``launch_decode`` step (waits for it)."""
        done, host, bs = launch
        done.synchronize()
        return host[:bs].tolist()

    def _stage(self, seqs, ahead=0):
        """Fill the next pinned staging copy for a decode step of ``seqs`` whose requests are
        ``ahead`` tokens longer than their host records (rows past the batch: token 0, slot
        -1, length 0, the padding table row); returns the graph bucket."""
        bs = len(seqs)
        bucket = next(b for b in self.graph_bs if b >= bs)
        k = self._stage_flip
        self._stage_flip ^= 1
        h = self._stage_np[k]
        page = self.block_size
        bt = h["block_tables"]
        # table rows and state slots change only with the batch (a request's pages are reserved
        # for its lifetime), so a host copy keeps them while it serves the same batch
        key = (bucket, tuple((s.seq_id, s.seq_slot, len(s.block_table)) for s in seqs))
        if self._stage_key[k] != key:
            h["seq_slots"][:bs] = [s.seq_slot for s in seqs]
            h["seq_slots"][bs:] = self.pad_slot
            h["input_ids"][bs:] = 0
            h["context_lens"][bs:] = 0
            h["slot_mapping"][bs:] = -1
            bt[:bucket] = 0
            for i, s in enumerate(seqs):
                bt[i, :len(s.block_table)] = s.block_table
            self._stage_key[k] = key
        lens = np.fromiter((len(s) for s in seqs), dtype=np.int64, count=bs) + ahead
        if not ahead:
            h["input_ids"][:bs] = [s.last_token for s in seqs]
        h["context_lens"][:bs] = lens
        pos = lens - 1        # the new token's cache slot: its position's row in its position's page
        h["slot_mapping"][:bs] = bt[np.arange(bs), pos // page] * page + pos % page
        return bucket

    def _run_decode_graph(self, seqs):
        """Replay the smallest captured bucket that fits: the step's inputs go in one H2D
        copy of the staging buffer (rows past the batch: token 0, slot -1, length 0, the
        tables' spare row), the graph runs the model and the LM head.  Returns (logits
        (bs, V), greedy ids (bs,) or None)."""
        bs = len(seqs)
        bucket = self._stage(seqs)
        self._stage_dev.copy_(self._stage_hosts[self._stage_flip ^ 1], non_blocking=True)
        g = self.graph_flip
        self.graph_flip ^= 1
        self.graphs[bucket][g].replay()
        logits, ids = self.graph_out[bucket][g]
        return logits[:bs], (None if ids is None else ids[:bs])

    # ------------------------------------------------------------------ inputs
    def _to_dev(self, values, dtype):
        """A host list or numpy array as a device tensor (pinned staging, asynchronous copy)."""
        t = torch.from_numpy(values).to(dtype) if isinstance(values, np.ndarray) else torch.tensor(values, dtype=dtype)
        if self.device.type != "cuda":
            return t
        return t.pin_memory().to(self.device, non_blocking=True)

    def prepare_block_tables(self, seqs):
        width = max(len(s.block_table) for s in seqs) if seqs else 0
        return self._to_dev([s.block_table + [-1] * (width - len(s.block_table)) for s in seqs], torch.int32)

    def prepare_prefill(self, seqs):
        """Token ids, cache slots and the route of one prefill batch (``:328-449``)."""
        # per-token arrays built with numpy: a prefill batch holds up to max_num_batched_tokens
        # tokens, and per-token Python loops and list->tensor conversions cost tens of ms there
        ids, pos, slot = [], [], []
        cu_q, cu_k = [0], [0]
        max_q = max_k = 0
        bs = self.block_size
        for seq in seqs:
            start = seq.num_cached_tokens
            end = start + seq.num_scheduled_tokens
            ids.append(np.asarray(seq[start:end], dtype=np.int64))
            p = np.arange(start, end, dtype=np.int64)
            pos.append(p)
            # page = block_table[pos // page_size], row = pos % page_size
            slot.append(np.asarray(seq.block_table, dtype=np.int64)[p // bs] * bs + p % bs)
            cu_q.append(cu_q[-1] + end - start)
            cu_k.append(cu_k[-1] + end)
            max_q, max_k = max(max_q, end - start), max(max_k, end)
        input_ids, positions, slot_mapping = (np.concatenate(a) for a in (ids, pos, slot))
        seqlens = [cu_q[i + 1] - cu_q[i] for i in range(len(seqs))]
        fresh = all(s.num_cached_tokens == 0 and s.num_scheduled_tokens == len(s) for s in seqs)
        within = sum(seqlens) <= self.config.max_num_batched_tokens
        dense = len(seqs) > 1 and seqlens[0] > 0 and len(set(seqlens)) == 1 and fresh and within
        grouped = (len(seqs) > 1 and not dense and all(n > 0 for n in seqlens) and fresh and within
                   and self.config.hf_config.dtype in (torch.bfloat16, torch.float16))
        block_tables = self.prepare_block_tables(seqs) if cu_k[-1] > cu_q[-1] else None
        kw = {}
        if fresh and all(n > 0 for n in seqlens):
            # per-token (sequence start, end, table row): the packed convolutions' map
            offs = np.asarray(cu_q, dtype=np.int64)
            starts = np.repeat(offs[:-1], seqlens)
            ends = np.repeat(offs[1:], seqlens)
            slots = np.repeat(np.asarray([s.seq_slot for s in seqs], dtype=np.int64), seqlens)
            kw.update(token_seq_starts=self._to_dev(starts, torch.int32), token_seq_ends=self._to_dev(ends, torch.int32),
                      token_seq_slots=self._to_dev(slots, torch.int32))
        if grouped:
            ts, tq, tl, packed = [], [], [], 0
            for n in seqlens:                 # one entry per 128-row query tile (:390-404)
                for q0 in range(0, n, POLAR_TILE_ROWS):
                    ts.append(packed)
                    tq.append(q0)
                    tl.append(n)
                packed += n
            kw.update(polar_tile_seq_starts=self._to_dev(ts, torch.int32),
                      polar_tile_q_starts=self._to_dev(tq, torch.int32),
                      polar_tile_seq_lens=self._to_dev(tl, torch.int32))
        ctx = set_context(True, cu_seqlens_q=self._to_dev(cu_q, torch.int32),
                          cu_seqlens_k=self._to_dev(cu_k, torch.int32), max_seqlen_q=max_q, max_seqlen_k=max_k,
                          slot_mapping=self._to_dev(slot_mapping, torch.int32), block_tables=block_tables,
                          seqlens_q=seqlens, conv_state_tables=self.conv_state_tables,
                          seq_slots=self._to_dev([s.seq_slot for s in seqs], torch.int64),
                          dense_prefill=dense, dense_batch_size=len(seqs) if dense else 0,
                          dense_seq_len=seqlens[0] if dense else 0, grouped_polar_prefill=grouped, **kw)
        ctx.seqs = seqs
        return self._to_dev(input_ids, torch.int64), self._to_dev(positions, torch.int64)

    def prepare_decode(self, seqs):
        """One new token per sequence (``:451-480``): ``context_lens`` includes it, and its
        cache slot is its position's row in its position's page (a sequence may hold pages
        beyond its current length: they are reserved for its lifetime)."""
        input_ids = [s.last_token for s in seqs]
        positions = [len(s) - 1 for s in seqs]
        context_lens = [len(s) for s in seqs]
        bs = self.block_size
        slot_mapping = [s.block_table[p // bs] * bs + p % bs for s, p in zip(seqs, positions)]
        set_context(False, slot_mapping=self._to_dev(slot_mapping, torch.int32),
                    context_lens=self._to_dev(context_lens, torch.int32),
                    block_tables=self.prepare_block_tables(seqs), conv_state_tables=self.conv_state_tables,
                    seq_slots=self._to_dev([s.seq_slot for s in seqs], torch.int64))
        return self._to_dev(input_ids, torch.int64), self._to_dev(positions, torch.int64)

    # ------------------------------------------------------------------ forward
    @torch.inference_mode()
    def run_model(self, input_ids, positions, is_prefill):
        """The model and its LM head, eager (prefill, or decode without graphs)."""
        return self.model.compute_logits(self.model(input_ids, positions))

    @torch.inference_mode()
    def run(self, seqs, is_prefill):
        """Schedule-step entry (``:520-533``): slots for new sequences, inputs, forward,
        sampling; returns one token id per sequence.  ``last_logits`` keeps the step's
        logits (one row per sequence; after a graph replay, valid until the next step)."""
        for seq in seqs:
            if seq.seq_slot < 0:
                self.alloc_seq_slot(seq)
        temps = [s.temperature for s in seqs]
        greedy = all(t == 0 for t in temps)
        ids = None
        if not is_prefill and self._uses_graph(len(seqs)):
            logits, ids = self._run_decode_graph(seqs)
        else:
            input_ids, positions = self.prepare_prefill(seqs) if is_prefill else self.prepare_decode(seqs)
            logits = self.run_model(input_ids, positions, is_prefill)
        self.last_logits = logits
        if ids is None or not greedy:
            ids = self.sampler(logits, self._to_dev(temps, torch.float32), all_greedy=greedy)
        reset_context()
        return ids.tolist()

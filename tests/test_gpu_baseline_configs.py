"""Parity at the full BASELINE.json configurations, through the HIP path, against the
CPU oracle on the same seeded inputs.

* one global block (Polar + gated-delta memory + MLP), hidden 1,024,
  8 / 2 heads, d = 128, B = 1, T = 2,048, fp32, every parameter N(0, 0.02) from seed 0
  (the reference's own test convention, ``tests/test_dense_prefill.py:105-106``),
  input N(0, 1) -- max-abs <= 1e-4 against ``oracle/block.global_block``, on the
  inference route and on the training (autograd) route.
* the prefill ops at B = 8, T = 2,048, 8 / 2 heads, d = 128, bf16 --
  Polar against the streaming oracle (fp32, k_block 512) and the gated-delta memory
  with the layer's raw-logit gates against the FLA-contract oracle, both <= 2e-2
  relative (max|a-b| / max|b|).
* B = 1, T = 262,144, all 8 / 2 heads -- Polar on sampled rows (first,
  tile edges, last) through the exact row oracle; gated delta against the fp32 oracle
  over the whole output and state, and one call == two calls split at a chunk
  boundary with the fp32 state carried, bitwise.
* the graph-replayed decode step that ``bench.py`` times (store_kvcache ->
  Polar decode -> gated-delta step, 64 sequences, ctx ~ U[1,024, 32,768], shuffled
  256-token pages) == the same step run eagerly, bitwise over three steps (outputs,
  KV pages and state table); and each step against the oracle on sampled sequences
  (decode output, the KV rows written, the readout and the updated state rows).
* Sharp scores in 16 bits: q scaled by 8 and 16 drives the 16-bit kernel's
  overflow-redo branch (a block whose exponentials exceed the optimistic bound is
  recomputed against its true max); bf16 and fp16 against the fp32 oracle.
"""

import sys
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

from oracle import block as OB
from oracle import gated_delta as OG
from oracle import polar as OP
from tests.helpers import max_abs, polar_params, rel_err

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
HQ, HKV, D = 8, 2, 128


def _say(msg):
    print(f"[baseline-configs] {msg}", flush=True)


# --------------------------------------------------------------------------- configs[0]
def _c1_block():
    from atma_amd.layers.global_attention import GlobalBlock
    torch.manual_seed(0)
    blk = GlobalBlock(1024, head_dim=128)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0.0, 0.02)
    return blk


@pytest.mark.parametrize("route", ["inference", "training"])
def test_configs0_global_block_fp32(dev, route):
    _say(f"configs[0] block fp32 T=2048 route={route}")
    blk = _c1_block()
    x = torch.randn(1, 2048, 1024, generator=torch.Generator().manual_seed(0))
    sd = {k: v.detach().cpu().clone() for k, v in blk.state_dict().items()}
    ref = OB.global_block(sd, x, H=HQ, Hkv=HKV, dk=D)
    blk = blk.to(dev)
    xd = x.to(dev)
    if route == "training":
        xd.requires_grad_(True)
        out = blk(xd)
        out.sum().backward()      # the route must also run its backward
        assert all(p.grad is not None for p in blk.parameters())
        out = out.detach()
    else:
        with torch.no_grad():
            out = blk(xd)
    assert max_abs(out, ref) <= 1e-4, max_abs(out, ref)


# --------------------------------------------------------------------------- configs[1]
def test_configs1_polar_full_size_bf16(dev):
    from atma_amd.kernel import polar_attention_fwd
    _say("configs[1] Polar B=8 T=2048 8/2 d=128 bf16")
    B, T = 8, 2048
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(B, h, T, D, generator=g).bfloat16() for h in (HQ, HKV, HKV))
    p = polar_params(HQ, D, seed=1)        # parity set: P ~ N(0, 1)
    n = torch.arange(1, T + 1, dtype=torch.float32)
    c, m = polar_attention_fwd(q.to(dev), k.to(dev), v.to(dev), n.to(dev), **{a: b.to(dev) for a, b in p.items()})
    c, m = c.cpu(), m.cpu()
    c_ref, m_ref = OP.polar_online(q.float(), k.float(), v.float(), n, params=p, k_block=512)
    assert rel_err(c, c_ref) <= 2e-2, rel_err(c, c_ref)
    assert rel_err(m, m_ref) <= 2e-2, rel_err(m, m_ref)


def test_configs1_gated_delta_raw_gates_bf16(dev):
    from atma_amd.kernel import chunk_gated_delta_rule
    _say("configs[1] gated delta B=8 T=2048 8/2 d=128 bf16, raw gate logits")
    B, T = 8, 2048
    g = torch.Generator().manual_seed(2)
    q = torch.randn(B, T, HQ, D, generator=g).bfloat16()
    k, v = (torch.randn(B, T, HKV, D, generator=g).bfloat16() for _ in range(2))
    zg, zb = torch.randn(B, T, HQ, generator=g), torch.randn(B, T, HQ, generator=g)
    o, S = chunk_gated_delta_rule(q.to(dev), k.to(dev), v.to(dev), zg.to(dev), zb.to(dev), scale=1.0,
                                  initial_state=torch.zeros(B, HQ, D, D, device=dev), output_final_state=True,
                                  use_qk_l2norm_in_kernel=True, gate_bias=(3.9, 0.0))
    o, S = o.cpu(), S.cpu()
    kx, vx = (t.repeat_interleave(HQ // HKV, 2).float() for t in (k, v))
    o_ref, S_ref = OG.chunk_gated_delta_rule(q.float(), kx, vx, F.logsigmoid(zg + 3.9), torch.sigmoid(zb),
                                             scale=1.0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert rel_err(o, o_ref) <= 2e-2, rel_err(o, o_ref)
    assert rel_err(S, S_ref) <= 2e-2, rel_err(S, S_ref)


# --------------------------------------------------------------------------- configs[2]
T_LONG = 262144


def test_configs2_polar_t262144_rows_bf16(dev):
    from atma_amd.kernel import polar_attention_fwd
    _say("configs[2] Polar B=1 T=262144 8/2 d=128 bf16 (row-sampled)")
    g = torch.Generator(device=dev).manual_seed(3)
    q = torch.randn(1, HQ, T_LONG, D, device=dev, generator=g, dtype=torch.bfloat16)
    k = torch.randn(1, HKV, T_LONG, D, device=dev, generator=g, dtype=torch.bfloat16)
    v = torch.randn(1, HKV, T_LONG, D, device=dev, generator=g, dtype=torch.bfloat16)
    p = polar_params(HQ, D, seed=3, prior=True)
    n = torch.arange(1, T_LONG + 1, dtype=torch.float32)
    c, m = polar_attention_fwd(q, k, v, n.to(dev), **{a: b.to(dev) for a, b in p.items()})
    rows = torch.tensor([0, 1, 127, 128, 4095, 65536, 131071, 200003, T_LONG - 2, T_LONG - 1])
    c_rows, m_rows = c[:, :, rows.to(dev)].cpu(), m[:, :, rows.to(dev)].cpu()
    assert torch.isfinite(c.float()).all() and torch.isfinite(m.float()).all()
    del c, m
    qs = q[:, :, rows.to(dev)].float().cpu()
    kc, vc = k.float().cpu(), v.float().cpu()
    # the exact row oracle (polar_rows) on the sampled query rows: each row's own count
    c_ref, m_ref = OP.polar_online(qs, kc, vc, n[rows], params=p, k_block=8192)
    assert rel_err(c_rows, c_ref) <= 2e-2, rel_err(c_rows, c_ref)
    assert rel_err(m_rows, m_ref) <= 2e-2, rel_err(m_rows, m_ref)


def test_configs2_gated_delta_t262144_bf16(dev):
    from atma_amd.kernel import chunk_gated_delta_rule
    _say("configs[2] gated delta B=1 T=262144 8/2 d=128 bf16")
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, T_LONG, HQ, D, generator=g).bfloat16()
    k, v = (torch.randn(1, T_LONG, HKV, D, generator=g).bfloat16() for _ in range(2))
    zg, zb = torch.randn(1, T_LONG, HQ, generator=g), torch.randn(1, T_LONG, HQ, generator=g)
    kw = dict(scale=1.0, output_final_state=True, use_qk_l2norm_in_kernel=True, gate_bias=(3.9, 0.0))
    qd, kd, vd, zgd, zbd = (t.to(dev) for t in (q, k, v, zg, zb))
    o, S = chunk_gated_delta_rule(qd, kd, vd, zgd, zbd, **kw)
    h = T_LONG // 2 + 64 * 7         # a chunk boundary off the midpoint
    o1, S1 = chunk_gated_delta_rule(qd[:, :h], kd[:, :h], vd[:, :h], zgd[:, :h], zbd[:, :h], **kw)
    o2, S2 = chunk_gated_delta_rule(qd[:, h:], kd[:, h:], vd[:, h:], zgd[:, h:], zbd[:, h:],
                                    initial_state=S1, **kw)
    # (one head group of a sequence this long takes the segmented recurrence, whose
    # segment entry states are combined in fp32: a split run agrees to rounding)
    assert rel_err(torch.cat([o1, o2], 1), o) <= 5e-3 and rel_err(S2, S) <= 5e-3
    o, S = o.cpu(), S.cpu()
    del qd, kd, vd, o1, o2
    kx, vx = (t.repeat_interleave(HQ // HKV, 2).float() for t in (k, v))
    o_ref, S_ref = OG.chunk_gated_delta_rule(q.float(), kx, vx, F.logsigmoid(zg + 3.9), torch.sigmoid(zb),
                                             scale=1.0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert rel_err(o, o_ref) <= 2e-2, rel_err(o, o_ref)
    assert rel_err(S, S_ref) <= 2e-2, rel_err(S, S_ref)


def test_configs2_timed_step_t65536_overlapped(dev):
    """The configs[2] step exactly as ``bench.py`` times it at T = 65,536, 8 / 2 heads: the
    memory branch on the side stream with its recurrence unsegmented (start signal), Polar
    launched once the recurrence has started.  Polar on sampled rows against the exact row
    oracle; the memory output and final state against the fp32 FLA-contract oracle."""
    bench = _bench()
    _say("configs[2] timed step B=1 T=65536 8/2 d=128 bf16, overlapped schedule")
    w = bench.Prefill(torch, dev, 1, 65536, seed=5)
    assert w.overlap                         # the layer's schedule at this shape
    (c, m), (o, S) = w.step_overlap()
    (c2, m2), (o2, S2) = w.step_sequential() # the sequential schedule: segmented recurrence
    torch.cuda.synchronize()
    assert torch.equal(c, c2) and torch.equal(m, m2)
    # the two schedules' recurrences differ in rounding only
    assert rel_err(o2.float(), o.float()) <= 1e-2 and rel_err(S2, S) <= 1e-3, (rel_err(o2.float(), o.float()),
                                                                               rel_err(S2, S))
    del c2, m2, o2, S2
    T = w.T
    rows = torch.tensor([0, 1, 63, 127, 128, 4095, 30001, 65535 - 128, T - 2, T - 1])
    c_rows, m_rows = c[:, :, rows.to(dev)].float().cpu(), m[:, :, rows.to(dev)].float().cpu()
    o, S = o.float().cpu(), S.cpu()
    q, k, v = w.q.float().cpu(), w.k.float().cpu(), w.v.float().cpu()
    zg, zb = w.zg.cpu(), w.zb.cpu()
    p = {a: b.float().cpu() for a, b in w.p.items()}
    del w, c, m
    n = torch.arange(1, T + 1, dtype=torch.float32)
    c_ref, m_ref = OP.polar_online(q[:, :, rows], k, v, n[rows], params=p, k_block=8192)
    assert rel_err(c_rows, c_ref) <= 2e-2, rel_err(c_rows, c_ref)
    assert rel_err(m_rows, m_ref) <= 2e-2, rel_err(m_rows, m_ref)
    kx, vx = (t.transpose(1, 2).repeat_interleave(HQ // HKV, 2) for t in (k, v))
    o_ref, S_ref = OG.chunk_gated_delta_rule(q.transpose(1, 2), kx, vx, F.logsigmoid(zg + 3.9), torch.sigmoid(zb),
                                             scale=1.0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert rel_err(o, o_ref) <= 2e-2, rel_err(o, o_ref)
    assert rel_err(S, S_ref) <= 2e-2, rel_err(S, S_ref)


# --------------------------------------------------------------------------- configs[3]
def _bench():
    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    import bench
    return bench


def test_configs3_graph_replay_equals_eager_and_oracle(dev):
    bench = _bench()
    _say("configs[3] decode step B=64 ctx~U[1024,32768]: graph replay vs eager vs oracle")
    eager = bench.Decode(torch, dev)
    graph = bench.Decode(torch, dev)        # same seed: identical pages, tables and inputs
    assert torch.equal(eager.table, graph.table) and torch.equal(eager.kc, graph.kc)
    graph.capture()                         # two warm-up steps, then the capture
    for _ in range(2):
        eager.step()
    torch.cuda.synchronize()
    bt, ctx = eager.bt.cpu(), eager.ctx.cpu()
    page = eager.kc.shape[1]
    sampled = sorted({int(ctx.argmax()), int(ctx.argmin()), 7, 41})
    p = {n: t.cpu() for n, t in eager.p.items()}
    slots = eager.slots.cpu()
    for step in range(3):
        rows_before = eager.table[eager.slots].cpu()
        c1, m1, r1 = eager.step()
        graph.replay()
        c2, m2, r2 = graph.graph_out
        torch.cuda.synchronize()
        assert torch.equal(c1, c2) and torch.equal(m1, m2) and torch.equal(r1, r2), step
        assert torch.equal(eager.table, graph.table), step
        assert torch.equal(eager.kc, graph.kc) and torch.equal(eager.vc, graph.vc), step
        # against the oracle on sampled sequences
        kn, vn = eager.knew.cpu(), eager.vnew.cpu()
        for b in sampled:
            n = int(ctx[b])
            npg = (n + page - 1) // page
            pages = bt[b, :npg].long()
            kc, vc = eager.kc[pages.to(dev)].cpu(), eager.vc[pages.to(dev)].cpu()
            last = n - 1
            assert torch.equal(kc[last // page, last % page], kn[b]) and \
                torch.equal(vc[last // page, last % page], vn[b]), (step, b)
            c_ref, m_ref = OP.polar_decode_paged(eager.q[b:b + 1].cpu().float(), kc.float(), vc.float(),
                                                 torch.arange(npg).view(1, -1), torch.tensor([n]), params=p)
            assert rel_err(c1[b:b + 1].cpu(), c_ref) <= 2e-2, (step, b)
            assert rel_err(m1[b:b + 1].cpu(), m_ref) <= 2e-2, (step, b)
        tab = rows_before.clone()   # (B, H, dk, dv) rows of this step's slots
        # grouped KV heads: query head h reads KV head h // (HQ // HKV)
        kx, vx = (t.cpu().repeat_interleave(HQ // HKV, 1) for t in (eager.knew, eager.vnew))
        r_ref = OG.gated_delta_decode_step(eager.q.cpu(), kx, vx, eager.gamma.cpu(), eager.beta.cpu(), tab,
                                           torch.arange(len(slots)))
        assert max_abs(r1.cpu(), r_ref) <= 2e-4, (step, max_abs(r1.cpu(), r_ref))
        assert max_abs(eager.table[eager.slots].cpu(), tab) <= 2e-5, step


# --------------------------------------------------------------------------- sharp scores
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [8.0, 16.0])
def test_sharp_scores_16bit_redo_path(dev, dtype, scale):
    from atma_amd.kernel import polar_attention_fwd
    _say(f"sharp scores {dtype} q x {scale}")
    B, T = 2, 777
    g = torch.Generator().manual_seed(int(scale))
    q = (torch.randn(B, HQ, T, D, generator=g) * scale).to(dtype)
    k, v = (torch.randn(B, HKV, T, D, generator=g).to(dtype) for _ in range(2))
    p = polar_params(HQ, D, seed=5)
    n = torch.arange(1, T + 1, dtype=torch.float32)
    c, m = polar_attention_fwd(q.to(dev), k.to(dev), v.to(dev), n.to(dev), **{a: b.to(dev) for a, b in p.items()})
    c, m = c.cpu(), m.cpu()
    assert torch.isfinite(c.float()).all() and torch.isfinite(m.float()).all()
    c_ref, m_ref = OP.polar_online(q.float(), k.float(), v.float(), n, params=p, k_block=256)
    assert rel_err(c, c_ref) <= 2e-2, rel_err(c, c_ref)
    assert rel_err(m, m_ref) <= 2e-2, rel_err(m, m_ref)

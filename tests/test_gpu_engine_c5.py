"""BASELINE configs[4] at its own shapes: the served 378M model through the paged engine.

``Atma(AtmaConfig())``: 16 blocks (4 global Polar + memory, 12 LFM2 conv), hidden 1,024,
head_dim 128 with 8 / 2 heads, squared-ReLU 4x MLP, vocab 50,304, 256-token KV pages.
Weights N(0, 0.02) from seed 0 as configs[4] states, except the RMSNorm gains, which are
set to 1 so that activations keep unit scale through the 16 blocks (with N(0, 0.02) gains
every logit is ~1e-2 and a comparison says little).

The pattern is ``tests/verify.py:549-617``, over every generated step: the oracle
(``oracle/model.atma_logits``, CPU) runs once per sequence on its final token history,
and, the model being causal, its logits at position p are the engine's logits of the step
that fed position p.

* fp32: two ragged prompts (300, 512 tokens: the per-sequence route) in one prefill
  batch and two equal ones (400, 400: the dense route) in the next, 3 greedy tokens each,
  decode replayed from the bucket-4 graph; every step's logits within 1e-4 of the fp64
  oracle.
* bf16 at the configs[4] workload: 32 prompts of 2,048 tokens (one dense prefill, the
  bucket-32 decode graph), 3 greedy tokens; the graph-replayed run equals the eager run
  bit for bit, and two sampled sequences agree with the fp32 oracle (on the bf16-rounded
  weights) at every step within 8e-2 relative (max|a-b| / max|b|); measured 3.6e-2 on
  sequence 0 and 5.2e-2 on sequence 21.  That is above the kernels' 2e-2 (and the
  reference's 5e-2 16-bit bar for one kernel, ``kernel/test_polar_kernel.py:119-128``)
  because every projection output, activation and the residual stream are stored in bf16
  through 16 blocks; the same model in fp32 through the same kernels and routes (above)
  is within 2.5e-5 of the oracle, so the gap is the storage precision's.
"""

import pytest
import torch

from oracle import model as OM
from tests.helpers import max_abs, rel_err

pytestmark = pytest.mark.gpu


def _model(dtype):
    from atma_amd.engine import Atma, AtmaConfig
    hf = AtmaConfig(dtype=dtype)
    m = Atma(hf).init_weights(0.02, 0)
    with torch.no_grad():
        for n, p in m.named_parameters():
            if n.endswith(("norm1.weight", "norm2.weight")) or n == "norm.weight":
                p.fill_(1.0)
    return hf, m


def _oracle_sd(model, dtype):
    return {k: v.detach().to("cpu", dtype).clone() for k, v in model.state_dict().items()}


def _engine(hf, model, *, max_seqs, budget, max_len, eager):
    from atma_amd.engine import Config, LLMEngine
    pages = max_seqs * ((max_len + 255) // 256) + 4
    cfg = Config(kvcache_block_size=256, max_num_seqs=max_seqs, max_num_batched_tokens=budget,
                 max_model_len=max_len, num_kvcache_blocks=pages, enforce_eager=eager, hf_config=hf)
    return LLMEngine(cfg, model=model)


def _drive(engine, prompts, new_tokens):
    """Step by hand; per step: (is_prefill, [(seq index, position fed last)], logits rows)."""
    from atma_amd.engine import SamplingParams
    sp = SamplingParams(temperature=0.0, max_tokens=new_tokens, ignore_eos=True)
    seqs = [engine.add_request(p, sp) for p in prompts]
    index = {s.seq_id: i for i, s in enumerate(seqs)}
    steps = []
    while not engine.is_finished():
        batch, is_prefill = engine.scheduler.schedule()
        where = [(index[s.seq_id], s.num_cached_tokens + s.num_scheduled_tokens - 1) for s in batch]
        toks = engine.model_runner.run(batch, is_prefill)
        steps.append((is_prefill, where, engine.model_runner.last_logits.float().cpu()))
        for s in engine.scheduler.commit(batch, toks):
            engine.model_runner.free_seq_slot(s)
    return seqs, steps


def _oracle_logits(hf, sd, tokens):
    kw = dict(num_layers=hf.num_hidden_layers, H=hf.num_attention_heads, Hkv=hf.num_key_value_heads,
              dk=hf.head_dim)
    with torch.no_grad():
        return OM.atma_logits(sd, torch.tensor(tokens)[None], **kw)[0]


def _prompts(lengths, seed, vocab):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, vocab, (n,), generator=g).tolist() for n in lengths]


def test_served_378m_fp32_every_step_matches_oracle(dev):
    hf, model = _model(torch.float32)
    engine = _engine(hf, model, max_seqs=4, budget=812, max_len=520, eager=False)
    prompts = _prompts([300, 512, 400, 400], 11, hf.vocab_size)
    seqs, steps = _drive(engine, prompts, new_tokens=3)
    engine.exit()
    routes = [(p, len(w)) for p, w, _ in steps]
    assert routes == [(True, 2), (True, 2), (False, 4), (False, 4)], routes
    sd = _oracle_sd(model, torch.float64)
    worst = 0.0
    for i, s in enumerate(seqs):
        ref = _oracle_logits(hf, sd, s.token_ids[:-1])
        for _, where, logits in steps:
            for row, (j, pos) in enumerate(where):
                if j == i:
                    err = max_abs(logits[row], ref[pos])
                    worst = max(worst, err)
                    assert err <= 1e-4, (i, pos, err)
    print(f"fp32 378M: worst max-abs logit error {worst:.2e}")


def test_served_378m_bf16_c5_workload_graph_equals_eager_and_matches_oracle(dev):
    hf, model = _model(torch.bfloat16)
    prompts = _prompts([2048] * 32, 0, hf.vocab_size)
    runs = []
    for eager in (True, False):
        engine = _engine(hf, model, max_seqs=32, budget=32 * 2048, max_len=2048 + 3, eager=eager)
        seqs, steps = _drive(engine, prompts, new_tokens=3)
        engine.exit()
        runs.append((seqs, steps))
        del engine
        torch.cuda.empty_cache()
    (seqs_e, steps_e), (seqs_g, steps_g) = runs
    assert [(p, len(w)) for p, w, _ in steps_g] == [(True, 32), (False, 32), (False, 32)]
    assert [s.completion_token_ids for s in seqs_e] == [s.completion_token_ids for s in seqs_g]
    assert all(torch.equal(a[2], b[2]) for a, b in zip(steps_e, steps_g))
    sd = _oracle_sd(model, torch.float32)
    worst = 0.0
    for i in (0, 21):
        ref = _oracle_logits(hf, sd, seqs_g[i].token_ids[:-1])
        for _, where, logits in steps_g:
            row = [j for j, _ in where].index(i)
            err = rel_err(logits[row], ref[where[row][1]])
            worst = max(worst, err)
            assert err <= 8e-2, (i, where[row][1], err)
    print(f"bf16 378M, 32 x 2048: worst relative logit error {worst:.2e}")

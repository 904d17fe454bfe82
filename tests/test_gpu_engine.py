"""The paged engine end to end on the GPU (BASELINE configs[4]'s path at a tiny size)
against the whole-model CPU oracle (``oracle/model.py``, ``model/reference.py:236-269``),
the ``tests/verify.py:549-617`` pattern extended to every step of a greedy generation.

At every prefill and decode step, each scheduled sequence's logits are compared with the
oracle's last-position logits over that sequence's full token history (the engine's own
greedy tokens, so an argmax near-tie cannot desynchronise the two): fp32 max-abs <= 1e-4
and the greedy token equal to the oracle's argmax unless the oracle's top-two gap is
below 1e-4.  bf16: max|a-b| / max|b| <= 5e-2, the reference's 16-bit bar
(``kernel/test_polar_kernel.py:119-128``): unlike the kernel tests (bf16 inputs, fp32
arithmetic, 2e-2), here every projection output, activation and the residual stream of
the whole model are rounded to bf16 through four blocks and the LM head.  Routes: dense (equal fresh prompts),
per-sequence (fp32 ragged), grouped tile-mapped Polar (bf16 ragged), graph-replayed
decode; the graph-replayed run equals the eager run bit for bit."""

import pytest
import torch

from oracle import model as OM
from tests.helpers import max_abs, rel_err

pytestmark = pytest.mark.gpu

TINY = dict(vocab_size=512, num_hidden_layers=4, hidden_size=256, head_dim=64)


def _model(dtype, seed=0):
    from atma_amd.engine import Atma, AtmaConfig
    hf = AtmaConfig(**TINY, dtype=dtype)
    m = Atma(hf).init_weights(0.05, seed)
    with torch.no_grad():
        for n, p in m.named_parameters():       # RMSNorm gains at 1 so activations keep their scale
            if n.endswith(("norm1.weight", "norm2.weight")) or n == "norm.weight":
                p.fill_(1.0)
    sd = {k: v.detach().double().clone() for k, v in m.state_dict().items()}
    return hf, m, sd


def _engine(hf, model, eager, max_num_seqs=4, pages=64):
    from atma_amd.engine import Config, LLMEngine
    cfg = Config(kvcache_block_size=16, max_num_seqs=max_num_seqs, max_num_batched_tokens=4096,
                 max_model_len=160, num_kvcache_blocks=pages, enforce_eager=eager, hf_config=hf)
    return LLMEngine(cfg, model=model)


def _drive(engine, prompts, new_tokens):
    """Step the engine by hand, recording each step's histories, logits and tokens."""
    from atma_amd.engine import SamplingParams
    sp = SamplingParams(temperature=0.0, max_tokens=new_tokens, ignore_eos=True)
    seqs = [engine.add_request(p, sp) for p in prompts]
    records = []
    while not engine.is_finished():
        batch, is_prefill = engine.scheduler.schedule()
        hist = [list(s.token_ids[:s.num_cached_tokens + s.num_scheduled_tokens]) for s in batch]
        toks = engine.model_runner.run(batch, is_prefill)
        records.append((is_prefill, hist, engine.model_runner.last_logits.float().cpu(), toks))
        for s in engine.scheduler.commit(batch, toks):
            engine.model_runner.free_seq_slot(s)
    return seqs, records


def _check_against_oracle(hf, sd, records, dtype):
    kw = dict(num_layers=hf.num_hidden_layers, H=hf.num_attention_heads, Hkv=hf.num_key_value_heads,
              dk=hf.head_dim)
    n = 0
    for is_prefill, hist, logits, toks in records:
        for row, (h, tok) in enumerate(zip(hist, toks)):
            ref = OM.atma_logits(sd, torch.tensor(h)[None], **kw)[0, -1]
            got = logits[row]
            if dtype == torch.float32:
                assert max_abs(got, ref) <= 1e-4, (is_prefill, len(h), max_abs(got, ref))
                top2 = ref.topk(2).values
                if (top2[0] - top2[1]).item() >= 1e-4:
                    assert tok == int(ref.argmax()), (is_prefill, len(h))
            else:
                assert rel_err(got, ref) <= 5e-2, (is_prefill, len(h), rel_err(got, ref))
            n += 1
    return n


def _prompts(lengths, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, TINY["vocab_size"], (n,), generator=g).tolist() for n in lengths]


@pytest.mark.parametrize("lengths", [[40, 40, 40], [17, 40, 33]], ids=["dense", "per_sequence"])
def test_engine_fp32_every_step_matches_oracle(dev, lengths):
    hf, model, sd = _model(torch.float32)
    engine = _engine(hf, model, eager=False)
    seqs, records = _drive(engine, _prompts(lengths, 1), new_tokens=6)
    assert records[0][0] and len(records[0][1]) == 3 and all(not r[0] for r in records[1:])
    assert _check_against_oracle(hf, sd, records, torch.float32) == 3 * 6
    assert all(len(s.completion_token_ids) == 6 for s in seqs)
    engine.exit()


@pytest.mark.parametrize("lengths", [[17, 40, 129], [48, 48]], ids=["grouped", "dense"])
def test_engine_bf16_every_step_matches_oracle(dev, lengths):
    hf, model, sd = _model(torch.bfloat16)
    engine = _engine(hf, model, eager=False)
    _, records = _drive(engine, _prompts(lengths, 2), new_tokens=5)
    # the oracle runs the bf16-rounded weights in fp64
    assert _check_against_oracle(hf, sd, records, torch.bfloat16) == len(lengths) * 5
    engine.exit()


def test_engine_graph_replay_equals_eager(dev):
    """Decode through captured HIP graphs (padded to the batch bucket, padding rows on the
    tables' spare row) == the same generation run eagerly, logits and tokens bit for bit;
    a sequence finishing early leaves a batch smaller than its bucket."""
    from atma_amd.engine import SamplingParams
    hf, model, _ = _model(torch.bfloat16, seed=3)
    prompts = _prompts([23, 50, 9], 3)
    out = []
    for eager in (True, False):
        engine = _engine(hf, model, eager=eager)
        sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True) for m in (7, 4, 7)]
        seqs = [engine.add_request(p, s) for p, s in zip(prompts, sps)]
        logits = []
        while not engine.is_finished():
            engine.step()
            logits.append(engine.model_runner.last_logits.clone())
        out.append(([s.completion_token_ids for s in seqs], logits))
        engine.exit()
    (tok_e, log_e), (tok_g, log_g) = out
    assert tok_e == tok_g
    assert len(log_e) == len(log_g) and all(torch.equal(a, b) for a, b in zip(log_e, log_g))


def test_pipelined_generate_equals_stepping(dev):
    """``generate``'s pipelined decode (each step launched before the previous step's tokens
    are read back, its input ids left on the device by that step's graph) == the same
    requests stepped one synchronous step at a time, token for token: ragged token limits
    end runs early, and an end-of-sequence id met mid-run drops the step launched behind it."""
    from atma_amd.engine import Config, LLMEngine, SamplingParams
    hf, model, _ = _model(torch.bfloat16, seed=5)
    prompts = _prompts([23, 50, 9, 31], 4)
    limits = (9, 5, 12, 12)

    def run(eos, pipelined):
        cfg = Config(kvcache_block_size=16, max_num_seqs=4, max_num_batched_tokens=4096, max_model_len=160,
                     num_kvcache_blocks=64, enforce_eager=False, hf_config=hf, eos=eos)
        engine = LLMEngine(cfg, model=model)
        sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=False) for m in limits]
        if pipelined:
            out = [r["token_ids"] for r in engine.generate(prompts, sps)]
        else:
            seqs = [engine.add_request(p, sp) for p, sp in zip(prompts, sps)]
            while not engine.is_finished():
                engine.step()
            out = [s.completion_token_ids for s in seqs]
        engine.exit()
        return out

    free = run(-1, False)                    # no end-of-sequence id
    assert run(-1, True) == free
    assert [len(t) for t in free] == list(limits)
    eos = free[2][6]                         # request 2 meets it at its 7th token, mid-run
    stepped = run(eos, False)
    assert len(stepped[2]) <= 7 and stepped[2][-1] == eos
    assert run(eos, True) == stepped


def test_pipelined_generate_with_queued_requests(dev):
    """Seven requests on four state rows: each pipelined run ends where a request finishes,
    the queued ones are admitted and prefilled, and decoding resumes in a new run -- the
    tokens equal stepping one synchronous step at a time."""
    from atma_amd.engine import Config, LLMEngine, SamplingParams
    hf, model, _ = _model(torch.bfloat16, seed=6)
    prompts = _prompts([23, 50, 9, 31, 12, 40, 17], 7)
    limits = (6, 3, 9, 4, 5, 8, 2)
    outs = []
    for pipelined in (False, True):
        cfg = Config(kvcache_block_size=16, max_num_seqs=4, max_num_batched_tokens=4096, max_model_len=160,
                     num_kvcache_blocks=64, enforce_eager=False, hf_config=hf)
        engine = LLMEngine(cfg, model=model)
        sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True) for m in limits]
        if pipelined:
            outs.append([r["token_ids"] for r in engine.generate(prompts, sps)])
        else:
            seqs = [engine.add_request(p, sp) for p, sp in zip(prompts, sps)]
            while not engine.is_finished():
                engine.step()
            outs.append([s.completion_token_ids for s in seqs])
        engine.exit()
    assert outs[0] == outs[1]
    assert [len(t) for t in outs[0]] == list(limits)


def test_generate_reports_throughput(dev):
    hf, model, _ = _model(torch.bfloat16, seed=4)
    engine = _engine(hf, model, eager=False)
    from atma_amd.engine import SamplingParams
    res = engine.generate(_prompts([32, 32, 32, 32], 5), SamplingParams(temperature=0.0, max_tokens=8,
                                                                         ignore_eos=True))
    assert [len(r["token_ids"]) for r in res] == [8] * 4
    m = engine.last_metrics
    assert m["prefill_tokens"] == 128 and m["decode_tokens"] == 4 * 7
    assert m["prefill_throughput"] > 0 and m["decode_throughput"] > 0
    engine.exit()


def test_tight_page_pool_runs_requests_in_turn_with_the_same_tokens(dev):
    """A pool that holds one request's lifetime pages at a time: the others wait queued,
    then reuse the freed pages and state-table rows (zeroed on release).  Each request's
    tokens equal those of a fresh engine serving it alone (the same batch of one, the same
    routes): no request sees another's KV pages, conv tails or memory state."""
    from atma_amd.engine import SamplingParams
    hf, model, _ = _model(torch.bfloat16, seed=6)
    prompts = _prompts([30, 45, 21], 7)
    sp = SamplingParams(temperature=0.0, max_tokens=6, ignore_eos=True)
    alone = []
    for p in prompts:
        engine = _engine(hf, model, eager=False, pages=64)
        alone.append(engine.generate([p], sp)[0]["token_ids"])
        engine.exit()
    engine = _engine(hf, model, eager=False, pages=4)   # 4 pages = 64 tokens: one request's 51 at most
    seqs = [engine.add_request(p, sp) for p in prompts]
    while not engine.is_finished():
        batch, is_prefill = engine.scheduler.schedule()
        assert len(batch) == 1                          # one request at a time
        toks = engine.model_runner.run(batch, is_prefill)
        for s in engine.scheduler.commit(batch, toks):
            engine.model_runner.free_seq_slot(s)
    engine.exit()
    assert [s.completion_token_ids for s in seqs] == alone

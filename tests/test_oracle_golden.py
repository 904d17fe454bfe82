"""The oracle's block and model glue against tensors written by the reference's own modules.

``tests/golden/block_glue.pt`` holds the outputs of the reference's ``PolarAttention``,
``TitansMemory``, ``MLP``, ``LFM2Conv``, ``Block`` and a 4-block ``ReferenceModel``
(``model/reference.py``, ``model/layers.py``, ``model/blocks.py``) on seeded inputs, written by
``tests/golden/make_block_fixtures.py`` in the build container.  The parameters and inputs
are rebuilt here from the stored names, shapes and seeds.

These pin the conventions no closed form reaches: the q / gate split
(``model/reference.py:131-132``), the combine ``proj(c * sigmoid(gate)) + mu_proj(mag)``
(``:183-191``), the memory branch's biases, norms and output gate (``model/blocks.py:463-490``),
the MLP's value / gate order (``model/layers.py:27-31``), the LFM2 ``B, C, x`` split
(``model/reference.py:37-48``), the pre-norm residuals (``:226-229``) and the final norm, LM
head and soft cap (``:262-269``).

Bars: fp64 paths agree to 1e-10 relative (the same arithmetic, summed in another order);
fp32 paths to 5e-6 relative (the reference computes the memory branch and the logits in
fp32, the oracle's chunked scan groups its sums differently).  A swapped convention moves
every output by O(1).
"""

import os
import sys

import pytest
import torch

from oracle import block as OB
from oracle import model as OM

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from make_block_fixtures import input_value, param_value  # noqa: E402

FIXTURES = os.path.join(HERE, "golden", "block_glue.pt")


@pytest.fixture(scope="module")
def fx():
    return torch.load(FIXTURES, weights_only=True)


def _sd(params, dtype):
    prefix = params.get("prefix", "")
    return {prefix + n: param_value(prefix + n, s, params["seed"], dtype)
            for n, s in zip(params["names"], params["shapes"])}


def _x(fx, case, dtype):
    m = fx["meta"]
    return input_value((m["batch"], m["seq"], m["dim"]), case["x_seed"], dtype)


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max()).item()


def _heads(fx):
    m = fx["meta"]
    return dict(H=m["heads"], Hkv=m["kv_heads"], dk=m["head_dim"])


@pytest.mark.parametrize("window", [None, 8])
def test_polar_attention_fp64_matches_reference(fx, window):
    case = fx[f"polar_w{window or 0}_f64"]
    sd = _sd(case["params"], torch.float64)
    with torch.no_grad():
        y = OB.polar_attention(sd, _x(fx, case, torch.float64), window=window, mem=False, native_eps=True,
                               **_heads(fx))
    assert _rel(y, case["y"]) < 1e-10


def test_polar_attention_with_memory_fp32_matches_reference(fx):
    case = fx["polar_mem_f32"]
    sd = _sd(case["params"], torch.float32)
    with torch.no_grad():
        y = OB.polar_attention(sd, _x(fx, case, torch.float32), mem=True, **_heads(fx))
    assert _rel(y, case["y"]) < 5e-6


def test_memory_branch_fp32_matches_reference(fx):
    case = fx["titans_f32"]
    m = fx["meta"]
    sd = _sd(case["params"], torch.float32)
    q, k, v = (input_value((m["batch"], m["heads"], m["seq"], m["head_dim"]), s, torch.float32)
               for s in case["qkv_seeds"])
    with torch.no_grad():
        y, _ = OB.memory_branch(sd, _x(fx, case, torch.float32), q, k, v)
    assert _rel(y, case["y"]) < 5e-6


def test_mlp_fp64_matches_reference(fx):
    case = fx["mlp_f64"]
    sd = _sd(case["params"], torch.float64)
    with torch.no_grad():
        y = OB.mlp({"mlp." + n: t for n, t in sd.items()}, _x(fx, case, torch.float64))
    assert _rel(y, case["y"]) < 1e-10


def test_lfm2_conv_fp64_matches_reference(fx):
    case = fx["lfm2_f64"]
    sd = _sd(case["params"], torch.float64)
    with torch.no_grad():
        y = OM.lfm2_conv(sd, _x(fx, case, torch.float64))
    assert _rel(y, case["y"]) < 1e-10


def test_global_block_fp32_matches_reference(fx):
    case = fx["block_global_f32"]
    sd = _sd(case["params"], torch.float32)
    with torch.no_grad():
        y = OB.global_block(sd, _x(fx, case, torch.float32), mem=True, **_heads(fx))
    assert _rel(y, case["y"]) < 5e-6


def test_conv_block_fp64_matches_reference(fx):
    case = fx["block_conv_f64"]
    sd = _sd(case["params"], torch.float64)
    with torch.no_grad():
        y = OM.conv_block(sd, _x(fx, case, torch.float64))
    assert _rel(y, case["y"]) < 1e-10


def test_model_logits_fp32_match_reference(fx):
    case = fx["model_f32"]
    sd = _sd(case["params"], torch.float32)
    with torch.no_grad():
        logits = OM.atma_logits(sd, case["ids"], num_layers=case["num_layers"], mem=True, **_heads(fx))
    assert logits.dtype == torch.float32
    assert _rel(logits, case["logits"]) < 5e-6


def test_product_modules_take_the_reference_parameter_names(fx):
    """The host layer's modules register the reference's parameter names in its order, so a
    checkpoint of the reference loads into them strictly."""
    from atma_amd.layers.global_attention import MLP, GlobalBlock
    m = fx["meta"]
    blk = GlobalBlock(m["dim"], head_dim=m["head_dim"], window=None)
    assert [n for n, _ in blk.named_parameters()] == fx["block_global_f32"]["params"]["names"]
    assert [n for n, _ in MLP(m["dim"]).named_parameters()] == fx["mlp_f64"]["params"]["names"]


def test_engine_model_takes_the_reference_parameter_names(fx):
    """The served model holds ``ReferenceModel``'s parameter names and shapes, so a reference
    checkpoint loads into it strictly.  (Only the order of ``norm`` and ``proj`` differs: the
    served model registers them as the reference's engine does, ``inference/models/atma.py:738-739``,
    the training model the other way round, ``model/reference.py:258-259``; loading is by key.)"""
    from atma_amd.engine.config import AtmaConfig
    from atma_amd.engine.model import Atma
    case, m = fx["model_f32"], fx["meta"]
    model = Atma(AtmaConfig(vocab_size=case["vocab"], num_hidden_layers=case["num_layers"],
                            hidden_size=m["dim"], head_dim=m["head_dim"]))
    got = {n: list(p.shape) for n, p in model.named_parameters()}
    assert got == dict(zip(case["params"]["names"], case["params"]["shapes"]))

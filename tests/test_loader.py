"""Checkpoint format of the reference (``train.py:115-133``: ``{"model": sd}`` with
``_orig_mod.`` stripped; ``inference/utils/loader.py:5-39``): a block of a full-model
checkpoint loads into the global-layer modules by its prefix, compiled-model keys load
after stripping, ``strict`` raises on a layout mismatch, and the file is read without
unpickling code (weights_only)."""

import pytest
import torch

from atma_amd.layers import GlobalBlock, load_model, save_checkpoint


def _block(seed):
    torch.manual_seed(seed)
    b = GlobalBlock(256, head_dim=64)
    with torch.no_grad():
        for p in b.parameters():
            p.normal_(0.0, 0.02)
    return b


def test_block_prefix_roundtrip(tmp_path):
    src = _block(0)
    path = tmp_path / "weights.pt"
    other = {"_orig_mod.blocks.0.attn.q.weight": torch.zeros(3), "embed.weight": torch.zeros(2)}
    sd = {"_orig_mod.blocks.2." + k: v for k, v in src.state_dict().items()}
    torch.save({"model": {**other, **sd}}, path)
    dst = load_model(_block(1), str(path), strict=True, prefix="blocks.2.")
    for (k, a), (_, b) in zip(src.state_dict().items(), dst.state_dict().items()):
        assert torch.equal(a, b), k
    attn = load_model(_block(1).attn, path, strict=True, prefix="blocks.2.attn.")
    assert torch.equal(attn.v_null, src.attn.v_null) and torch.equal(attn.mem.proj.weight, src.attn.mem.proj.weight)


def test_save_then_load_and_strict_mismatch(tmp_path):
    src = _block(2)
    path = tmp_path / "w.pt"
    save_checkpoint(src, path, prefix="blocks.5.")
    raw = torch.load(path, weights_only=True)
    assert set(raw) == {"model"} and all(k.startswith("blocks.5.") for k in raw["model"])
    dst = load_model(_block(3), path, prefix="blocks.5.")
    assert torch.equal(dst.mlp.fc.weight, src.mlp.fc.weight)
    with pytest.raises(RuntimeError, match="layout mismatch"):
        load_model(_block(3), path, strict=True, prefix="blocks.4.")

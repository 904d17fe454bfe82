"""Checkpoint loading for the global-layer modules.

The reference saves ``weights.pt`` as ``{"model": state_dict}`` with torch.compile's
``_orig_mod.`` prefix stripped (``train.py:115-133``) and loads it with
``load_model`` (``inference/utils/loader.py:5-39``): unwrap ``"model"``, strip
``_orig_mod.``, ``load_state_dict(strict=False)``, raise on a layout mismatch only when
``strict``.  The modules here register their parameters under the reference's names
(``blocks.{i}.attn.*``, ``blocks.{i}.mlp.*``, ``blocks.{i}.norm{1,2}.*``), so one block
of a full-model checkpoint loads by its prefix.  Files are read with
``torch.load(weights_only=True)``: nothing in a checkpoint is executed.
"""

import torch
from torch import nn


def read_state_dict(path_or_state_dict):
    """The checkpoint's tensors with ``_orig_mod.`` stripped from every key."""
    if isinstance(path_or_state_dict, (str, bytes)) or hasattr(path_or_state_dict, "__fspath__"):
        sd = torch.load(path_or_state_dict, map_location="cpu", weights_only=True)
        if isinstance(sd, dict) and "model" in sd:
            sd = sd["model"]
    else:
        sd = path_or_state_dict
    return {k.removeprefix("_orig_mod."): v for k, v in sd.items()}


def load_model(model: nn.Module, path_or_state_dict, *, strict: bool = False, prefix: str = "") -> nn.Module:
    """``inference/utils/loader.py:5-39`` for a module of this package.  ``prefix`` (e.g.
    ``"blocks.2."`` for a GlobalBlock, ``"blocks.2.attn."`` for a PolarAttention) selects
    one block of a full-model checkpoint; keys outside it are ignored.  Returns the model;
    with ``strict`` a missing or unexpected key raises RuntimeError."""
    sd = read_state_dict(path_or_state_dict)
    if prefix:
        sd = {k[len(prefix):]: v for k, v in sd.items() if k.startswith(prefix)}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    if strict and (missing or unexpected):
        raise RuntimeError(f"checkpoint layout mismatch: missing={missing}, unexpected={unexpected}")
    return model


def save_checkpoint(model: nn.Module, path, prefix: str = ""):
    """Write ``{"model": state_dict}`` as ``train.py:115-121`` does (CPU tensors,
    ``_orig_mod.`` stripped), with every key under ``prefix``."""
    sd = {prefix + k.removeprefix("_orig_mod."): v.detach().cpu() for k, v in model.state_dict().items()}
    torch.save({"model": sd}, path)

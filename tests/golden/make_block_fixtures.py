"""Write golden tensors for the oracle's block and model glue from the reference itself.

BUILD CONTAINER ONLY.  This script imports the reference's pure-PyTorch modules
(``model/reference.py``, ``model/layers.py``, ``model/blocks.py``) from the reference
checkout (default ``/root/reference``, or ``$ATMA_REFERENCE``), runs them on small
seeded inputs on the CPU, and writes tensors only: the reference's outputs, with the
parameter names and shapes and the seeds from which the test rebuilds the inputs and
parameters (``param_value``, ``input_value``), all
loadable with ``torch.load(..., weights_only=True)``.  Nothing of the reference is
copied; the fixtures are data.  The GPU box never runs this script (the reference is
absent there); the CPU test ``tests/test_oracle_golden.py`` reads what it wrote.

What the fixtures pin, and why only an import can pin it: the conventions of the
glue around the kernels -- the q / gate split of the q projection
(``model/reference.py:131-132``), the combine ``proj(c * sigmoid(gate)) + mu_proj(mag)``
(``:183-191``), the memory branch's gate biases, l2 norm, readout RMSNorm and output
gate (``model/blocks.py:463-490``), the MLP's value / gate order
(``model/layers.py:27-31``), the LFM2 conv's ``B, C, x`` split (``model/reference.py:37-48``),
the block's pre-norm residuals (``:226-229``), and the model's final norm, LM head and
soft cap (``:262-269``).  Swapping any of those orders leaves every closed form and
invariant of the kernels intact, so no mathematical pin sees it.

Parameters: every tensor N(0, 0.02) (the reference tests' convention,
``tests/test_dense_prefill.py:105-106``), except the five Polar scalars, which are N(0, 1)
so the temperature, null sink and magnitude are exercised away from their priors, and
the RMSNorm weights, which are 1 + N(0, 0.02) so that activations keep unit scale.

Run:  python tests/golden/make_block_fixtures.py   (writes tests/golden/block_glue.pt)
"""

import os
import sys
import zlib

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "block_glue.pt")

_POLAR_SCALARS = ("v_null", "null_base", "null_slope_raw", "len_gain_raw", "mag_beta_raw")


def param_value(name, shape, seed, dtype):
    """The value of parameter ``name``: a pure function of (seed, name, shape), so the
    test rebuilds every state dict from the stored names and shapes alone."""
    g = torch.Generator().manual_seed(seed * 1_000_003 + zlib.crc32(name.encode()))
    noise = torch.randn(tuple(shape), generator=g, dtype=torch.float64)
    leaf = name.rsplit(".", 1)[-1]
    if leaf in _POLAR_SCALARS:
        return noise.to(dtype)
    if ("." + name).rsplit(".", 2)[-2].startswith("norm") and leaf == "weight" and len(shape) == 1:
        return (1.0 + 0.02 * noise).to(dtype)
    return (0.02 * noise).to(dtype)


def _init(mod, seed):
    with torch.no_grad():
        for name, p in mod.named_parameters():
            p.copy_(param_value(name, p.shape, seed, p.dtype))
    return {"seed": seed, "names": [n for n, _ in mod.named_parameters()],
            "shapes": [list(p.shape) for _, p in mod.named_parameters()]}


def input_value(shape, seed, dtype):
    """A seeded N(0, 1) input, rebuilt by the test from (shape, seed, dtype)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn(tuple(shape), generator=g, dtype=torch.float64).to(dtype)


def _x(shape, seed, dtype):
    return input_value(shape, seed, dtype)


def main():
    ref_root = os.environ.get("ATMA_REFERENCE", "/root/reference")
    sys.path.insert(0, ref_root)
    from model.config import AtmaConfig
    from model.layers import MLP
    from model.reference import Block, LFM2Conv, Linear, PolarAttention, ReferenceModel

    torch.set_num_threads(min(8, os.cpu_count() or 1))
    dim, dk, B, T = 256, 64, 2, 40
    fx = {"meta": {"dim": dim, "head_dim": dk, "heads": dim // dk, "kv_heads": dim // dk // 4,
                   "batch": B, "seq": T}}

    # 1. PolarAttention without the memory branch, fp64 (no fp32 step anywhere on this path)
    for window in (None, 8):
        mod = PolarAttention(dim, head_dim=dk, window=window, mem_enabled=False).double()
        params = _init(mod, seed=10)
        x = _x((B, T, dim), 11, torch.float64)
        with torch.no_grad():
            y = mod(x)
        fx[f"polar_w{window or 0}_f64"] = {"params": params, "x_seed": 11, "y": y}

    # 2. PolarAttention with the torch memory branch, fp32 (the branch computes in fp32
    #    whatever the input dtype: model/blocks.py:465-467,481-483)
    mod = PolarAttention(dim, head_dim=dk, window=None, mem_enabled=True, mem_chunk=16,
                         mem_kernel="torch").float()
    params = _init(mod, seed=20)
    x = _x((B, T, dim), 21, torch.float32)
    with torch.no_grad():
        y = mod(x)
    fx["polar_mem_f32"] = {"params": params, "x_seed": 21, "y": y}

    # 3. the memory branch alone on given (B, H, T, dk) inputs, fp32
    H = dim // dk
    mem = mod.mem
    q_t, k_t, v_t = (_x((B, H, T, dk), s, torch.float32) for s in (30, 31, 32))
    with torch.no_grad():
        y = mem(x, q_t, k_t, v_t)
    params = {"seed": 20, "names": [n[4:] for n in params["names"] if n.startswith("mem.")],
              "shapes": [s for n, s in zip(params["names"], params["shapes"]) if n.startswith("mem.")],
              "prefix": "mem."}
    fx["titans_f32"] = {"params": params, "x_seed": 21, "qkv_seeds": [30, 31, 32], "y": y}

    # 4. MLP and LFM2 conv, fp64
    mlp = MLP(dim, linear_cls=Linear).double()
    params = _init(mlp, seed=40)
    x = _x((B, T, dim), 41, torch.float64)
    with torch.no_grad():
        fx["mlp_f64"] = {"params": params, "x_seed": 41, "y": mlp(x)}
    conv = LFM2Conv(dim, kernel_size=3).double()
    params = _init(conv, seed=50)
    x = _x((B, T, dim), 51, torch.float64)
    with torch.no_grad():
        fx["lfm2_f64"] = {"params": params, "x_seed": 51, "y": conv(x)}

    # 5. whole blocks: global (memory on, fp32) and conv (fp64)
    blk = Block(dim, attention=True, head_dim=dk, attn_window=None, mem_enabled=True, mem_chunk=16,
                mem_kernel="torch").float()
    params = _init(blk, seed=60)
    x = _x((B, T, dim), 61, torch.float32)
    with torch.no_grad():
        fx["block_global_f32"] = {"params": params, "x_seed": 61, "y": blk(x)}
    blk = Block(dim, attention=False, conv_kernel_size=3).double()
    params = _init(blk, seed=70)
    x = _x((B, T, dim), 71, torch.float64)
    with torch.no_grad():
        fx["block_conv_f64"] = {"params": params, "x_seed": 71, "y": blk(x)}

    # 6. a 4-block model (Local-Local-Global-Local), fp32, memory on, no window
    cfg = AtmaConfig(vocab_size=97, num_hidden_layers=4, hidden_size=dim, head_dim=dk,
                     attn_window=None, mem_enabled=True, mem_chunk=16, mem_kernel="torch",
                     attn_kernel="torch", dtype=torch.float32)
    model = ReferenceModel(cfg).float()
    params = _init(model, seed=80)
    g = torch.Generator().manual_seed(81)
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=g)
    with torch.no_grad():
        logits = model(ids)
    fx["model_f32"] = {"params": params, "ids": ids, "logits": logits,
                       "num_layers": cfg.num_hidden_layers, "vocab": cfg.vocab_size}

    torch.save(fx, OUT)
    print(f"wrote {OUT}: {sorted(k for k in fx if k != 'meta')}")


if __name__ == "__main__":
    main()

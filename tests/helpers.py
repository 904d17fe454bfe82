"""Shared test helpers (tolerances, seeded parameters)."""

import torch


def rel_err(a, b):
    """max|a-b| / max|b| (the stricter per-tensor form of the bf16 bar)."""
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def max_abs(a, b):
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def polar_params(H, d, *, seed=0, prior=False, dtype=torch.float32, device="cpu"):
    """Polar parameters: the reference priors (model/reference.py:17-20) or N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    if prior:
        p = dict(v_null=torch.randn(H, d, generator=g) * 0.1,
                 null_base=torch.full((H,), 2.0), null_slope_raw=torch.full((H,), 0.5),
                 len_gain_raw=torch.full((H,), -1.0), mag_beta_raw=torch.full((H,), -1.5))
    else:
        p = {n: torch.randn(*s, generator=g) for n, s in
             (("v_null", (H, d)), ("null_base", (H,)), ("null_slope_raw", (H,)),
              ("len_gain_raw", (H,)), ("mag_beta_raw", (H,)))}
    return {n: t.to(device=device, dtype=dtype) for n, t in p.items()}

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


def bwd16_chain_reference(kr, kt, qt, tm, tt, rt, vt, ot, got, f, s0, dst):
    """fp32 torch restatement of ``gated_delta_bwd16_chain`` on the same tiles (the
    kernel's products round their right operand -- the state, Y, U, dU, dY -- to 16 bits;
    this one does not).  Forward chain: Y = diag(beta)(V - diag(Ga) K S),
    S <- Ga_C S + K^T diag(w) T Y; backward chain: dU = diag(w) K dS + Rq^T dO,
    dY = T^T dU, dS <- Ga_C dS + Q^T (Ga dO) - K^T diag(Ga beta) dY.
    Returns (s_entry, ds_end, dy, ds0) as the op does."""
    BH, NC, C, D = kr.shape
    F = lambda x: x.float()  # noqa: E731
    o = dict(device=kr.device, dtype=torch.float32)
    S = torch.zeros(BH, D, D, **o) if s0 is None else s0.float().clone()
    s_entry, ds_end = torch.empty(BH, NC, D, D, **o), torch.empty(BH, NC, D, D, **o)
    dy = torch.empty(BH, NC, C, D, **o)
    for c in range(NC):
        Ga, w, b, GaC = f[:, c, 0], f[:, c, 1], f[:, c, 2], f[:, c, 3, :1, None]
        s_entry[:, c] = S
        Y = b[..., None] * (F(vt[:, c]).transpose(-1, -2) - Ga[..., None] * (F(kr[:, c]) @ S))
        S = GaC * S + F(kt[:, c]) @ (w[..., None] * (F(tm[:, c]) @ Y))
    dS = torch.zeros(BH, D, D, **o) if dst is None else dst.float().clone()
    for c in reversed(range(NC)):
        Ga, w, b, GaC = f[:, c, 0], f[:, c, 1], f[:, c, 2], f[:, c, 3, :1, None]
        ds_end[:, c] = dS
        dU = w[..., None] * (F(kr[:, c]) @ dS) + F(rt[:, c]) @ F(ot[:, c]).transpose(-1, -2)
        dY = F(tt[:, c]) @ dU
        dy[:, c] = dY
        dS = GaC * dS + F(qt[:, c]) @ F(got[:, c]).transpose(-1, -2) - F(kt[:, c]) @ ((Ga * b)[..., None] * dY)
    return s_entry, ds_end, dy, dS

"""Seeded inputs and checks shared by the GPU parity tests.

Inputs are drawn on the CPU from a torch.Generator and moved to the device,
as the reference's kernel tests do (kernel/test_fused_attn.py:24-37, :113-115).
"""
import math

import numpy as np
import torch

from oracle import saf_oracle as orc

ATOL = 2e-2      # bf16/fp16 attention output max-abs bound (north_star)
RTOL_L2 = 1e-2   # ... and relative-L2 bound


def make_pattern(n, S, seed):
    """Random lower-triangular row-stochastic (n, S, S) patterns
    (kernel/test_fused_attn.py:24-27)."""
    g = torch.Generator().manual_seed(seed)
    p = torch.rand(n, S, S, generator=g).tril()
    return p / p.sum(-1, keepdim=True).clamp(min=1e-9)


def make_decomp(H, S, seed, scale=0.8):
    """Random alpha/rho (H, S) and their normaliser z computed in float64 and
    stored in fp32 (kernel/test_fused_attn.py:30-37)."""
    g = torch.Generator().manual_seed(seed)
    alpha = torch.randn(H, S, generator=g) * scale
    rho = torch.randn(H, S, generator=g) * scale
    z = torch.from_numpy(orc.decomposed_logz(alpha.numpy(), rho.numpy())).float()
    return alpha, rho, z


def closed_params(H, S, kinds):
    """alpha/rho/z (fp32, (H, S)) for heads with closed-form kinds
    {h: ("mean"|"decay"|"window", param)}; other rows are zero."""
    alpha = np.zeros((H, S))
    rho = np.zeros((H, S))
    for h, (kind, prm) in kinds.items():
        alpha[h], rho[h] = orc.closed_form_params(kind, prm, S)
    z = orc.decomposed_logz(alpha, rho)
    f = lambda a: torch.from_numpy(a).float()
    # rho's -inf entries survive the fp32 cast; z is finite for every row
    return f(alpha), f(rho), f(z)


def compare(y, ref, atol=ATOL, rtol_l2=RTOL_L2, what=""):
    y = y.detach().float().cpu().numpy().astype(np.float64)
    assert y.shape == ref.shape, (y.shape, ref.shape)
    assert np.isfinite(y).all(), f"{what}: non-finite output"
    err = np.abs(y - ref)
    max_abs = float(err.max()) if err.size else 0.0
    denom = float(np.linalg.norm(ref)) or 1.0
    rel = float(np.linalg.norm(y - ref)) / denom
    assert max_abs <= atol and rel <= rtol_l2, \
        f"{what}: max_abs={max_abs:.3e} (<= {atol}) rel_l2={rel:.3e} (<= {rtol_l2})"
    return max_abs, rel


def routing(H, states):
    """frozen / hidx int32 tables for {head: state} (others live)."""
    frozen = torch.zeros(H, dtype=torch.int32)
    for h, s in states.items():
        frozen[h] = s
    live = [h for h in range(H) if int(frozen[h]) == 0]
    hidx = torch.zeros(H, dtype=torch.int32)
    for slot, h in enumerate(live):
        hidx[h] = slot
    return frozen, hidx, live


def qkv(B, H, T, hd, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    base = [torch.randn(B, H, T, hd, generator=g) for _ in range(3)]
    return [t.to(dtype) for t in base]


def f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def scale_of(hd):
    return 1.0 / math.sqrt(hd)

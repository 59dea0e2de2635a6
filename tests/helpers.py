"""Shared input generators and comparison helpers for the tests (seeded, CPU-side)."""

from __future__ import annotations

import torch


def addresses(B, T, R, seed, dtype=torch.float32, dist="normal", nu=3.0):
    """(B,T,R) query and key addresses ~ N(0,1)/sqrt(R) (or Student-t(nu)/sqrt(R)),
    generated in fp32 on the CPU and cast, so every consumer sees identical bits."""
    g = torch.Generator().manual_seed(seed)
    if dist == "normal":
        qa = torch.randn(B, T, R, generator=g)
        ka = torch.randn(B, T, R, generator=g)
    elif dist == "student_t":
        # t = z / sqrt(chi2_nu / nu), chi2 from a sum of squared normals
        def t_sample():
            z = torch.randn(B, T, R, generator=g)
            c = (torch.randn(int(nu), B, T, R, generator=g) ** 2).sum(0)
            return z / torch.sqrt(c / nu)
        qa, ka = t_sample(), t_sample()
    else:
        raise ValueError(dist)
    return (qa / R ** 0.5).to(dtype), (ka / R ** 0.5).to(dtype)


def qkv(B, H, T, D, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(B, H, T, D, generator=g).to(dtype) for _ in range(3))


def plant(qa, ka, frac, seed, factor=4.0):
    """Set ka[b, j] = factor * qa[b, i] for a seeded `frac` of key positions j, with i
    uniform in [j, T): the planted key is a sharp winner for query i."""
    g = torch.Generator().manual_seed(seed)
    B, T, _ = ka.shape
    ka = ka.clone()
    n = max(1, int(frac * T))
    plants = []
    for b in range(B):
        js = torch.randperm(T, generator=g)[:n]
        for j in js.tolist():
            i = int(torch.randint(j, T, (1,), generator=g))
            ka[b, j] = (factor * qa[b, i].float()).to(ka.dtype)
            plants.append((b, i, j))
    return ka, plants


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """Norm-wise relative error ||a - b||_inf / ||b||_inf (in float64)."""
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0)

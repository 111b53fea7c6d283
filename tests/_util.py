"""Shared helpers for the parity tests (seeded synthetic inputs, error metrics)."""
from __future__ import annotations

import numpy as np
import torch


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def synth(seed, R, C, G, N, T, x_dtype=torch.float16, outliers=8, gscale=1e-4, wscale=0.02):
    """BASELINE-style synthetic inputs: X ~ N(0,1) with outlier channels x20, W ~ N(0, wscale^2),
    saliency ~ LogNormal(0,1) clipped at its 0.99 quantile per group, G ~ N(0, gscale^2)."""
    r = rng(seed)
    X = r.standard_normal((N, T, C), dtype=np.float32)
    X[:, :, r.choice(C, min(outliers, C), replace=False)] *= 20.0
    W = r.standard_normal((R, C), dtype=np.float32) * wscale
    s = r.lognormal(0.0, 1.0, size=(N, T, G)).astype(np.float32)
    for g in range(G):
        s[..., g] = np.minimum(s[..., g], np.quantile(s[..., g], 0.99))
    grad = r.standard_normal((R, C), dtype=np.float32) * gscale
    return (torch.from_numpy(X).to(x_dtype), torch.from_numpy(W).to(torch.float16),
            torch.from_numpy(s), torch.from_numpy(grad))


def rel_fro(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    den = b.norm()
    return float((a - b).norm() / (den if den > 0 else 1.0))


def code_flips(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return int((a != b).sum())

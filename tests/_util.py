"""Shared helpers for the parity tests (seeded synthetic inputs, error metrics)."""
from __future__ import annotations

import json
import os

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


def w_rel_fro(a, b):
    """||a - b||_F / ||b||_F of two weight tensors in float64, on a's device (the dequantized weights
    the north star compares; each flipped code moves one weight by a quantisation step)."""
    a = a.detach()
    b = b.detach().to(a.device)
    den = b.double().norm()
    return float((a.double() - b.double()).norm() / (den if den > 0 else 1.0))


def code_flips(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return int((a != b).sum())


def flip_report(codes_gpu, codes_ref, ratio, perm=None):
    """Where two code tensors differ, how far the reference's rounded value r = w / scale (the
    oracle's ``record_ratio``; torch.round rounds half to even, quant_utils.py:477) lies from
    the nearest rounding midpoint k + 1/2.  An exact tie is r == k + 1/2; otherwise the
    distance is counted in units of the fp32 spacing at |r| (ulps).  With ``perm`` (the
    act_order column order, in which the column loop quantizes) the first flip of each row is
    "primary"; the later ones follow the different error feedback an earlier flip of their row
    causes, and are reported apart."""
    a = codes_gpu.detach().cpu().to(torch.float64)
    b = codes_ref.detach().cpu().to(torch.float64)
    r = ratio.detach().cpu().to(torch.float32)
    if perm is not None:
        p = perm.detach().cpu()
        a, b, r = a[:, p], b[:, p], r[:, p]
    diff = (a != b)
    out = {"flips": int(diff.sum())}
    if out["flips"] == 0:
        out.update(exact_ties=0, primary=0)
        return out
    first = diff.cumsum(1) == 1
    primary = diff & first

    def dist(mask):
        rv = r[mask].numpy().astype(np.float32)
        d = np.abs(rv.astype(np.float64) - (np.floor(rv.astype(np.float64)) + 0.5))
        ulp = np.spacing(np.abs(rv)).astype(np.float64)
        return d, d / ulp

    d_all, u_all = dist(diff)
    d_pri, u_pri = dist(primary)
    out.update(
        exact_ties=int((d_all == 0).sum()),
        primary=int(primary.sum()),
        primary_exact_ties=int((d_pri == 0).sum()),
        primary_ulps_le_1=int((u_pri <= 1).sum()), primary_ulps_le_16=int((u_pri <= 16).sum()),
        primary_ulps_le_256=int((u_pri <= 256).sum()), primary_ulps_le_4096=int((u_pri <= 4096).sum()),
        primary_ulps_median=float(np.median(u_pri)), primary_ulps_max=float(u_pri.max()),
        primary_dist_max=float(d_pri.max()),
        all_ulps_median=float(np.median(u_all)), all_dist_max=float(d_all.max()),
        code_delta_max=int((a - b).abs().max()))
    return out


def log_parity(rec):
    """Print one case's numbers and, when RQ_PARITY_LOG names a file, append them to it as JSON."""
    print(json.dumps(rec), flush=True)
    path = os.environ.get("RQ_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")

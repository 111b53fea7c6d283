"""Loader for the golden vectors written by ``make_golden.py`` (data only, no reference code)."""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

PATH = Path(__file__).resolve().parent / "golden_cases.npz"


def unpack_upper(flat: np.ndarray, n: int, symmetric: bool) -> np.ndarray:
    out = np.zeros((n, n), dtype=flat.dtype)
    iu = np.triu_indices(n)
    out[iu] = flat
    if symmetric:
        il = np.tril_indices(n, -1)
        out[il] = out.T[il]
    return out


@dataclass
class GoldenCase:
    meta: dict
    arrays: dict

    @property
    def name(self):
        return self.meta["name"]

    def t(self, key):
        return torch.from_numpy(np.array(self.arrays[key]))

    def H(self):
        C, G = self.meta["C"], self.meta["G"]
        flat = self.arrays["H_upper"]
        return torch.from_numpy(np.stack([unpack_upper(flat[g], C, True) for g in range(G)]))

    def sub(self, s, tag):
        key = f"sub{s}_{tag}"
        if key not in self.arrays:
            return None
        a = self.arrays[key]
        C = self.meta["C"]
        if tag == "Hinv_init":
            a = unpack_upper(a, C, True)
        elif tag == "Hinv_upper_cholesky":
            a = unpack_upper(a, C, False)
        return torch.from_numpy(np.array(a))


def quadratic_refresh(X, W0, G0):
    """Deterministic stand-in for a layer backward (``gradient_refresh_fn``), shared by the
    golden-vector script, the oracle tests and the GPU tests: the gradient of
    0.5 tr((W - W0) A (W - W0)^T) + <G0, W> with A = X^T X / n, scaled by (1 + slide_alpha) / 2
    when the caller passes ``slide_alpha`` (block_gd).  Computed in float64, returned float32."""
    Xf = torch.as_tensor(X).double().reshape(-1, torch.as_tensor(X).shape[-1])
    A = (Xf.T @ Xf) / Xf.shape[0]
    W0 = torch.as_tensor(W0).double()
    G0 = torch.as_tensor(G0).double()

    def fn(weight_snapshot, slide_alpha=None):
        dev = weight_snapshot.device
        D = weight_snapshot.double() - W0.to(dev)
        grad = D @ A.to(dev) + G0.to(dev)
        if slide_alpha is not None:
            grad = grad * (0.5 + 0.5 * float(slide_alpha))
        loss = float(0.5 * (D * (D @ A.to(dev))).sum())
        return grad.float(), {"mean_refresh_loss": loss, "slide_alpha": slide_alpha}
    return fn


class GoldenSet:
    def __init__(self, cases, beta):
        self.all_cases = cases
        self.cases = [c for c in cases if c.meta.get("kind") != "gptq"]      # GPTQPlus
        self.gptq_cases = [c for c in cases if c.meta.get("kind") == "gptq"]  # classic GPTQ
        self.beta = beta

    @classmethod
    def load(cls):
        z = np.load(PATH, allow_pickle=False)
        meta = json.loads(bytes(z["__meta__"]).decode())
        cases = []
        for m in meta:
            prefix = m["name"] + "__"
            arrays = {k[len(prefix):]: z[k] for k in z.files if k.startswith(prefix)}
            cases.append(GoldenCase(m, arrays))
        beta = {k: z[k] for k in z.files if k.startswith("beta")}
        return cls(cases, beta)

    def by_name(self, name):
        for c in self.all_cases:
            if c.name == name:
                return c
        raise KeyError(name)

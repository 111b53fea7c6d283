"""CPU restatement of the classic GPTQ class the reference ships next to GPTQ+ (TEST
INFRASTRUCTURE ONLY: only ``tests/`` may import it, as the checker of the drop-in
``gptq_plus_mp_quant_amd.GPTQ``).

Follows ``gptq_utils/gptq_utils.py:23-180`` op for op on CPU tensors:

* ``add_batch`` (:33-43): running mean, ``H *= n / (n + b)``, ``x <- sqrt(2 / n) x``,
  ``H += x x^T``;
* ``fasterquant`` (:45-171): RTN fallback for an all-zero H, dead columns, static groups from
  the dead-fixed unpermuted W, act_order by ``argsort(diag(H))``, the damped chain
  chol -> cholesky_inverse -> chol(upper) with +0.0015 retries and a ValueError at 1, the
  column loop ``err = (w - q) / d`` with dynamic groups re-fitted on the working W at every
  group start, the trailing update, un-permute.  The quantizer left on the object is the one
  the reference leaves (the last dynamic fit, or the last static group used).

Pinned by golden vectors from the reference class itself (``tests/golden/make_golden.py``).
"""
from __future__ import annotations

import copy
import math

import torch

from .gptqplus_cpu import FasterquantResult


class GPTQOracle:
    def __init__(self, weight: torch.Tensor):
        self.weight = weight.clone()
        self.rows, self.columns = weight.shape
        self.H = torch.zeros((self.columns, self.columns))
        self.nsamples = 0
        self.quantizer = None

    # gptq_utils.py:33-43
    def add_batch(self, inp, out=None):
        if len(inp.shape) == 2:
            inp = inp.unsqueeze(0)
        tmp = inp.shape[0]
        if len(inp.shape) == 3:
            inp = inp.reshape((-1, inp.shape[-1]))
        inp = inp.t()
        self.H *= self.nsamples / (self.nsamples + tmp)
        self.nsamples += tmp
        inp = math.sqrt(2 / self.nsamples) * inp.float()
        self.H += inp.matmul(inp.t())

    # gptq_utils.py:45-171
    def fasterquant(self, blocksize=128, percdamp=0.01, groupsize=-1, actorder=False,
                    static_groups=False) -> FasterquantResult:
        W = self.weight.clone().float()
        Scale = W.clone()
        W_int = W.clone()
        if not self.quantizer.ready():
            self.quantizer.find_params(W)
        H = self.H
        self.H = None
        if (H == 0).all():
            H = torch.eye(self.columns).to(H)
        dead = torch.diag(H) == 0
        H[dead, dead] = 1
        W[:, dead] = 0
        groups = None
        if static_groups:
            groups = []
            for i in range(0, self.columns, groupsize):
                q = copy.deepcopy(self.quantizer)
                q.find_params(W[:, i:(i + groupsize)])
                groups.append(q)
        perm = invperm = None
        if actorder:
            perm = torch.argsort(torch.diag(H), descending=True)
            W = W[:, perm]
            H = H[perm][:, perm]
            invperm = torch.argsort(perm)
        self.perm = perm
        Q = torch.zeros_like(W)
        damp_percent = percdamp
        while 1 > damp_percent > 0:
            try:
                damp = damp_percent * torch.mean(torch.diag(H))
                diag = torch.arange(self.columns)
                H[diag, diag] += damp
                H = torch.linalg.cholesky(H)
                H = torch.cholesky_inverse(H)
                H = torch.linalg.cholesky(H, upper=True)
                Hinv = H
                break
            except torch._C._LinAlgError:
                damp_percent += 0.0015
        if not (0 < damp_percent < 1):
            raise ValueError(f"Quantization: `damp_percent` must between 0 and 1. current is {damp_percent}")
        for i1 in range(0, self.columns, blocksize):
            i2 = min(i1 + blocksize, self.columns)
            count = i2 - i1
            W1 = W[:, i1:i2].clone()
            Q1 = torch.zeros_like(W1)
            W_int1 = torch.zeros_like(W1)
            Scale1 = torch.zeros_like(W1)
            Err1 = torch.zeros_like(W1)
            Hinv1 = Hinv[i1:i2, i1:i2]
            for i in range(count):
                w = W1[:, i]
                d = Hinv1[i, i]
                if groupsize != -1:
                    if not static_groups:
                        if (i1 + i) % groupsize == 0:
                            self.quantizer.find_params(W[:, (i1 + i):(i1 + i + groupsize)])
                    else:
                        idx = i1 + i
                        if actorder:
                            idx = perm[idx]
                        self.quantizer = groups[idx // groupsize]
                q, int_weight, scale = self.quantizer.fake_quantize(w.unsqueeze(1))
                Q1[:, i] = q.flatten()
                q = q.flatten()
                W_int1[:, i] = int_weight.flatten()
                Scale1[:, i] = scale.flatten()
                err1 = (w - q) / d
                W1[:, i:] -= err1.unsqueeze(1).matmul(Hinv1[i, i:].unsqueeze(0))
                Err1[:, i] = err1
            Q[:, i1:i2] = Q1
            W_int[:, i1:i2] = W_int1
            Scale[:, i1:i2] = Scale1
            W[:, i2:] -= Err1.matmul(Hinv[i1:i2, i2:])
        if actorder:
            Q = Q[:, invperm]
            # the reference un-permutes Q only; W_int / Scale keep the permuted column order
        Q_out = Q.reshape(self.weight.shape).to(self.weight.dtype)
        if torch.any(torch.isnan(Q_out)):
            raise ValueError("NaN in weights")
        return FasterquantResult(Q=Q_out, Q_fp32=Q, W_int=W_int, Scale=Scale, subgroups=[])

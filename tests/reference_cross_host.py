"""The reference's own op sequence (the oracle: torch on the CPU, MKL BLAS / LAPACK) on identical
inputs on two hosts, to size how far the reference's 4-bit codes move with the host's BLAS /
LAPACK build alone (a baseline for the GPU path's own-chain flip counts).

  python tests/reference_cross_host.py run OUT.npz C      # on each host: seeded inputs, codes
  python tests/reference_cross_host.py compare A.npz B.npz

One subgroup (R = 2048, NUM_GROUPS = 1), C columns, 16 x 2048 tokens with 8 outlier channels,
w4 asymmetric per-channel, act_order, B = 128; inputs from seeded CPU generators, so both hosts
see the same bits.  Not collected by pytest (CPU-only measurement, minutes at C = 28672).
"""
import hashlib
import os
import sys
import time

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer  # noqa: E402


def run(out, C):
    R, G, N, T = 2048, 1, 16, 2048
    g = torch.Generator()
    g.manual_seed(77)
    t0 = time.time()
    W = (torch.randn((R, C), generator=g) * 0.015).half()
    s = torch.exp(torch.randn((N, T, G), generator=g))
    s[..., 0].clamp_(max=float(torch.quantile(s[..., 0].flatten(), 0.99)))
    o = GPTQPlusOracle(W, s, torch.zeros(R, C), G, 0.0, 0.0)
    o.quantizer = make_quantizer(4, False)
    for j in range(0, N, 4):
        gx = torch.Generator()
        gx.manual_seed(1000 + j)
        X = torch.randn((4, T, C), generator=gx).half()
        X[:, :, :8] *= 20
        o.add_batch(X)
    o.finalize_hessian()
    t1 = time.time()
    res = o.fasterquant(blocksize=128, percdamp=0.01, groupsize=-1, actorder=True, static_groups=True)
    t2 = time.time()
    codes = res.W_int.to(torch.int16).numpy().astype(np.int8) + 8                 # 0 .. 15
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    np.savez_compressed(out, packed=packed, Hinv_diag=torch.diagonal(res.subgroups[0].Hinv).numpy())
    hH = hashlib.sha256(o.H.numpy().tobytes()).hexdigest()[:16]
    print(f"C={C}: H sha256 {hH}, damp {res.subgroups[0].damp_percent}, hessian {t1 - t0:.0f} s, "
          f"fasterquant {t2 - t1:.0f} s", flush=True)


def compare(fa, fb):
    a, b = np.load(fa), np.load(fb)
    pa, pb = a["packed"], b["packed"]
    flips = int(((pa & 15) != (pb & 15)).sum() + ((pa >> 4) != (pb >> 4)).sum())
    n = pa.size * 2
    da, db = a["Hinv_diag"].astype(np.float64), b["Hinv_diag"].astype(np.float64)
    print(f"{flips} / {n} codes differ ({100 * flips / n:.4f} %); diag(H^-1) rel. difference "
          f"{np.linalg.norm(da - db) / np.linalg.norm(db):.2e}")


if __name__ == "__main__":
    if sys.argv[1] == "run":
        run(sys.argv[2], int(sys.argv[3]))
    else:
        compare(sys.argv[2], sys.argv[3])

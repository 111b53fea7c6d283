"""Parity with the reference's op sequence at the full BASELINE shapes of one linear:
configs[0] (q_proj 4096 x 4096, NUM_GROUPS = 1, w4 asym per-channel, act_order, B = 128, GPTQ+
term off) and configs[1] (the same with NUM_GROUPS = 4 and the GPTQ+ term on at alpha = 0),
128 x 2048 calibration tokens fed in add_batch chunks of 16 samples.

The CPU oracle cannot form the 4 x 4096^2 Hessians from 262144 tokens in a test's time, so:
- act_square is computed by the oracle from the same chunks (gptq_plus_utils.py:856, 889) and
  must equal the GPU's bit for bit, and the act_order permutation must equal the oracle's
  torch.argsort of it (:1046) exactly;
- the GPU's finalized H is handed to the oracle, which then runs the reference's fasterquant
  (fp32 LAPACK chain, column loop, trailing update) on the CPU;
- with the oracle's H^-1 injected the codes must be equal (Z = 0: every later stage is
  bit-exact); with the GPU's own fp64 chain, H^-1 within 1e-4 (rel. Frobenius) of the
  oracle's, code flips <= 0.01 %, and the layer reconstruction error
  ||(W - Q) X^T||^2 / ||W X^T||^2 over all tokens within 0.5 % of the oracle's.
Each case's numbers are printed and, when RQ_PARITY_LOG names a file, appended to it as JSON.
"""
import json
import os

import pytest
import torch

from gptq_plus_mp_quant_amd import GPTQPlus, WeightQuantizer
from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
from tests._util import rel_fro

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
R = C = 4096
N, T, BSZ = 128, 2048, 16
CASES = {"configs0_q_proj_G1": dict(G=1, seed=11), "configs1_q_proj_G4": dict(G=4, seed=12)}


def _inputs(seed, G):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    X = torch.empty((N, T, C), dtype=torch.float16, device=DEV)
    for i in range(N):
        X[i] = torch.randn((T, C), generator=gen, device=DEV).half()
    X[:, :, torch.randperm(C, generator=gen, device=DEV)[:8]] *= 20
    W = (torch.randn((R, C), generator=gen, device=DEV) * 0.02).half()
    s = torch.exp(torch.randn((N, T, G), generator=gen, device=DEV))
    for g in range(G):
        s[..., g].clamp_(max=float(torch.quantile(s[..., g].flatten(), 0.99)))
    grad = torch.randn((R, C), generator=gen, device=DEV) * 1e-4
    return X, W, s, grad


def _recon(W, Q, X):
    """||(W - Q) X^T||^2 / ||W X^T||^2 over every token (fp32 products, fp64 sums)."""
    D = (W.float() - Q.float())
    num = den = 0.0
    for j in range(0, N, BSZ):
        x = X[j:j + BSZ].reshape(-1, C).float()
        num += float((D @ x.T).double().pow(2).sum())
        den += float((W.float() @ x.T).double().pow(2).sum())
    return num / den


def _log(rec):
    print(json.dumps(rec), flush=True)
    path = os.environ.get("RQ_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")


@pytest.mark.parametrize("name", list(CASES))
def test_full_shape_parity(name):
    G, seed = CASES[name]["G"], CASES[name]["seed"]
    print(f"{name}: generating inputs", flush=True)
    X, W, s, grad = _inputs(seed, G)
    layer = torch.nn.Linear(C, R, bias=False).to(DEV, torch.float16)

    def gpu_obj():
        layer.weight.data.copy_(W)
        g = GPTQPlus(layer, saliency=s, gradient=grad, num_groups=G, alpha=0.0, reference_loss=0.0)
        g.quantizer = WeightQuantizer()
        g.quantizer.configure(4, perchannel=True, sym=False, mse=False)
        return g

    g = gpu_obj()
    for j in range(0, N, BSZ):
        g.add_batch(X[j:j + BSZ], None)
    g.finalize_hessian()
    H_gpu = g.H.clone()
    fq = dict(blocksize=128, percdamp=0.01, groupsize=-1, actorder=True, static_groups=True)

    # oracle: act_square from the same chunks, H from the GPU
    o = GPTQPlusOracle(W.cpu(), s.cpu(), grad.cpu(), G, 0.0, 0.0)
    o.quantizer = make_quantizer(4, False)
    for j in range(0, N, BSZ):
        o.add_batch(X[j:j + BSZ].cpu(), hessian=False)
    o.finalize_hessian()
    o.H = H_gpu.cpu()
    act_bad = int((g.act_square.cpu() != o.act_square).sum())
    print(f"{name}: act_square entries differing from the CPU sum: {act_bad}/{C}", flush=True)
    res = o.fasterquant(**fq)
    ref_perm = res.subgroups[0].perm
    ties = int(C - torch.unique(o.act_square).numel())

    # (1) GPU with its own act_square / perm and the oracle's H^-1: bit-exact codes
    g.fasterquant(export_to_et=True, inject={"hinv": [(r.Hinv_init.to(DEV), r.Hinv.to(DEV)) for r in res.subgroups]},
                  **fq)
    torch.cuda.synchronize()
    perm_bad = int((g.perm.cpu() != ref_perm).sum())
    flips_inj = int((layer.int_weight.cpu() != res.W_int).sum())
    q_equal = torch.equal(layer.weight.data.cpu(), res.Q)

    # (2) everything the GPU's own: fp64 Cholesky chain
    g2 = gpu_obj()
    g2.H = H_gpu.clone()
    g2.act_square = g.act_square.clone()
    g2.token_count, g2.index, g2._finalized = g.token_count, g.index, True
    g2.fasterquant(export_to_et=True, keep_hinv=True, **fq)
    torch.cuda.synchronize()
    hinv_err = max(rel_fro(g2.Hinv_all[k], r.Hinv) for k, r in enumerate(res.subgroups))
    hinit_err = max(rel_fro(g2.Hinv_init_all[k], r.Hinv_init) for k, r in enumerate(res.subgroups))
    flips_own = int((layer.int_weight.cpu() != res.W_int).sum())
    n = res.W_int.numel()
    e_gpu = _recon(W, layer.weight.data, X)
    e_ref = _recon(W, res.Q.to(DEV), X)
    rec = dict(case=name, R=R, C=C, G=G, tokens=N * T, act_square_mismatch=act_bad, exact_ties_in_act_square=ties,
               perm_mismatch=perm_bad, flips_with_oracle_hinv=flips_inj, q_equal_with_oracle_hinv=q_equal,
               flips_own_chain=flips_own, codes=n, hinv_rel_fro=hinv_err, hinv_init_rel_fro=hinit_err,
               recon_gpu=e_gpu, recon_oracle=e_ref, recon_rel_diff=abs(e_gpu - e_ref) / e_ref,
               damp=[i["damp_percent"] for i in g2.subgroup_info],
               oracle_damp=[r.damp_percent for r in res.subgroups])
    _log(rec)
    assert act_bad == 0
    assert perm_bad == 0
    assert flips_inj == 0 and q_equal
    assert hinv_err <= 1e-4 and hinit_err <= 1e-4
    assert flips_own <= n // 10000
    assert abs(e_gpu - e_ref) <= 0.005 * e_ref

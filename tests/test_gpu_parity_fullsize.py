"""Parity with the reference's op sequence at the full BASELINE shapes of one linear:
configs[0] (q_proj 4096 x 4096, NUM_GROUPS = 1, w4 asym per-channel, act_order, B = 128, GPTQ+
term off) and configs[1] (the same with NUM_GROUPS = 4 and the GPTQ+ term on at alpha = 0),
128 x 2048 calibration tokens fed in add_batch chunks of 16 samples; configs[1] also with bf16
activations and weights (the reference's add_batch casts any float input to fp32, so the
products are the same kind; the GPU forms them from three bf16 pieces of 8 bits each in every
Hessian mode, and writes the weight back rounded to bf16).

Three comparisons per case:
- each side end to end on its own: the oracle accumulates its Hessians from the same chunks
  (the reference's fp32 `weighted` and bmm, gptq_plus_utils.py:846-850) and runs its own fp32
  LAPACK chain; the GPU runs its exact-product Hessian (the default) and its own fp64 chain.
  H within 1e-4 (rel. Frobenius, per group) of the oracle's, act_square bit for bit, the
  act_order permutation equal, the layer reconstruction error ||(W - Q) X^T||^2 / ||W X^T||^2
  over all tokens within 0.5 % of the oracle's, code flips <= 0.01 %.  Every flip is classified
  by the oracle's pre-rounding value w / scale: exact rounding ties, and the distance of the
  others from the rounding midpoint (tests/_util.flip_report).  The first flip of each row
  ("primary"; the later ones follow the row's changed error feedback) must be an exact tie or
  within 256 fp32 ulps of one, and at most 0.001 % of the codes.  The same holds for the opt-in
  two-piece Hessian ("split16");
- the GPU's finalized H handed to the oracle: with the oracle's H^-1 injected the codes must be
  equal (Z = 0: every later stage is bit-exact);
- the GPU's own fp64 chain on that H: H^-1 within 1e-4 of the oracle's, flips <= 0.01 %, and
  the reconstruction error within 0.5 %.
Each case's numbers are printed and, when RQ_PARITY_LOG names a file, appended to it as JSON.
"""
import json
import os

import pytest
import torch

from gptq_plus_mp_quant_amd import GPTQPlus, WeightQuantizer
from gptq_plus_mp_quant_amd import kernels as K
from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
from tests._util import flip_report, rel_fro, w_rel_fro

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
R = C = 4096
N, T, BSZ = 128, 2048, 16
CASES = {"configs0_q_proj_G1": dict(G=1, seed=11), "configs1_q_proj_G4": dict(G=4, seed=12),
         "configs1_q_proj_G4_bf16": dict(G=4, seed=13, dtype=torch.bfloat16)}


def _inputs(seed, G, dtype=torch.float16):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    X = torch.empty((N, T, C), dtype=dtype, device=DEV)
    for i in range(N):
        X[i] = torch.randn((T, C), generator=gen, device=DEV).to(dtype)
    X[:, :, torch.randperm(C, generator=gen, device=DEV)[:8]] *= 20
    W = (torch.randn((R, C), generator=gen, device=DEV) * 0.02).to(dtype)
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
    dtype = CASES[name].get("dtype", torch.float16)
    X, W, s, grad = _inputs(seed, G, dtype)
    layer = torch.nn.Linear(C, R, bias=False).to(DEV, dtype)

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

    # the oracle end to end: its own Hessians from the same chunks, its own chain
    o_own = GPTQPlusOracle(W.cpu(), s.cpu(), grad.cpu(), G, 0.0, 0.0)
    o_own.quantizer = make_quantizer(4, False)
    for j in range(0, N, BSZ):
        print(f"{name}: oracle add_batch chunk {j // BSZ}", flush=True)
        o_own.add_batch(X[j:j + BSZ].cpu())
    o_own.finalize_hessian()
    h_err = [rel_fro(H_gpu[k], o_own.H[k]) for k in range(G)]
    res_own = o_own.fasterquant(record_ratio=True, **fq)
    print(f"{name}: H rel-Frobenius per group {h_err}", flush=True)

    # the oracle on the GPU's H (act_square: its own, from the same chunks)
    o = GPTQPlusOracle(W.cpu(), s.cpu(), grad.cpu(), G, 0.0, 0.0)
    o.quantizer = make_quantizer(4, False)
    o.act_square = o_own.act_square.clone()
    o.index, o.token_count, o._finalized = o_own.index, o_own.token_count, True
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
    w_own_chain = w_rel_fro(layer.weight.data, res.Q)
    w_own_h = w_rel_fro(layer.weight.data, res_own.Q)
    # (3) each side's own Hessian and chain: the GPU's default H (g2's) against the oracle's
    # own; then the opt-in two-piece Hessian, accumulated again
    own = flip_report(g2.codes, res_own.W_int, res_own.ratio, res_own.subgroups[0].perm)
    e_own_ref = _recon(W, res_own.Q.to(DEV), X)
    g3 = gpu_obj()
    with K.hessian_math("split16"):
        for j in range(0, N, BSZ):
            g3.add_batch(X[j:j + BSZ], None)
    g3.finalize_hessian()
    h2_err = [rel_fro(g3.H[k], o_own.H[k]) for k in range(G)]
    g3.fasterquant(**fq)
    torch.cuda.synchronize()
    own2 = flip_report(g3.codes, res_own.W_int, res_own.ratio, res_own.subgroups[0].perm)
    e_own2_gpu = _recon(W, layer.weight.data, X)
    w_own2 = w_rel_fro(layer.weight.data, res_own.Q)
    rec = dict(case=name, R=R, C=C, G=G, tokens=N * T, act_square_mismatch=act_bad, exact_ties_in_act_square=ties,
               perm_mismatch=perm_bad, flips_with_oracle_hinv=flips_inj, q_equal_with_oracle_hinv=q_equal,
               flips_own_chain=flips_own, codes=n, hinv_rel_fro=hinv_err, hinv_init_rel_fro=hinit_err,
               recon_gpu=e_gpu, recon_oracle=e_ref, recon_rel_diff=abs(e_gpu - e_ref) / e_ref,
               damp=[i["damp_percent"] for i in g2.subgroup_info],
               oracle_damp=[r.damp_percent for r in res.subgroups],
               own_h_rel_fro=h_err, own_flips=own, own_recon_gpu=e_gpu, own_recon_oracle=e_own_ref,
               own_recon_rel_diff=abs(e_gpu - e_own_ref) / e_own_ref,
               split16_h_rel_fro=h2_err, split16_own_flips=own2, split16_own_recon_gpu=e_own2_gpu,
               split16_own_recon_rel_diff=abs(e_own2_gpu - e_own_ref) / e_own_ref,
               w_rel_fro_own_chain=w_own_chain, w_rel_fro_own_hessian=w_own_h, split16_w_rel_fro_own_hessian=w_own2)
    _log(rec)
    assert act_bad == 0
    assert perm_bad == 0
    assert flips_inj == 0 and q_equal
    assert hinv_err <= 1e-4 and hinit_err <= 1e-4
    assert flips_own <= n // 10000
    assert abs(e_gpu - e_ref) <= 0.005 * e_ref
    assert max(h_err) <= 1e-4 and max(h2_err) <= 1e-4
    for r in (own, own2):
        assert r["flips"] <= n // 10000
        assert r["primary"] <= n // 100000 and r.get("primary_ulps_le_256", 0) == r["primary"]
    assert abs(e_gpu - e_own_ref) <= 0.005 * e_own_ref
    assert abs(e_own2_gpu - e_own_ref) <= 0.005 * e_own_ref

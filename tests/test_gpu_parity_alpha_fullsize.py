"""Parity of the GPTQ+ first-order term at a full BASELINE linear shape: q_proj 4096 x 4096,
NUM_GROUPS = 4, w4 asym per-channel, act_order, B = 128, the term on (alpha = 0.05, gradient
~ N(0, 1e-4^2)), 16 x 2048 tokens with outlier channels.  Three cases: the frozen mode with
reference_loss = 1e-3 (beta ~ 1e-7); surrogate_online (the first-order term re-evaluated
before every column, :580-584) with reference_loss = 50 (beta ~ 5e-3); block_gd with SGD
(:1572-1848) and reference_loss = 50, whose layer backward is an elementwise quadratic that
both devices evaluate identically (_diag_refresh).  The
oracle (the reference's op sequence on the host CPU) runs act_square and fasterquant on the
GPU's finalized H (gptq_plus_utils.py:174-194, 563-578 for the terms, :1500-1570 for the
trailing update with Z != 0).

- act_square bit for bit, the act_order permutation equal to the oracle's argsort;
- with the oracle's H^-1 factors and its (beta, Z, GHinv) injected: codes and the written
  weight equal (the column loop and the three k-ordered trailing products are the reference's
  op for op);
- with only the oracle's H^-1 injected: the GPU's beta equal to the reference formula
  (:183-193) evaluated in IEEE fp32 with numpy on the oracle's row statistic c, and within one
  rounding step of the oracle's own beta (1e-5 relative, or 2^-23; at most 1 % of the rows
  off the IEEE value by more than 1e-5, from c's summation order); Z and GHinv within 1e-5
  (rel. Frobenius) of the
  oracle's once rescaled by the two betas' ratio; code flips <= 0.01 %.
  At this shape beta = 1 - sqrt(1 - ratio) with ratio ~ 2e-7, where fp32 resolves beta only
  in steps of 2^-24: the reference's own value depends on the host.  1 - ratio rounds to
  1 - 3 * 2^-24, whose square root lies 4e-15 below a rounding midpoint.  IEEE fp32 (numpy,
  the GPU, torch on an Intel Xeon) gives beta = 2^-23, while torch's CPU sqrt on the AMD EPYC
  GPU host gives 2^-24.  Z and GHinv scale with beta row by row;
- with the GPU's own fp64 chain: H^-1 within 1e-4, reconstruction error within 0.5 % of the
  oracle's, code flips <= 0.02 %.
- each side end to end on its own (test_gptqplus_term_own_hessian, frozen mode, reference_loss
  = 50 so that beta ~ 5e-3 is resolved well above fp32's step): the oracle forms its own H from
  the same chunks and runs its own chain and terms; H within 1e-4 (rel. Frobenius, per group),
  act_square and the permutation equal, reconstruction error within 0.5 %, the first flip of
  each row an exact tie or within 4096 fp32 ulps of one (the two chains start from Hessians
  that differ by the fp32 summation orders), at most 0.001 % of the codes, total below 0.1 %.
The cases' numbers are printed and appended to RQ_PARITY_LOG (JSON lines) when it is set.
"""
import json
import os

import numpy as np
import pytest
import torch

from gptq_plus_mp_quant_amd import GPTQPlus, WeightQuantizer
from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
from tests._util import flip_report, rel_fro, w_rel_fro

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
R, C, G, N, T, BSZ = 4096, 4096, 4, 16, 2048, 8
ALPHA = 0.05
CASES = {"frozen_refloss_1e-3": ("frozen", 1e-3), "surrogate_online_refloss_50": ("surrogate_online", 50.0),
         "block_gd_sgd_refloss_50": ("block_gd", 50.0)}
BLOCK_GD = dict(grad_optimizer="sgd", grad_lr=0.008, grad_reg_strategy="none", second_order_scale=1.0, grad_clip=1.0)


def _diag_refresh(a, W0, G0):
    """A layer backward for block_gd that both devices evaluate identically: the gradient of
    0.5 sum_j a_j ||W[:, j] - W0[:, j]||^2 + <G0, W>, elementwise in float64, returned float32
    (scaled by (1 + slide_alpha) / 2 when the caller passes slide_alpha)."""
    def fn(weight_snapshot, slide_alpha=None):
        dev = weight_snapshot.device
        D = weight_snapshot.double() - W0.to(dev)
        grad = D * a.to(dev) + G0.to(dev)
        if slide_alpha is not None:
            grad = grad * (0.5 + 0.5 * float(slide_alpha))
        return grad.float(), {"mean_refresh_loss": float(0.5 * (D * D * a.to(dev)).sum().cpu()),
                              "slide_alpha": slide_alpha}
    return fn
FQ = dict(blocksize=128, percdamp=0.01, groupsize=-1, actorder=True, static_groups=True)


def _obj(layer, W, s, grad, ref_loss):
    layer.weight.data.copy_(W)
    g = GPTQPlus(layer, saliency=s, gradient=grad, num_groups=G, alpha=ALPHA, reference_loss=ref_loss)
    g.quantizer = WeightQuantizer()
    g.quantizer.configure(4, perchannel=True, sym=False, mse=False)
    return g


def _rerun(layer, W, s, grad, ref_loss, src, H, act, **kw):
    g = _obj(layer, W, s, grad, ref_loss)
    g.H, g.act_square = H.clone(), act.clone()
    g.index, g.token_count, g._finalized = src.index, src.token_count, True
    g.fasterquant(export_to_et=True, keep_hinv=True, **FQ, **kw)
    torch.cuda.synchronize()
    return g


@pytest.mark.parametrize("case", list(CASES))
def test_gptqplus_term_parity_full_linear(case):
    mode, REF_LOSS = CASES[case]
    gen = torch.Generator(device=DEV)
    gen.manual_seed(36)
    X = torch.randn((N, T, C), generator=gen, device=DEV).half()
    X[:, :, torch.randperm(C, generator=gen, device=DEV)[:8]] *= 20
    W = (torch.randn((R, C), generator=gen, device=DEV) * 0.02).half()
    s = torch.exp(torch.randn((N, T, G), generator=gen, device=DEV))
    for k in range(G):
        s[..., k].clamp_(max=float(torch.quantile(s[..., k].flatten(), 0.99)))
    grad = torch.randn((R, C), generator=gen, device=DEV) * 1e-4
    extra = {}
    if mode == "block_gd":
        a = X.reshape(-1, C).double().pow(2).mean(0).cpu()
        extra = dict(BLOCK_GD, gradient_refresh_fn=_diag_refresh(a, W.double().cpu(), grad.double().cpu()))
    layer = torch.nn.Linear(C, R, bias=False).to(DEV, torch.float16)
    g = _obj(layer, W, s, grad, REF_LOSS)
    for j in range(0, N, BSZ):
        g.add_batch(X[j:j + BSZ], None)
    g.finalize_hessian()
    torch.cuda.synchronize()
    H_keep, act_keep = g.H.clone(), g.act_square.clone()

    o = GPTQPlusOracle(W.cpu(), s.cpu(), grad.cpu(), G, ALPHA, REF_LOSS)
    o.quantizer = make_quantizer(4, False)
    for j in range(0, N, BSZ):
        o.add_batch(X[j:j + BSZ].cpu(), hessian=False)
    o.finalize_hessian()
    o.H = H_keep.cpu()
    act_bad = int((act_keep.cpu() != o.act_square).sum())
    res = o.fasterquant(g_update_mode=mode, **FQ, **extra)
    subs = res.subgroups
    hinv = [(r.Hinv_init.to(DEV), r.Hinv.to(DEV)) for r in subs]
    terms = [(r.beta.to(DEV), r.Z.to(DEV), r.GHinv.to(DEV)) for r in subs]
    R_s = R // G
    z_rel = max(float(r.Z.abs().max()) for r in subs) / float(W.float().abs().max())

    g1 = _rerun(layer, W, s, grad, REF_LOSS, g, H_keep, act_keep, g_update_mode=mode,
                inject={"hinv": hinv, "terms": terms}, **extra)
    perm_bad = int((g1.perm.cpu() != subs[0].perm).sum())
    flips_all = int((layer.int_weight.cpu() != res.W_int).sum())
    q_equal = torch.equal(layer.weight.data.cpu(), res.Q)
    g1.free()

    g2 = _rerun(layer, W, s, grad, REF_LOSS, g, H_keep, act_keep, g_update_mode=mode, inject={"hinv": hinv},
                **extra)
    target = 2 * (ALPHA / (R * C)) * REF_LOSS
    beta_ieee_bad = beta_step_bad = 0
    beta_err = z_err = gh_err = 0.0
    for k, (info, r) in enumerate(zip(g2.subgroup_info, subs)):
        # the reference's row statistic (torch fp32 on the host), then IEEE fp32 in numpy
        gs = grad[k * R_s:(k + 1) * R_s].cpu()[:, r.perm]
        gh = gs.matmul(r.Hinv_init)
        c = ((gs * gh).sum(dim=1) - ((gh ** 2) / torch.diagonal(r.Hinv_init).unsqueeze(0)).mean(1)).numpy()
        c = np.maximum(c, np.float32(target))
        ratio = np.clip(np.where(c > 0, np.float32(target) / c, np.float32(0)), 0, 1).astype(np.float32)
        b_ieee = (np.float32(1) - np.sqrt(np.maximum(np.float32(1) - ratio, np.float32(0)))).astype(np.float32)
        gb, ob = info["beta"].cpu(), r.beta
        beta_ieee_bad += int((np.abs(gb.numpy() - b_ieee) > 1e-5 * np.abs(b_ieee)).sum())
        beta_step_bad += int(((gb - ob).abs() > torch.maximum(1e-5 * ob.abs(), torch.tensor(2.0 ** -23))).sum())
        beta_err = max(beta_err, rel_fro(gb, ob))
        scale = torch.where(ob != 0, gb.double() / ob.double(), torch.ones_like(ob, dtype=torch.float64))[:, None]
        z_err = max(z_err, rel_fro(g2.Z[k * R_s:(k + 1) * R_s], r.Z.double() * scale))
        gh_err = max(gh_err, rel_fro(g2.GHinv_initial[k * R_s:(k + 1) * R_s], r.GHinv.double() * scale))
    flips_terms = int((layer.int_weight.cpu() != res.W_int).sum())
    g2.free()

    g3 = _rerun(layer, W, s, grad, REF_LOSS, g, H_keep, act_keep, g_update_mode=mode, **extra)
    hinv_err = max(rel_fro(g3.Hinv_all[k], r.Hinv) for k, r in enumerate(subs))
    flips_own = int((layer.int_weight.cpu() != res.W_int).sum())
    n = res.W_int.numel()
    x = X.reshape(-1, C).float()
    Wx = float((W.float() @ x.T).double().pow(2).sum())
    e_gpu = float(((W.float() - layer.weight.data.float()) @ x.T).double().pow(2).sum()) / Wx
    e_ref = float(((W.float() - res.Q.to(DEV).float()) @ x.T).double().pow(2).sum()) / Wx
    w_own = w_rel_fro(layer.weight.data, res.Q)
    g3.free()
    g.free()
    rec = dict(case=f"configs1_q_proj_G4_alpha_{case}", mode=mode, R=R, C=C, G=G, tokens=N * T, alpha=ALPHA, ref_loss=REF_LOSS,
               z_max_over_w_max=z_rel, act_square_mismatch=act_bad, perm_mismatch=perm_bad,
               flips_with_oracle_hinv_and_terms=flips_all, q_equal_with_oracle_hinv_and_terms=q_equal,
               beta_rel_fro=beta_err, beta_rows_not_ieee=beta_ieee_bad, beta_rows_beyond_one_step=beta_step_bad,
               z_rel_fro_beta_rescaled=z_err, ghinv_rel_fro_beta_rescaled=gh_err,
               flips_with_oracle_hinv=flips_terms, flips_own_chain=flips_own, codes=n, hinv_rel_fro=hinv_err,
               recon_gpu=e_gpu, recon_oracle=e_ref, recon_rel_diff=abs(e_gpu - e_ref) / e_ref,
               w_rel_fro_own_chain=w_own)
    print(json.dumps(rec), flush=True)
    path = os.environ.get("RQ_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")
    assert act_bad == 0 and perm_bad == 0
    assert flips_all == 0 and q_equal
    assert beta_ieee_bad <= R // 100 and beta_step_bad == 0
    assert z_err <= 1e-5 and gh_err <= 1e-5
    assert flips_terms <= n // 10000
    assert hinv_err <= 1e-4
    assert abs(e_gpu - e_ref) <= 0.005 * e_ref
    assert flips_own <= n // 5000


def test_gptqplus_term_own_hessian():
    ref_loss = 50.0
    gen = torch.Generator(device=DEV)
    gen.manual_seed(37)
    X = torch.randn((N, T, C), generator=gen, device=DEV).half()
    X[:, :, torch.randperm(C, generator=gen, device=DEV)[:8]] *= 20
    W = (torch.randn((R, C), generator=gen, device=DEV) * 0.02).half()
    s = torch.exp(torch.randn((N, T, G), generator=gen, device=DEV))
    for k in range(G):
        s[..., k].clamp_(max=float(torch.quantile(s[..., k].flatten(), 0.99)))
    grad = torch.randn((R, C), generator=gen, device=DEV) * 1e-4
    layer = torch.nn.Linear(C, R, bias=False).to(DEV, torch.float16)
    g = _obj(layer, W, s, grad, ref_loss)
    for j in range(0, N, BSZ):
        g.add_batch(X[j:j + BSZ], None)
    g.finalize_hessian()
    torch.cuda.synchronize()
    print("GPTQ+ term, own Hessians: oracle add_batch", flush=True)
    o = GPTQPlusOracle(W.cpu(), s.cpu(), grad.cpu(), G, ALPHA, ref_loss)
    o.quantizer = make_quantizer(4, False)
    for j in range(0, N, BSZ):
        o.add_batch(X[j:j + BSZ].cpu())
    o.finalize_hessian()
    h_err = [rel_fro(g.H[k], o.H[k]) for k in range(G)]
    act_bad = int((g.act_square.cpu() != o.act_square).sum())
    print(f"GPTQ+ term, own Hessians: H rel-Frobenius {h_err}; oracle fasterquant", flush=True)
    res = o.fasterquant(record_ratio=True, **FQ)
    g.fasterquant(**FQ)
    torch.cuda.synchronize()
    perm = res.subgroups[0].perm
    perm_bad = int((g.perm.cpu() != perm).sum())
    rep = flip_report(g.codes, res.W_int, res.ratio, perm)
    n = res.W_int.numel()
    x = X.reshape(-1, C).float()
    Wx = float((W.float() @ x.T).double().pow(2).sum())
    e_gpu = float(((W.float() - layer.weight.data.float()) @ x.T).double().pow(2).sum()) / Wx
    e_ref = float(((W.float() - res.Q.to(DEV).float()) @ x.T).double().pow(2).sum()) / Wx
    w_own = w_rel_fro(layer.weight.data, res.Q)
    beta_g = torch.cat([i["beta"].reshape(-1).cpu() for i in g.subgroup_info])
    beta_o = torch.cat([r.beta.reshape(-1) for r in res.subgroups])
    rec = dict(case="configs1_q_proj_G4_alpha_frozen_refloss_50_own_hessian", R=R, C=C, G=G, tokens=N * T,
               alpha=ALPHA, ref_loss=ref_loss, codes=n, act_square_mismatch=act_bad, perm_mismatch=perm_bad,
               h_rel_fro=h_err, beta_rel_fro=rel_fro(beta_g, beta_o), beta_mean=float(beta_o.mean()), flips=rep,
               recon_gpu=e_gpu, recon_oracle=e_ref, recon_rel_diff=abs(e_gpu - e_ref) / e_ref, w_rel_fro=w_own)
    print(json.dumps(rec), flush=True)
    path = os.environ.get("RQ_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")
    g.free()
    assert act_bad == 0 and perm_bad == 0
    assert max(h_err) <= 1e-4
    assert abs(e_gpu - e_ref) <= 0.005 * e_ref
    assert rep["primary"] <= n // 100000 and rep.get("primary_ulps_le_4096", 0) == rep["primary"]
    assert rep["flips"] <= n // 1000

"""Parity at the shapes of BASELINE configs[2]: the seven linears of a Llama-3-8B decoder
layer (q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096, down 4096x14336), NUM_GROUPS = 4,
w4 asym per-channel, act_order, B = 128, at a reduced token count (16 samples x 2048).  The
Hessians come from the layer's own call pattern: q/k/v and gate/up through add_batch_shared
over their shared input (gptq_plus_utils.py:6990-7039), o and down through add_batch.

Per linear, each side end to end on its own (test_layer_linear_own_hessian): the oracle
accumulates its Hessians from the same chunks (the reference's fp32 `weighted` and bmm,
gptq_plus_utils.py:846-850) and runs its own fp32 LAPACK chain; the GPU its exact-product
Hessian (the default) and fp64 chain, and again with the opt-in two-piece Hessian.  H within
1e-4 (rel. Frobenius, per group), act_square bit for bit, reconstruction error within 0.5 %,
code flips within the bars below, and every flip classified by the oracle's pre-rounding
value w / scale (exact rounding ties; distance of the others from the rounding midpoint).

Per linear, against the CPU oracle given the GPU's finalized H (test_layer_linear_parity):
- act_square bit for bit, and the act_order permutation equal to the oracle's argsort;
- with the oracle's fp32 H^-1 injected: codes and the written weight equal (Z = 0);
- with the GPU's fp64 chain: H^-1 and H^-1_init within 1e-4 (rel. Frobenius), reconstruction
  error ||(W - Q) X^T||^2 / ||W X^T||^2 within 0.5 %, and the code flips classified: the first
  differing code of each row ("primary") must lie within 256 fp32 ulps of a rounding midpoint of
  the reference's value w / scale (an exact tie or a near-tie), and at most 0.001 % of the codes
  may be primary; the later flips of such a row follow its changed error feedback (the column
  loop carries each code's error into every later column of the row, :1330-1356), a different
  but equally valid rounding path, and the reconstruction error bounds their effect.  Total
  flips <= 0.01 % at C = 4096.  At C = 14336 the reference's fp32 LAPACK chain is itself 6e-7
  away from the exact factor (measured here against an fp64 factorisation on the host) while
  the GPU's is within fp32 rounding of it (3e-8): there the GPU's factor must be the closer one,
  and the total (cascades included) is reported, with a sanity bound of 0.1 %.
Each case's numbers are printed and appended to RQ_PARITY_LOG (JSON lines) when it is set.
"""
import json
import os

import pytest
import torch

from gptq_plus_mp_quant_amd import GPTQPlus, WeightQuantizer, add_batch_shared
from gptq_plus_mp_quant_amd import kernels as K
from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
from tests._util import flip_report, rel_fro, w_rel_fro

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
G, N, T, BSZ = 4, 16, 2048, 8
MODULES = [("q_proj", 4096, 4096, "attn"), ("k_proj", 1024, 4096, "attn"), ("v_proj", 1024, 4096, "attn"),
           ("o_proj", 4096, 4096, "o"), ("gate_proj", 14336, 4096, "mlp"), ("up_proj", 14336, 4096, "mlp"),
           ("down_proj", 4096, 14336, "down")]
WIDTH = {"attn": 4096, "o": 4096, "mlp": 4096, "down": 14336}
FQ = dict(blocksize=128, percdamp=0.01, groupsize=-1, actorder=True, static_groups=True)


def _log(rec):
    print(json.dumps(rec), flush=True)
    path = os.environ.get("RQ_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")


@pytest.fixture(scope="module")
def layer_state():
    gen = torch.Generator(device=DEV)
    gen.manual_seed(31)
    xs = {}
    for key, C in WIDTH.items():
        X = torch.randn((N, T, C), generator=gen, device=DEV).half()
        X[:, :, torch.randperm(C, generator=gen, device=DEV)[:8]] *= 20
        xs[key] = X
    mods, objs, layers = {}, {}, {}
    for name, R, C, key in MODULES:
        W = (torch.randn((R, C), generator=gen, device=DEV) * 0.02).half()
        s = torch.exp(torch.randn((N, T, G), generator=gen, device=DEV))
        for g in range(G):
            s[..., g].clamp_(max=float(torch.quantile(s[..., g].flatten(), 0.99)))
        grad = torch.randn((R, C), generator=gen, device=DEV) * 1e-4
        layer = torch.nn.Linear(C, R, bias=False).to(DEV, torch.float16)
        layer.weight.data.copy_(W)
        mods[name], layers[name] = (W, s, grad, key), layer
        objs[name] = _new_gpu(mods[name], layer)

    def accumulate(objs):
        for key in WIDTH:
            group = [objs[n] for n, _, _, k in MODULES if k == key]
            for j in range(0, N, BSZ):
                if len(group) > 1:
                    add_batch_shared(group, xs[key][j:j + BSZ])
                else:
                    group[0].add_batch(xs[key][j:j + BSZ], None)
        for g in objs.values():
            g.finalize_hessian()

    accumulate(objs)
    # the finalized Hessians of the default (exact-product) mode, kept for the own-Hessian test,
    # and those of the opt-in two-piece mode
    own = {n: (g.H.clone(), g.act_square.clone(), g.index, g.token_count) for n, g in objs.items()}
    objs2 = {n: _new_gpu(mods[n], layers[n]) for n in objs}
    with K.hessian_math("split16"):
        accumulate(objs2)
    own2 = {n: g.H for n, g in objs2.items()}
    torch.cuda.synchronize()
    return xs, mods, objs, layers, own, own2


def _new_gpu(mod, layer, H=None, act=None, index=0, token_count=0):
    W, s, grad, _ = mod
    layer.weight.data.copy_(W)
    g = GPTQPlus(layer, saliency=s, gradient=grad, num_groups=G, alpha=0.0, reference_loss=0.0)
    g.quantizer = WeightQuantizer()
    g.quantizer.configure(4, perchannel=True, sym=False, mse=False)
    if H is not None:
        g.H, g.act_square = H.clone(), act.clone()
        g.index, g.token_count, g._finalized = index, token_count, True
    return g


def _recon(W, Q, X):
    D = W.float() - Q.float()
    x = X.reshape(-1, X.shape[-1]).float()
    return float((D @ x.T).double().pow(2).sum()) / float((W.float() @ x.T).double().pow(2).sum())


@pytest.mark.parametrize("name", [m[0] for m in MODULES])
def test_layer_linear_parity(layer_state, name):
    xs, mods, objs, layers, _, _ = layer_state
    W, s, grad, key = mods[name]
    g, layer = objs[name], layers[name]
    R, C = W.shape
    print(f"{name}: R={R} C={C}", flush=True)
    o = GPTQPlusOracle(W.cpu(), s.cpu(), grad.cpu(), G, 0.0, 0.0)
    o.quantizer = make_quantizer(4, False)
    for j in range(0, N, BSZ):
        o.add_batch(xs[key][j:j + BSZ].cpu(), hessian=False)
    o.finalize_hessian()
    o.H = g.H.cpu()
    act_bad = int((g.act_square.cpu() != o.act_square).sum())
    res = o.fasterquant(record_ratio=True, **FQ)

    H_keep, act_keep = g.H.clone(), g.act_square.clone()
    g.fasterquant(export_to_et=True, inject={"hinv": [(r.Hinv_init.to(DEV), r.Hinv.to(DEV)) for r in res.subgroups]},
                  **FQ)
    torch.cuda.synchronize()
    perm_bad = int((g.perm.cpu() != res.subgroups[0].perm).sum())
    flips_inj = int((layer.int_weight.cpu() != res.W_int).sum())
    q_equal = torch.equal(layer.weight.data.cpu(), res.Q)

    layer.weight.data.copy_(W)
    g2 = GPTQPlus(layer, saliency=s, gradient=grad, num_groups=G, alpha=0.0, reference_loss=0.0)
    g2.quantizer = WeightQuantizer()
    g2.quantizer.configure(4, perchannel=True, sym=False, mse=False)
    g2.H, g2.act_square = H_keep, act_keep
    g2.index, g2.token_count, g2._finalized = g.index, g.token_count, True
    g2.fasterquant(export_to_et=True, keep_hinv=True, **FQ)
    torch.cuda.synchronize()
    hinv_err = max(rel_fro(g2.Hinv_all[k], r.Hinv) for k, r in enumerate(res.subgroups))
    hinit_err = max(rel_fro(g2.Hinv_init_all[k], r.Hinv_init) for k, r in enumerate(res.subgroups))
    flips_own = int((layer.int_weight.cpu() != res.W_int).sum())
    n = res.W_int.numel()
    e_gpu = _recon(W, layer.weight.data, xs[key])
    e_ref = _recon(W, res.Q.to(DEV), xs[key])
    w_own = w_rel_fro(layer.weight.data, res.Q)
    rec = dict(case=f"configs2_layer_{name}", R=R, C=C, G=G, tokens=N * T, act_square_mismatch=act_bad, w_rel_fro_own_chain=w_own,
               exact_ties_in_act_square=int(C - torch.unique(o.act_square).numel()), perm_mismatch=perm_bad,
               flips_with_oracle_hinv=flips_inj, q_equal_with_oracle_hinv=q_equal, flips_own_chain=flips_own,
               codes=n, hinv_rel_fro=hinv_err, hinv_init_rel_fro=hinit_err, recon_gpu=e_gpu, recon_oracle=e_ref,
               recon_rel_diff=abs(e_gpu - e_ref) / e_ref,
               own_chain_flip_report=flip_report(g2.codes, res.W_int, res.ratio, res.subgroups[0].perm))
    if C == 14336:
        # the GPU's fp64 chain on one subgroup against an fp64 factorisation on the host
        sub = 0
        Hw = H_keep[sub][g2.perm][:, g2.perm].double().cpu()
        dead = torch.diagonal(Hw) == 0
        Hw[dead, dead] = 1
        damp = float(torch.tensor(g2.subgroup_info[sub]["damp_percent"], dtype=torch.float32))
        idx = torch.arange(C)
        Hw32 = Hw.float()
        Hw32[idx, idx] += damp * torch.mean(torch.diagonal(Hw32))
        Hinv64 = torch.cholesky_inverse(torch.linalg.cholesky(Hw32.double()))
        U64 = torch.linalg.cholesky(Hinv64, upper=True)
        rec["hinv_vs_fp64_host"] = rel_fro(g2.Hinv_all[sub], U64)
        rec["hinv_init_vs_fp64_host"] = rel_fro(g2.Hinv_init_all[sub], Hinv64)
        rec["oracle_hinv_vs_fp64_host"] = rel_fro(res.subgroups[sub].Hinv, U64)
        del Hw, Hw32, Hinv64, U64
    _log(rec)
    assert act_bad == 0 and perm_bad == 0
    assert flips_inj == 0 and q_equal
    assert hinv_err <= 1e-4 and hinit_err <= 1e-4
    assert abs(e_gpu - e_ref) <= 0.005 * e_ref
    fr = rec["own_chain_flip_report"]
    assert fr["primary"] <= n // 100000 and fr.get("primary_ulps_le_256", 0) == fr["primary"]
    if C == 14336:
        assert rec["hinv_vs_fp64_host"] <= 1e-6 and rec["hinv_init_vs_fp64_host"] <= 1e-6
        assert rec["hinv_vs_fp64_host"] < rec["oracle_hinv_vs_fp64_host"]
        assert flips_own <= n // 1000
    else:
        assert flips_own <= n // 10000
    g.free()
    g2.free()


@pytest.mark.parametrize("name", [m[0] for m in MODULES])
def test_layer_linear_own_hessian(layer_state, name):
    """Each side end to end: the oracle forms its own H from the chunks and runs its own chain; the
    GPU its exact-product H (default) and its fp64 chain, then the two-piece H ("split16")."""
    xs, mods, _, layers, own, own2 = layer_state
    W, s, grad, key = mods[name]
    layer = layers[name]
    R, C = W.shape
    print(f"{name}: R={R} C={C}: oracle Hessians", flush=True)
    o = GPTQPlusOracle(W.cpu(), s.cpu(), grad.cpu(), G, 0.0, 0.0)
    o.quantizer = make_quantizer(4, False)
    for j in range(0, N, BSZ):
        o.add_batch(xs[key][j:j + BSZ].cpu())
    o.finalize_hessian()
    H3, act, index, tokens = own[name]
    h_err = [rel_fro(H3[k], o.H[k]) for k in range(G)]
    h2_err = [rel_fro(own2[name][k], o.H[k]) for k in range(G)]
    act_bad = int((act.cpu() != o.act_square).sum())
    print(f"{name}: H rel-Frobenius {h_err} (split16 {h2_err}); oracle fasterquant", flush=True)
    res = o.fasterquant(record_ratio=True, **FQ)
    perm = res.subgroups[0].perm
    n = res.W_int.numel()
    e_ref = _recon(W, res.Q.to(DEV), xs[key])
    out = {}
    for mode, H in (("split16x3", H3), ("split16", own2[name])):
        g = _new_gpu(mods[name], layer, H, act, index, tokens)
        g.fasterquant(**FQ)
        torch.cuda.synchronize()
        out[mode] = (flip_report(g.codes, res.W_int, res.ratio, perm), _recon(W, layer.weight.data, xs[key]),
                     w_rel_fro(layer.weight.data, res.Q))
        g.free()
    rep3, e3, w3 = out["split16x3"]
    rep2, e2, w2 = out["split16"]
    rec = dict(case=f"configs2_layer_{name}_own_hessian", R=R, C=C, G=G, tokens=N * T, codes=n,
               act_square_mismatch=act_bad, h_rel_fro=h_err, split16_h_rel_fro=h2_err,
               flips=rep3, recon_gpu=e3, recon_oracle=e_ref, recon_rel_diff=abs(e3 - e_ref) / e_ref,
               split16_flips=rep2, split16_recon_gpu=e2, split16_recon_rel_diff=abs(e2 - e_ref) / e_ref,
               oracle_damp=[r.damp_percent for r in res.subgroups], w_rel_fro=w3, split16_w_rel_fro=w2)
    _log(rec)
    assert act_bad == 0
    assert max(h_err) <= 1e-4 and max(h2_err) <= 1e-4
    assert abs(e3 - e_ref) <= 0.005 * e_ref and abs(e2 - e_ref) <= 0.005 * e_ref
    # primary flips (the first of a row) only on exact ties or within 256 ulps of one; C = 14336:
    # the reference's fp32 chain error (see test_layer_linear_parity, which measures both chains
    # against an fp64 factorisation) lets the rows' cascades grow, sanity bound 0.1 %
    for r in (rep3, rep2):
        assert r["primary"] <= n // 100000 and r.get("primary_ulps_le_256", 0) == r["primary"]
        assert r["flips"] <= (n // 1000 if C == 14336 else n // 10000)

"""Parity at the shapes of BASELINE configs[2]: the seven linears of a Llama-3-8B decoder
layer (q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096, down 4096x14336), NUM_GROUPS = 4,
w4 asym per-channel, act_order, B = 128, at a reduced token count (16 samples x 2048).  The
Hessians come from the layer's own call pattern: q/k/v and gate/up through add_batch_shared
over their shared input (gptq_plus_utils.py:6990-7039), o and down through add_batch.

Per linear, against the CPU oracle given the GPU's finalized H (the oracle cannot form these
Hessians in a test's time):
- act_square bit for bit, and the act_order permutation equal to the oracle's argsort;
- with the oracle's fp32 H^-1 injected: codes and the written weight equal (Z = 0);
- with the GPU's fp64 chain: H^-1 and H^-1_init within 1e-4 (rel. Frobenius), reconstruction
  error ||(W - Q) X^T||^2 / ||W X^T||^2 within 0.5 %, code flips <= 0.01 % -- except at
  C = 14336, where the reference's fp32 LAPACK chain itself is 6e-7 away from the exact factor
  (measured here against an fp64 factorisation on the host) while the GPU's is within fp32
  rounding of it (3e-8), so codes near a rounding boundary follow the reference's chain error:
  there the bar is 0.02 %, and the GPU's factor must be closer to the fp64 one than the
  reference's is.
Each case's numbers are printed and appended to RQ_PARITY_LOG (JSON lines) when it is set.
"""
import json
import os

import pytest
import torch

from gptq_plus_mp_quant_amd import GPTQPlus, WeightQuantizer, add_batch_shared
from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
from tests._util import rel_fro

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
        g = GPTQPlus(layer, saliency=s, gradient=grad, num_groups=G, alpha=0.0, reference_loss=0.0)
        g.quantizer = WeightQuantizer()
        g.quantizer.configure(4, perchannel=True, sym=False, mse=False)
        mods[name], objs[name], layers[name] = (W, s, grad, key), g, layer
    for key in WIDTH:
        group = [objs[n] for n, _, _, k in MODULES if k == key]
        for j in range(0, N, BSZ):
            if len(group) > 1:
                add_batch_shared(group, xs[key][j:j + BSZ])
            else:
                group[0].add_batch(xs[key][j:j + BSZ], None)
    for g in objs.values():
        g.finalize_hessian()
    torch.cuda.synchronize()
    return xs, mods, objs, layers


def _recon(W, Q, X):
    D = W.float() - Q.float()
    x = X.reshape(-1, X.shape[-1]).float()
    return float((D @ x.T).double().pow(2).sum()) / float((W.float() @ x.T).double().pow(2).sum())


@pytest.mark.parametrize("name", [m[0] for m in MODULES])
def test_layer_linear_parity(layer_state, name):
    xs, mods, objs, layers = layer_state
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
    res = o.fasterquant(**FQ)

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
    rec = dict(case=f"configs2_layer_{name}", R=R, C=C, G=G, tokens=N * T, act_square_mismatch=act_bad,
               exact_ties_in_act_square=int(C - torch.unique(o.act_square).numel()), perm_mismatch=perm_bad,
               flips_with_oracle_hinv=flips_inj, q_equal_with_oracle_hinv=q_equal, flips_own_chain=flips_own,
               codes=n, hinv_rel_fro=hinv_err, hinv_init_rel_fro=hinit_err, recon_gpu=e_gpu, recon_oracle=e_ref,
               recon_rel_diff=abs(e_gpu - e_ref) / e_ref)
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
    if C == 14336:
        assert rec["hinv_vs_fp64_host"] <= 1e-6 and rec["hinv_init_vs_fp64_host"] <= 1e-6
        assert rec["hinv_vs_fp64_host"] < rec["oracle_hinv_vs_fp64_host"]
        assert flips_own <= n // 5000
    else:
        assert flips_own <= n // 10000
    g.free()
    g2.free()

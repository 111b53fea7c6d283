"""BASELINE configs[4] at its full shape: the Llama-3-70B down_proj, W 8192 x 28672 fp16
~ N(0, 0.015^2), NUM_GROUPS = 4 (four Hessians of 28672^2 fp32, 13.2 GB, resident in HBM),
128 x 2048 calibration tokens in 16-sample add_batch chunks, w4 asym per-channel, act_order,
B = 128, alpha = 0.  The oracle cannot run at this size, so the checks are properties that
hold at any size, with torch fp64 on the GPU as the checker:

- H: random bilinear probes u^T H_g v against fp64 sums over all 262144 tokens, H exactly
  symmetric (gptq_plus_utils.py:846-850, 875-890);
- the damped Cholesky chain (:519-533) of two subgroups: U upper with a positive diagonal,
  U equal to chol(H_work^-1, upper) computed in fp64 by torch to 1e-6, H^-1_init equal to
  H_work^-1 to 1e-6, and ||U^T U H_work - I||_F / sqrt(C) small;
- every code in the fake-quantizer's range and the weight equal to fp16(scale * code);
- the proxy loss sum_g tr((W - Q) H_g (W - Q)^T) below round-to-nearest's;
- a second run bit-identical (H, codes, weight).
"""
import pytest
import torch

from gptq_plus_mp_quant_amd import GPTQPlus, WeightQuantizer
from tests._util import log_parity

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
R, C = 8192, 28672
G, N, T, BSZ = 4, 128, 2048, 16
MAXQ = 15


def _inputs(seed):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    X = torch.empty((N, T, C), dtype=torch.float16, device=DEV)
    for i in range(N):
        X[i] = torch.randn((T, C), generator=gen, device=DEV).half()
    X[:, :, torch.randperm(C, generator=gen, device=DEV)[:8]] *= 20
    W = (torch.randn((R, C), generator=gen, device=DEV) * 0.015).half()
    s = torch.exp(torch.randn((N, T, G), generator=gen, device=DEV))
    for g in range(G):
        s[..., g].clamp_(max=float(torch.quantile(s[..., g].flatten(), 0.99)))
    grad = torch.randn((R, C), generator=gen, device=DEV) * 1e-4
    return X, W, s, grad


def _run(X, W, s, grad, keep_hinv):
    layer = torch.nn.Linear(C, R, bias=False).to(DEV, torch.float16)
    layer.weight.data.copy_(W)
    g = GPTQPlus(layer, saliency=s, gradient=grad, num_groups=G, alpha=0.0, reference_loss=0.0)
    g.quantizer = WeightQuantizer()
    g.quantizer.configure(4, perchannel=True, sym=False, mse=False)
    for j in range(0, N, BSZ):
        g.add_batch(X[j:j + BSZ], None)
    g.finalize_hessian()
    H = g.H.clone()
    g.fasterquant(blocksize=128, percdamp=0.01, actorder=True, static_groups=True, export_to_et=True,
                  keep_hinv=keep_hinv)
    torch.cuda.synchronize()
    out = dict(H=H, Q=layer.weight.data.clone(), codes=g.codes.clone(), w_int=layer.int_weight,
               scale_full=layer.scale, scale=g.quantizer.scale.clone(), perm=g.perm, info=g.subgroup_info)
    if keep_hinv:
        out.update(Hinv=g.Hinv_all, Hinit=g.Hinv_init_all)
    return out


def test_configs4_full_shape_properties():
    print("configs[4]: generating 128 x 2048 x 28672 inputs", flush=True)
    X, W, s, grad = _inputs(4242)
    a = _run(X, W, s, grad, keep_hinv=True)
    print("configs[4]: first run done", flush=True)
    H = a["H"]
    assert torch.equal(H, H.transpose(1, 2))

    # H probes against fp64 sums over every token
    gen = torch.Generator(device=DEV)
    gen.manual_seed(7)
    P = 4
    U = torch.randn((C, P), generator=gen, device=DEV, dtype=torch.float64)
    V = torch.randn((C, P), generator=gen, device=DEV, dtype=torch.float64)
    exp = torch.zeros((G, P), dtype=torch.float64, device=DEV)
    mag = torch.zeros((G, P), dtype=torch.float64, device=DEV)
    for j in range(0, N, BSZ // 4):
        x = X[j:j + BSZ // 4].reshape(-1, C).double()
        sj = s[j:j + BSZ // 4].reshape(-1, G).double()
        xu, xv = x @ U, x @ V
        exp += sj.T @ (xu * xv)
        mag += sj.T @ (xu.abs() * xv.abs())
        del x
    exp /= N * T
    mag /= N * T
    got = torch.stack([(U * (H[g].double() @ V)).sum(0) for g in range(G)])
    perr = ((got - exp).abs() / mag).max().item()
    print(f"H probes: max |u'Hv - fp64| / sum|.| = {perr:.3g}", flush=True)
    rec = dict(case="configs4_full_shape_properties", R=R, C=C, G=G, tokens=N * T, h_probe_max_rel=perr)
    assert perr <= 1e-5

    # the damped Cholesky chain of two subgroups against torch fp64 on the GPU
    perm = a["perm"]
    idx = torch.arange(C, device=DEV)
    for sub in (0, 3):
        info = a["info"][sub]
        assert info["attempts"] == 1 and not info["identity_fallback"]
        Hw = H[sub][perm][:, perm].clone()
        dead = torch.diagonal(Hw) == 0
        Hw[dead, dead] = 1
        Hw[idx, idx] += float(torch.tensor(info["damp_percent"], dtype=torch.float32)) * torch.mean(torch.diagonal(Hw))
        Hw = Hw.double()
        Uk = a["Hinv"][sub]
        assert bool((torch.tril(Uk, -1) == 0).all()) and bool((torch.diagonal(Uk) > 0).all())
        Hinv64 = torch.cholesky_inverse(torch.linalg.cholesky(Hw))
        U64 = torch.linalg.cholesky(Hinv64, upper=True)
        e_u = float((Uk.double() - U64).norm() / U64.norm())
        e_i = float((a["Hinit"][sub].double() - Hinv64).norm() / Hinv64.norm())
        Ud = Uk.double()
        resid = float(((Ud.T @ Ud) @ Hw - torch.eye(C, device=DEV, dtype=torch.float64)).norm()) / C ** 0.5
        print(f"subgroup {sub}: U vs fp64 {e_u:.3g}, H^-1 vs fp64 {e_i:.3g}, ||U'U H - I||_F/sqrt(C) {resid:.3g}",
              flush=True)
        rec[f"subgroup{sub}"] = dict(u_vs_fp64=e_u, hinv_vs_fp64=e_i, resid=resid)
        assert e_u <= 1e-6 and e_i <= 1e-6
        assert resid <= 1e-2
        del Hw, Hinv64, U64, Ud
    del a["Hinv"], a["Hinit"]
    torch.cuda.empty_cache()

    # codes in range; the written weight is fp16(scale * code)
    assert int(a["codes"].min()) >= -(MAXQ + 1) and int(a["codes"].max()) <= MAXQ
    assert torch.equal(a["w_int"], a["codes"].float())
    assert torch.equal(a["Q"], (a["scale_full"] * a["w_int"]).half())

    # the error feedback beats round-to-nearest on the proxy loss
    Wf = W.float()
    rtn = (torch.clamp(torch.round(Wf / a["scale"]), -(MAXQ + 1), MAXQ) * a["scale"]).half()

    def proxy(Q):
        D = (W.double() - Q.double()).reshape(G, R // G, C)
        return sum(float(((D[g] @ H[g].double()) * D[g]).sum()) for g in range(G))
    e_q, e_r = proxy(a["Q"]), proxy(rtn)
    print(f"proxy loss: GPTQ+ {e_q:.6g}  RTN {e_r:.6g}  ratio {e_q / e_r:.3f}", flush=True)
    rec.update(proxy_gptqplus=e_q, proxy_rtn=e_r)
    assert e_q < e_r

    # determinism
    b = _run(X, W, s, grad, keep_hinv=False)
    same = {k: bool(torch.equal(a[k], b[k])) for k in ("H", "codes", "Q")}
    rec["second_run_identical"] = same
    log_parity(rec)
    for k, v in same.items():
        assert v, k

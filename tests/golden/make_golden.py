"""Write golden vectors by running the REFERENCE implementation on CPU, in this container only.

Run:  python tests/golden/make_golden.py [/root/reference]

Only this script touches the reference, and only to record input/output vectors for the
parts that no closed form or brute-force check pins (``compute_safe_beta_from_reference_loss``
and ``_compute_gradient_terms`` with alpha > 0, the static/dynamic group + block-atomic +
last-block-fallback combinations, the asym ``fake_quantize`` quirk inside ``fasterquant``).
Each case drives ``GPTQPlus`` exactly like ``accumulate_hessian_for_gptq`` and the
``fasterquant`` call of ``gptq_fwrd`` (gptq_plus_utils.py:6954-7039, 7467-7502), on
seeded CPU tensors.  The reference imports ``loguru`` (absent here) via
``utils/memory_utils.py:5``; a minimal logger stand-in is registered for the import.
``GPTQPlus.free`` is never called (it synchronises CUDA).

The vectors (inputs + outputs) are stored compressed in ``tests/golden/golden_cases.npz``.
"""
from __future__ import annotations

import importlib
import json
import logging
import sys
import types
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
OUT = HERE / "golden_cases.npz"
sys.path.insert(0, str(HERE))
from fixtures import quadratic_refresh  # noqa: E402  (data helper, no reference code)

# Case table.  R rows, C columns, G groups, N samples x T tokens, bits/sym, groupsize,
# act_order, blocksize, atomic, alpha/ref_loss, special input shaping.
CASES = [
    dict(name="g1_sym4_perchan_act", R=32, C=128, G=1, N=8, T=32, bits=4, sym=True, gs=-1, act=True, B=32, atomic=False, alpha=0.0, ref_loss=0.0),
    dict(name="g4_asym4_perchan_act_gplus", R=64, C=64, G=4, N=8, T=16, bits=4, sym=False, gs=-1, act=True, B=16, atomic=False, alpha=0.05, ref_loss=100.0, gscale=0.1),
    dict(name="g2_sym3_static_groups_act", R=32, C=64, G=2, N=8, T=16, bits=3, sym=True, gs=16, act=True, B=16, atomic=False, alpha=0.0, ref_loss=0.0),
    dict(name="g1_sym4_dynamic_groups", R=32, C=64, G=1, N=8, T=16, bits=4, sym=True, gs=16, act=False, B=16, atomic=False, alpha=0.0, ref_loss=0.0),
    dict(name="g4_sym4_atomic_perchan_act", R=64, C=64, G=4, N=8, T=16, bits=4, sym=True, gs=-1, act=True, B=16, atomic=True, alpha=0.0, ref_loss=0.0),
    dict(name="g2_sym4_atomic_dynamic_C48", R=32, C=48, G=2, N=8, T=16, bits=4, sym=True, gs=16, act=False, B=16, atomic=True, alpha=0.0, ref_loss=0.0),
    dict(name="g2_sym4_atomic_static_gplus", R=32, C=64, G=2, N=8, T=16, bits=4, sym=True, gs=16, act=True, B=16, atomic=True, alpha=0.05, ref_loss=1e6, gscale=1.0),
    dict(name="g1_sym4_ragged_C50_B32", R=32, C=50, G=1, N=8, T=16, bits=4, sym=True, gs=-1, act=False, B=32, atomic=False, alpha=0.0, ref_loss=0.0),
    dict(name="g2_asym4_deadcols_zero_rows", R=32, C=64, G=2, N=8, T=16, bits=4, sym=False, gs=-1, act=True, B=16, atomic=False, alpha=0.0, ref_loss=0.0, dead=True),
    dict(name="g1_sym4_indefinite_retry", R=16, C=32, G=1, N=4, T=16, bits=4, sym=True, gs=-1, act=True, B=16, atomic=False, alpha=0.0, ref_loss=0.0, negsal=0.35),
    dict(name="g1_sym4_indefinite_identity", R=16, C=32, G=1, N=4, T=16, bits=4, sym=True, gs=-1, act=False, B=16, atomic=False, alpha=0.0, ref_loss=0.0, negsal=50.0),
    dict(name="g2_sym4_mse_perchan_act", R=32, C=64, G=2, N=8, T=16, bits=4, sym=True, gs=-1, act=True, B=16, atomic=False, alpha=0.0, ref_loss=0.0, mse=True),
    dict(name="g2_asym3_mse_static_groups", R=32, C=64, G=2, N=8, T=16, bits=3, sym=False, gs=16, act=True, B=16, atomic=False, alpha=0.0, ref_loss=0.0, mse=True),
    dict(name="g1_sym4_mse_dynamic_atomic", R=32, C=48, G=1, N=8, T=16, bits=4, sym=True, gs=16, act=False, B=16, atomic=True, alpha=0.0, ref_loss=0.0, mse=True),
    dict(name="g2_sym4_surrogate_block_gplus", R=32, C=64, G=2, N=8, T=16, bits=4, sym=True, gs=-1, act=True, B=16, atomic=False, alpha=0.05, ref_loss=100.0, gscale=0.1, mode="surrogate_block"),
    dict(name="g2_asym4_surrogate_online_gplus", R=32, C=64, G=2, N=8, T=16, bits=4, sym=False, gs=16, act=True, B=16, atomic=False, alpha=0.05, ref_loss=100.0, gscale=0.1, mode="surrogate_online"),
    dict(name="g2_sym4_surrogate_online_atomic", R=32, C=48, G=2, N=8, T=16, bits=4, sym=True, gs=-1, act=True, B=16, atomic=True, alpha=0.05, ref_loss=100.0, gscale=0.1, mode="surrogate_online"),
    # block_gd / block_backward with a deterministic quadratic refresh (fixtures.quadratic_refresh)
    dict(name="g2_sym4_block_gd_sgd", R=32, C=64, G=2, N=8, T=16, bits=4, sym=True, gs=-1, act=True, B=16, atomic=False, alpha=0.05, ref_loss=100.0, gscale=0.1, mode="block_gd",
         fq=dict(grad_optimizer="sgd", grad_lr=8e-3, grad_reg_strategy="none", second_order_scale=1.0, grad_clip=1.0)),
    dict(name="g2_asym4_block_gd_adam_l2", R=32, C=64, G=2, N=8, T=16, bits=4, sym=False, gs=-1, act=True, B=16, atomic=False, alpha=0.05, ref_loss=100.0, gscale=0.1, mode="block_gd",
         fq=dict(grad_optimizer="adam", grad_lr=4e-3, grad_reg_strategy="l2", grad_reg_lambda=0.5, second_order_scale=0.9, grad_clip=0.5, slide_refresh_start=1, slide_refresh_block_total=6)),
    dict(name="g2_sym4_block_gd_hadam_hessian", R=32, C=64, G=2, N=8, T=16, bits=4, sym=True, gs=-1, act=False, B=16, atomic=False, alpha=0.05, ref_loss=100.0, gscale=0.1, mode="block_gd",
         fq=dict(grad_optimizer="h_adam", grad_lr=4e-3, grad_reg_strategy="hessian", grad_reg_lambda=0.1, curvature_damping=0.1, grad_clip=1.0)),
    dict(name="g2_sym4_block_gd_adam_gateopt_static", R=32, C=64, G=2, N=8, T=16, bits=4, sym=True, gs=16, act=True, B=16, atomic=False, alpha=0.05, ref_loss=100.0, gscale=0.1, mode="block_gd",
         fq=dict(grad_optimizer="adam", grad_lr=4e-3, grad_reg_strategy="quant_error_gate_optimized", grad_gate_floor=0.2, grad_gate_sharpness=2.0, grad_gate_sine_amp=0.001, grad_clip=1.0)),
    dict(name="g2_asym4_block_gd_sgd_gate_atomic", R=32, C=48, G=2, N=8, T=16, bits=4, sym=False, gs=-1, act=True, B=16, atomic=True, alpha=0.05, ref_loss=100.0, gscale=0.1, mode="block_gd",
         fq=dict(grad_optimizer="sgd", grad_lr=8e-3, grad_reg_strategy="quant_error_gate", grad_gate_floor=0.1, grad_gate_sharpness=1.0, second_order_scale=0.8, grad_clip=1.0)),
    dict(name="g2_sym4_block_backward", R=32, C=64, G=2, N=8, T=16, bits=4, sym=True, gs=-1, act=True, B=16, atomic=False, alpha=0.05, ref_loss=100.0, gscale=0.1, mode="block_backward"),
    dict(name="g2_asym4_block_backward_dyn_atomic", R=32, C=48, G=2, N=8, T=16, bits=4, sym=False, gs=16, act=False, B=16, atomic=True, alpha=0.05, ref_loss=100.0, gscale=0.1, mode="block_backward"),
]


# Classic GPTQ (gptq_utils/gptq_utils.py:23-180), driven like gptq_fwrd (:236-284): one
# add_batch per calibration sample, static_groups = act_order unless stated.
GPTQ_CASES = [
    dict(name="gptq_sym4_perchan_act", R=32, C=64, N=8, T=16, bits=4, sym=True, gs=-1, act=True, B=16),
    dict(name="gptq_asym4_static_act", R=32, C=64, N=8, T=16, bits=4, sym=False, gs=16, act=True, B=16),
    dict(name="gptq_sym3_dynamic_gs16_B32", R=32, C=64, N=8, T=16, bits=3, sym=True, gs=16, act=False, B=32),
    dict(name="gptq_sym4_dynamic_gs32_B16", R=32, C=64, N=8, T=16, bits=4, sym=True, gs=32, act=False, B=16),
    dict(name="gptq_asym4_dynamic_act", R=32, C=64, N=8, T=16, bits=4, sym=False, gs=16, act=True, B=16, static=False),
    dict(name="gptq_sym4_deadcols_ragged", R=32, C=50, N=8, T=16, bits=4, sym=True, gs=-1, act=True, B=32, dead=True),
    dict(name="gptq_asym4_mse_static", R=32, C=64, N=8, T=16, bits=4, sym=False, gs=32, act=True, B=16, mse=True),
    dict(name="gptq_sym4_nodata", R=32, C=64, N=0, T=16, bits=4, sym=True, gs=-1, act=False, B=16),
]


def synth_inputs(case, seed):
    """Seeded synthetic inputs (numpy PCG64), shaped like BASELINE.json's configs."""
    rng = np.random.Generator(np.random.PCG64(seed))
    R, C, G, N, T = case["R"], case["C"], case["G"], case["N"], case["T"]
    X = rng.standard_normal((N, T, C), dtype=np.float32)
    out_ch = rng.choice(C, size=min(4, C), replace=False)
    X[:, :, out_ch] *= 20.0
    W = (rng.standard_normal((R, C), dtype=np.float32) * 0.02)
    s = rng.lognormal(0.0, 1.0, size=(N, T, G)).astype(np.float32)
    for g in range(G):
        s[..., g] = np.minimum(s[..., g], np.quantile(s[..., g], 0.99))
    grad = (rng.standard_normal((R, C), dtype=np.float32) * case.get("gscale", 1e-4))
    if case.get("dead"):
        X[:, :, :5] = 0.0          # dead channels -> diag(H) == 0
        W[3, :] = 0.0              # all-zero row -> asym (-1, +1) branch
        X[:, :, 10] = X[:, :, 11]  # duplicated channel -> exact tie in act_square
    if case.get("negsal"):
        s[..., 0] -= case["negsal"] * s[..., 0].mean()   # indefinite H -> damping retries
    return (X.astype(np.float16), W.astype(np.float16), s, grad)


class _Capture:
    """Duck-typed diagnostic recorder (save_module_level / save_subgroup / save_block)."""

    def __init__(self):
        self.module = {}
        self.sub = {}

    def save_module_level(self, tag, tensor):
        if tensor is not None:
            self.module[tag] = tensor.detach().clone()

    def save_subgroup(self, sub_idx, tag, tensor):
        if tensor is not None:
            self.sub[(sub_idx, tag)] = tensor.detach().clone()

    def save_block(self, *a, **k):
        return None

    def record_loss(self, *a, **k):
        return None


def _upper(a):
    """Row-major upper triangle (incl. diagonal) of a square matrix: H, Hinv_init are exactly
    symmetric after the reference's symmetrisation / potri, Hinv is upper triangular."""
    return a[np.triu_indices(a.shape[0])]


def _import_reference(ref_root):
    if "loguru" not in sys.modules:
        lg = types.ModuleType("loguru")
        lg.logger = logging.getLogger("loguru-standin")
        sys.modules["loguru"] = lg
    sys.path.insert(0, str(ref_root))
    from gptq_utils import gptq_plus_utils as gpu
    from utils import quant_utils as qu
    return gpu, qu


def run_case(gpu, qu, case, seed):
    X, W, s, grad = synth_inputs(case, seed)
    torch.manual_seed(seed)
    layer = torch.nn.Linear(case["C"], case["R"], bias=False).to(torch.float16)
    layer.weight.data.copy_(torch.from_numpy(W))
    g = gpu.GPTQPlus(layer, saliency=torch.from_numpy(s), gradient=torch.from_numpy(grad),
                     num_groups=case["G"], alpha=case["alpha"], reference_loss=case["ref_loss"])
    g.quantizer = qu.WeightQuantizer()
    g.quantizer.configure(case["bits"], perchannel=True, sym=case["sym"], mse=case.get("mse", False))
    xs = torch.from_numpy(X)
    for j in range(0, xs.shape[0], 4):
        g.add_batch(xs[j:j + 4].data, None)
    g.finalize_hessian()
    H = g.H.clone()
    act = g.act_square.clone()
    cap = _Capture()
    extra = dict(case.get("fq", {}))
    if case.get("mode") in ("block_gd", "block_backward"):
        extra["gradient_refresh_fn"] = quadratic_refresh(X, W, grad)
    g.fasterquant(blocksize=case["B"], percdamp=0.01, groupsize=case["gs"], actorder=case["act"],
                  static_groups=case["act"], enable_gradient_update=True,
                  g_update_mode=case.get("mode", "frozen"),
                  export_to_et=True, block_atomic_quant=case["atomic"], diagnostic_recorder=cap,
                  **extra)
    out = {
        "X": X, "W": W, "s": s, "grad": grad,
        "H_upper": np.stack([_upper(h) for h in H.numpy()]), "act_square": act.numpy(),
        "Q": layer.weight.data.numpy(), "W_int": layer.int_weight.numpy().astype(np.int8),
        "Scale": layer.scale.numpy(),
        "qscale": g.quantizer.scale.numpy(), "qzero": g.quantizer.zero.numpy(),
    }
    for sub in range(case["G"]):
        for tag in ("Hinv_init", "Hinv_upper_cholesky", "beta", "Z_initial", "GHinv_initial", "perm"):
            t = cap.sub.get((sub, tag))
            if t is not None:
                a = t.numpy()
                if tag in ("Hinv_init", "Hinv_upper_cholesky"):
                    a = _upper(a)
                out[f"sub{sub}_{tag}"] = a
        fb = cap.sub.get((sub, "hessian_identity_fallback"))
        if fb is not None:
            out[f"sub{sub}_identity_fallback"] = np.asarray(bool(fb.item()))
    return out


def run_gptq_case(gq, qu, case, seed):
    c = dict(case, G=1, N=max(case["N"], 1))
    X, W, s, grad = synth_inputs(c, seed)
    layer = torch.nn.Linear(case["C"], case["R"], bias=False).to(torch.float16)
    layer.weight.data.copy_(torch.from_numpy(W))
    g = gq.GPTQ(layer)
    g.quantizer = qu.WeightQuantizer()
    g.quantizer.configure(case["bits"], perchannel=True, sym=case["sym"], mse=case.get("mse", False))
    xs = torch.from_numpy(X)
    for j in range(case["N"]):
        g.add_batch(xs[j].unsqueeze(0).data, None)
    H = g.H.clone()
    sync = torch.cuda.synchronize
    torch.cuda.synchronize = lambda *a, **k: None       # fasterquant synchronises CUDA
    try:
        g.fasterquant(blocksize=case["B"], percdamp=0.01, groupsize=case["gs"], actorder=case["act"],
                      static_groups=case.get("static", case["act"]), export_to_et=True)
    finally:
        torch.cuda.synchronize = sync
    return {"X": X[:case["N"]], "W": W, "H_upper": _upper(H.numpy())[None], "Q": layer.weight.data.numpy(),
            "W_int": layer.int_weight.numpy().astype(np.int8), "Scale": layer.scale.numpy(),
            "qscale": g.quantizer.scale.numpy(), "qzero": g.quantizer.zero.numpy()}


def beta_vectors(gpu):
    """compute_safe_beta_from_reference_loss on seeded inputs incl. its clamp / where branches."""
    rng = np.random.Generator(np.random.PCG64(1234))
    vecs = {}
    for k, (R, C, ref_loss, alpha, gsc) in enumerate([
            (16, 24, 1e-3, 0.05 / (16 * 24), 1.0),     # typical: ratio in (0, 1)
            (16, 24, 0.0, 0.05 / (16 * 24), 1.0),      # ref_loss <= 0 -> beta = 0
            (8, 12, 10.0, 0.5, 1e-3),                  # large target -> ratio clamps at 1
            (8, 12, 1e-6, 1e-4, 10.0)]):               # tiny target -> beta ~ 0
        G = rng.standard_normal((R, C)).astype(np.float32) * gsc
        A = rng.standard_normal((C, C)).astype(np.float32)
        Hinv_init = (A @ A.T / C + np.eye(C, dtype=np.float32)).astype(np.float32)
        beta, gh = gpu.compute_safe_beta_from_reference_loss(
            torch.from_numpy(G), torch.from_numpy(Hinv_init), ref_loss, alpha)
        vecs[f"beta{k}_G"] = G
        vecs[f"beta{k}_Hinv_init"] = Hinv_init
        vecs[f"beta{k}_params"] = np.asarray([ref_loss, alpha], dtype=np.float64)
        vecs[f"beta{k}_beta"] = beta.numpy()
        vecs[f"beta{k}_ghinv_init"] = gh.numpy()
    return vecs


def main():
    ref_root = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
    torch.backends.cuda.matmul.allow_tf32 = False
    gpu, qu = _import_reference(ref_root)
    arrays = {}
    meta = []
    for k, case in enumerate(CASES):
        seed = 1000 + k
        out = run_case(gpu, qu, case, seed)
        for key, val in out.items():
            arrays[f"{case['name']}__{key}"] = val
        meta.append(dict(case, seed=seed))
        print(f"case {case['name']}: codes={out['W_int'].size} "
              f"fallback={[out.get(f'sub{s}_identity_fallback') for s in range(case['G'])]}")
    arrays.update(beta_vectors(gpu))
    gq = importlib.import_module("gptq_utils.gptq_utils")
    for k, case in enumerate(GPTQ_CASES):
        seed = 3000 + k
        out = run_gptq_case(gq, qu, case, seed)
        for key, val in out.items():
            arrays[f"{case['name']}__{key}"] = val
        meta.append(dict(case, G=1, kind="gptq", seed=seed))
        print(f"gptq case {case['name']}: codes={out['W_int'].size}")
    arrays["__meta__"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    arrays["__torch_version__"] = np.frombuffer(torch.__version__.encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size / 1024:.1f} KiB)")


if __name__ == "__main__":
    main()

"""Benchmark: ms per linear (Hessian accumulation + GPTQ+ fasterquant) on one MI355X.

Workload: one 4096x4096 q_proj linear, fp16 W ~ N(0, 0.02^2);
calibration X = 128 samples x 2048 tokens x 4096 fp16 ~ N(0,1) with 8 outlier channels x20;
NUM_GROUPS = 4 token saliencies ~ LogNormal(0,1) clipped at their 0.99 quantile; GPTQ+
first-order term on with G ~ N(0, 1e-4^2) and alpha = 0; w4 asymmetric per-channel,
act_order, BLOCKSIZE = 128, percdamp = 0.01; 16-sample add_batch chunks.
A step = one linear: 8 add_batch calls + finalize_hessian + fasterquant, inputs resident in
HBM.  Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
  python bench.py --config cfg3|cfg4 [--cpu-baseline-layer]   # a whole Llama-3-8B layer
  python bench.py --config cfg5 [--cpu-baseline-sample]       # Llama-3-70B down_proj
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_MFMA_PEAK_TFLOPS = 157.3
FP16_MFMA_PEAK_TFLOPS = 2500.0      # dense fp16 / bf16 MFMA
SPLIT_PIECES = 3                    # fp16 MFMA products per exact fp32 product (split16 kernel)


def hessian_roofline(flops, ms, math, extra):
    """Roofline object for the Hessian accumulation.  `flops` counts 2 per (token, i <= j)
    element of every Hessian.  split16 runs on the fp16 MFMA pipe and needs SPLIT_PIECES fp16
    products per fp32 product, so its bound is the fp16 peak against SPLIT_PIECES x flops; the
    fp32-equivalent rate (flops / time against the fp32 MFMA peak) is what the metric's
    "% fp32-MFMA peak" reads."""
    eq = flops / (ms * 1e-3) / 1e12
    if math == "split16":
        ach, peak = SPLIT_PIECES * eq, FP16_MFMA_PEAK_TFLOPS
        kernel = "k_hessian_split<__half> (timed with its k_xprep + k_xfinish pre-pass)"
    else:
        ach, peak = eq, FP32_MFMA_PEAK_TFLOPS
        kernel = "k_hessian_accum<__half>"
    out = {"bound": "mfma", "achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s",
           "frac": round(ach / peak, 4), "kernel": kernel, "math": math,
           "fp32_equivalent": {"achieved": round(eq, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
                               "frac": round(eq / FP32_MFMA_PEAK_TFLOPS, 4)}}
    out.update(extra)
    return out

CFG = dict(R=4096, C=4096, G=4, N=128, T=2048, bsz=16, bits=4, sym=False, blocksize=128,
           percdamp=0.01, alpha=0.0, outliers=8, seed=20251201, wscale=0.02)
# the Llama-3-70B down_proj, one GPU's full share (4 Hessians of 28672^2 fp32)
CFG5 = dict(CFG, R=8192, C=28672, wscale=0.015)


def make_inputs(dev, cfg):
    """Synthetic inputs generated on the GPU from a fixed seed (torch Philox)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(cfg["seed"])
    N, T, C, R, G = cfg["N"], cfg["T"], cfg["C"], cfg["R"], cfg["G"]
    X = torch.empty((N, T, C), dtype=torch.float16, device=dev)
    for i in range(N):
        X[i] = torch.randn((T, C), generator=gen, device=dev, dtype=torch.float32).half()
    out_ch = torch.randperm(C, generator=gen, device=dev)[: cfg["outliers"]]
    X[:, :, out_ch] *= 20
    W = (torch.randn((R, C), generator=gen, device=dev) * cfg["wscale"]).half()
    s = torch.exp(torch.randn((N, T, G), generator=gen, device=dev))
    for g in range(G):
        q = torch.quantile(s[..., g].flatten(), 0.99)          # linear interpolation
        s[..., g].clamp_(max=float(q))
    grad = torch.randn((R, C), generator=gen, device=dev) * 1e-4
    return X, W, s, grad


# a full Llama-3-8B decoder layer; modules that read the same input share one X
LAYER8B = [("q_proj", 4096, 4096, "attn"), ("k_proj", 1024, 4096, "attn"), ("v_proj", 1024, 4096, "attn"),
           ("o_proj", 4096, 4096, "o"), ("gate_proj", 14336, 4096, "mlp"), ("up_proj", 14336, 4096, "mlp"),
           ("down_proj", 4096, 14336, "down")]


def hadamard(n, dev):
    """Sylvester Hadamard matrix of order n (a power of two), fp32."""
    H = torch.ones((1, 1), device=dev)
    while H.shape[0] < n:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return H


def rotation(C, gen, dev):
    """configs[3]'s seeded orthogonal rotation: diag(+-1) H_C / sqrt(C) for a power of two,
    Q_k (x) (diag(+-1) H_m / sqrt(m)) for C = k * m (QuaRot-style; C = 14336 = 7 * 2048)."""
    m = 1 << (C.bit_length() - 1)
    while C % m:
        m >>= 1
    k = C // m
    signs = torch.randint(0, 2, (m,), generator=gen, device=dev).float() * 2 - 1
    Hm = signs[:, None] * hadamard(m, dev) / (m ** 0.5)
    if k == 1:
        return Hm
    Qk, _ = torch.linalg.qr(torch.randn((k, k), generator=gen, device=dev).cpu())
    return torch.kron(Qk.contiguous().to(dev), Hm.contiguous())


def rotate_(X, Rm):
    """X <- X R in place, one calibration sample at a time (fp32 product, fp16 result)."""
    for i in range(X.shape[0]):
        X[i] = (X[i].float() @ Rm).half()


def make_layer_inputs(dev, cfg):
    gen = torch.Generator(device=dev)
    gen.manual_seed(cfg["seed"] + 1)
    N, T, G = cfg["N"], cfg["T"], cfg["G"]
    xs, rots = {}, {}
    for key, C in (("attn", 4096), ("o", 4096), ("mlp", 4096), ("down", 14336)):
        X = torch.empty((N, T, C), dtype=torch.float16, device=dev)
        for i in range(N):
            X[i] = torch.randn((T, C), generator=gen, device=dev, dtype=torch.float32).half()
        X[:, :, torch.randperm(C, generator=gen, device=dev)[: cfg["outliers"]]] *= 20
        if cfg.get("rotate"):
            rots[key] = rotation(C, gen, dev)
            rotate_(X, rots[key])
        xs[key] = X
    mods = {}
    for name, R, C, key in LAYER8B:
        W = (torch.randn((R, C), generator=gen, device=dev) * 0.02).half()
        if cfg.get("rotate"):
            W = (W.float() @ rots[key]).half()                 # W' = W R keeps X' W'^T = X W^T
        s = torch.exp(torch.randn((N, T, G), generator=gen, device=dev))
        for g in range(G):
            s[..., g].clamp_(max=float(torch.quantile(s[..., g].flatten(), 0.99)))
        grad = torch.randn((R, C), generator=gen, device=dev) * 1e-4
        mods[name] = (W, s, grad, key)
    return xs, mods


def one_layer(xs, mods, cfg, layers, timer=None):
    """Hessians of all 7 linears (shared inputs fused) + finalize + fasterquant of each."""
    from gptq_plus_mp_quant_amd import GPTQPlus, WeightQuantizer, add_batch_shared
    objs = {}
    for name, (W, s, grad, key) in mods.items():
        layers[name].weight.data.copy_(W)
        g = GPTQPlus(layers[name], saliency=s, gradient=grad, num_groups=cfg["G"], alpha=cfg["alpha"],
                     reference_loss=0.0)
        g.quantizer = WeightQuantizer()
        g.quantizer.configure(cfg["bits"], perchannel=True, sym=cfg["sym"], mse=False)
        objs[name] = g
    fq = fq_kwargs(cfg)
    for key in ("attn", "o", "mlp", "down"):
        group = [objs[n] for n, _, _, k in LAYER8B if k == key]
        for j in range(0, cfg["N"], cfg["bsz"]):
            if timer is not None:
                timer.start()
            add_batch_shared(group, xs[key][j:j + cfg["bsz"]])
            if timer is not None:
                timer.stop()
    for g in objs.values():
        g.finalize_hessian()
    for g in objs.values():
        g.fasterquant(**fq)
        g.free()
    return objs


def fq_kwargs(cfg):
    """fasterquant arguments of a config: configs[1..2] per-channel + act_order (static_groups
    follows act_order like the driver, :7472); configs[3] dynamic 128-column groups + atomic."""
    act = cfg.get("actorder", True)
    return dict(blocksize=cfg["blocksize"], percdamp=cfg["percdamp"], groupsize=cfg.get("groupsize", -1),
                actorder=act, static_groups=act, block_atomic_quant=cfg.get("atomic", False))


def layer_hessian_flops(cfg):
    ntok = cfg["N"] * cfg["T"]
    return sum(cfg["G"] * ntok * C * (C + 1) for _, _, C, _ in LAYER8B)


def cpu_baseline_layer(xs, mods, cfg):
    """CPU oracle for configs[2]: per input width, one add_batch chunk is timed and scaled by
    tokens (x N/bsz); every module's finalize_hessian + fasterquant is timed in full."""
    from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
    nchunks = cfg["N"] // cfg["bsz"]
    total, parts = 0.0, []
    for name, R, C, key in LAYER8B:
        W, s, grad, _ = mods[name]
        o = GPTQPlusOracle(W.cpu(), s.cpu(), grad.cpu(), cfg["G"], cfg["alpha"], 0.0)
        o.quantizer = make_quantizer(cfg["bits"], cfg["sym"])
        xc = xs[key][: cfg["bsz"]].cpu()
        t0 = time.perf_counter()
        o.add_batch(xc)
        t_acc = time.perf_counter() - t0
        o.index, o.token_count = cfg["N"], cfg["N"] * cfg["T"]
        t1 = time.perf_counter()
        o.finalize_hessian()
        o.fasterquant(**fq_kwargs(cfg))
        t_fq = time.perf_counter() - t1
        total += t_acc * nchunks + t_fq
        parts.append(f"{name}: 1/{nchunks} chunk {t_acc:.1f}s, fasterquant {t_fq:.1f}s")
        print(f"cpu baseline {name}: add_batch chunk {t_acc:.1f} s, finalize+fasterquant {t_fq:.1f} s",
              flush=True)
    return dict(value=round(total * 1e3 / len(LAYER8B), 1), unit="ms per linear (layer / 7, extrapolated)",
                cores=torch.get_num_threads(), kind="port",
                sample="oracle on host CPU; " + "; ".join(parts) + f"; layer {total:.1f} s")


CFG4 = dict(CFG, sym=True, groupsize=128, actorder=False, atomic=True, rotate=True)
WORKLOAD = {
    "cfg3": "configs[2]: Llama-3-8B decoder layer, 7 linears (q/k/v and gate/up Hessians fused over "
            "their shared input), NUM_GROUPS=4, 128x2048 tokens, w4 asym per-channel, act_order, B=128; "
            "value = layer time / 7, ms_per_step = layer",
    "cfg4": "configs[3]: Llama-3-8B decoder layer, seeded orthogonal (Hadamard-based) rotation of W and X, "
            "w4 sym, 128-column dynamic groups, BLOCK_ATOMIC_QUANT, NUM_GROUPS=4, 128x2048 tokens; "
            "value = layer time / 7, ms_per_step = layer",
}


def run_layer(args, dev):
    cfg = dict(CFG4 if args.config == "cfg4" else CFG)
    xs, mods = make_layer_inputs(dev, cfg)
    layers = {n: torch.nn.Linear(C, R, bias=False).to(dev, torch.float16) for n, R, C, _ in LAYER8B}
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        one_layer(xs, mods, cfg, layers)
    timer = EventTimer()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_layer(xs, mods, cfg, layers, timer)
    torch.cuda.synchronize()
    layer_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    h_ms_mean, n_launch = timer.mean_ms()
    h_ms_layer = h_ms_mean * n_launch / args.steps
    line = {
        "metric": "ms per linear (H-accum + fasterquant) at Llama-8B shapes; % fp32-MFMA peak",
        "value": round(layer_ms / len(LAYER8B), 2), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(layer_ms, 2), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32 (fp16 inputs; exact fp32 products)",
        "data": "synthetic (seeded, generated on the GPU)",
        "config": {"workload": WORKLOAD[args.config], "parallelism": "single GPU"},
        "roofline": hessian_roofline(layer_hessian_flops(cfg), h_ms_layer, args.hessian_math,
                                     {"traffic": None, "hessian_ms_per_layer": round(h_ms_layer, 2),
                                      "launches_per_layer": n_launch // args.steps,
                                      "flops_per_layer": layer_hessian_flops(cfg)}),
    }
    if args.cpu_baseline_layer:
        line["cpu_baseline"] = cpu_baseline_layer(xs, mods, cfg)
    print(json.dumps(line), flush=True)


def one_linear(X, W, s, grad, cfg, layer, timer=None):
    from gptq_plus_mp_quant_amd import GPTQPlus, WeightQuantizer
    layer.weight.data.copy_(W)
    g = GPTQPlus(layer, saliency=s, gradient=grad, num_groups=cfg["G"], alpha=cfg["alpha"], reference_loss=0.0)
    g.quantizer = WeightQuantizer()
    g.quantizer.configure(cfg["bits"], perchannel=True, sym=cfg["sym"], mse=False)
    for j in range(0, cfg["N"], cfg["bsz"]):
        if timer is not None:
            timer.start()
        g.add_batch(X[j:j + cfg["bsz"]], None)
        if timer is not None:
            timer.stop()
    g.finalize_hessian()
    g.fasterquant(**fq_kwargs(cfg))
    return g


class EventTimer:
    """HIP events on the stream the Hessian kernel is launched on (torch's current stream)."""

    def __init__(self):
        self.pairs = []

    def start(self):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs.append([e, None])

    def stop(self):
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.pairs[-1][1] = e

    def mean_ms(self):
        torch.cuda.synchronize()
        ts = [a.elapsed_time(b) for a, b in self.pairs]
        return sum(ts) / len(ts), len(ts)


def cpu_baseline(X, W, s, grad, cfg, chunks=2):
    """Time the CPU oracle (the reference's torch op sequence) on a bounded sample:
    `chunks` of the 8 add_batch calls (extrapolated linearly in tokens) plus the full
    finalize_hessian + fasterquant of the same linear."""
    from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
    threads = torch.get_num_threads()
    Xc = X[: chunks * cfg["bsz"]].cpu()
    sc, Wc, gc = s.cpu(), W.cpu(), grad.cpu()
    o = GPTQPlusOracle(Wc, sc, gc, cfg["G"], cfg["alpha"], 0.0)
    o.quantizer = make_quantizer(cfg["bits"], cfg["sym"])
    t0 = time.perf_counter()
    for j in range(0, Xc.shape[0], cfg["bsz"]):
        o.add_batch(Xc[j:j + cfg["bsz"]])
    t_acc = time.perf_counter() - t0
    # the remaining chunks only add to H; scale the measured accumulation time by tokens
    o.index = cfg["N"]
    o.token_count = cfg["N"] * cfg["T"]
    t1 = time.perf_counter()
    o.finalize_hessian()
    o.fasterquant(**fq_kwargs(cfg))
    t_fq = time.perf_counter() - t1
    nchunks = cfg["N"] // cfg["bsz"]
    total_s = t_acc * nchunks / chunks + t_fq
    return dict(value=round(total_s * 1e3, 1), unit="ms per linear (extrapolated)", cores=threads,
                kind="port",
                sample=(f"oracle (reference torch op sequence) on host CPU: {chunks}/{nchunks} add_batch "
                        f"chunks timed ({t_acc:.1f} s, x{nchunks // chunks} by tokens) + full "
                        f"finalize_hessian+fasterquant ({t_fq:.1f} s); {platform.processor() or platform.machine()}"))


def cpu_baseline_hessian_sample(X, s, cfg, samples=1):
    """configs[4] on the host is hours of work; time the oracle's add_batch on `samples` of the
    128 calibration samples and extrapolate by tokens.  A lower bound of the CPU path: the
    CPU finalize_hessian + fasterquant (four 28672^2 Cholesky chains, the block loop) are left out."""
    from oracle.gptqplus_cpu import GPTQPlusOracle
    C, G = cfg["C"], cfg["G"]
    o = GPTQPlusOracle(torch.zeros(G, C), s[:samples].cpu(), torch.zeros(G, C), G, 0.0, 0.0)
    xc = X[:samples].cpu()
    t0 = time.perf_counter()
    o.add_batch(xc)
    t = time.perf_counter() - t0
    scale = cfg["N"] // samples
    return dict(value=round(t * scale * 1e3, 1), unit="ms per linear (Hessian accumulation only, extrapolated)",
                cores=torch.get_num_threads(), kind="port",
                sample=(f"oracle add_batch on {samples}/{cfg['N']} samples ({t:.1f} s, x{scale} by tokens); "
                        "finalize_hessian + fasterquant not timed, so this is a lower bound"))


def copy_calibration(dev, nbytes=1 << 30, reps=3):
    """A plain device-to-device copy of known size, profiled with the same FETCH_SIZE /
    WRITE_SIZE counters to calibrate them (bytes moved = nbytes read + nbytes written)."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "reps": reps}), flush=True)


def gemm_calibration(dev):
    """Practical GEMM ceilings on this GPU: torch.matmul (hipBLASLt / rocBLAS) on large square
    operands in fp16, fp32 (TF32 off) and fp64, as TFLOP/s.  The split Hessian kernel's products
    run on the fp16 pipe, the Cholesky chain on the fp64 pipe, the trailing update on fp32."""
    torch.backends.cuda.matmul.allow_tf32 = False
    out = {}
    for name, dt, n, reps in (("fp16", torch.float16, 8192, 20), ("fp32", torch.float32, 8192, 5),
                              ("fp64", torch.float64, 8192, 3)):
        a = torch.randn(n, n, device=dev).to(dt)
        b = torch.randn(n, n, device=dev).to(dt)
        for _ in range(2):
            c = a @ b
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            c = a @ b
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out[name] = {"n": n, "ms": round(ms, 3), "tflops": round(2 * n ** 3 / ms / 1e9, 1)}
        del a, b, c
    print(json.dumps({"gemm_calibration": out}), flush=True)


def load_traffic(math):
    """Calibrated HBM bytes per Hessian launch of the given kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE measurement (None until measured)."""
    path = os.path.join(ROOT, "profiles", "hessian_traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            return (json.load(f).get(math) or {}).get("traffic_bytes_per_launch")
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-chunks", type=int, default=2)
    ap.add_argument("--config", choices=["cfg2", "cfg3", "cfg4", "cfg5"], default="cfg2",
                    help="cfg2: one q_proj linear (default); cfg3: a full Llama-3-8B layer; cfg4: the "
                         "layer rotated, w4 sym, dynamic 128-column groups, atomic; cfg5: the Llama-3-70B "
                         "down_proj 8192x28672")
    ap.add_argument("--cpu-baseline-layer", action="store_true",
                    help="with --config cfg3/cfg4: also time the CPU oracle on the layer (minutes)")
    ap.add_argument("--cpu-baseline-sample", action="store_true",
                    help="with --config cfg5: time the CPU oracle's Hessian accumulation on one sample")
    ap.add_argument("--hessian-math", choices=["split16", "fp32"], default="split16",
                    help="Hessian kernel for the fp16 inputs (split16: exact fp32 products from three "
                         "fp16 MFMA products; fp32: fp32 MFMA)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (counter calibration for the traffic figure)")
    ap.add_argument("--gemm-calibration", action="store_true",
                    help="only time torch.matmul (hipBLASLt / rocBLAS) in fp16 / fp32 / fp64: the "
                         "practical MFMA ceilings the kernels are compared with")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs the GPTQ+ hot path on one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding is a design note, not a launched path.", file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    from gptq_plus_mp_quant_amd import _native as nat
    nat.load().rq_hessian_math(nat.RQ_HMATH_SPLIT16 if args.hessian_math == "split16" else nat.RQ_HMATH_FP32)
    if args.copy_calibration:
        copy_calibration(dev)
        return
    if args.gemm_calibration:
        gemm_calibration(dev)
        return
    if args.config in ("cfg3", "cfg4"):
        run_layer(args, dev)
        return
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = dict(CFG5 if args.config == "cfg5" else CFG)
    X, W, s, grad = make_inputs(dev, cfg)
    layer = torch.nn.Linear(cfg["C"], cfg["R"], bias=False).to(dev, torch.float16)
    torch.cuda.synchronize()

    for _ in range(args.warmup):
        one_linear(X, W, s, grad, cfg, layer)
    torch.cuda.synchronize()

    timer = EventTimer()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_linear(X, W, s, grad, cfg, layer, timer)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps

    h_ms, n_launch = timer.mean_ms()
    ntok = cfg["bsz"] * cfg["T"]
    flops = cfg["G"] * ntok * cfg["C"] * (cfg["C"] + 1)       # upper triangle incl. diagonal

    line = {
        "metric": "ms per linear (H-accum + fasterquant) at Llama-8B shapes; % fp32-MFMA peak",
        "value": round(ms_per_step, 2),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (fp16 inputs; exact fp32 products)",
        "data": "synthetic (seeded, generated on the GPU)",
        "config": {"workload": ("configs[4]: Llama-3-70B down_proj 8192x28672, W ~ N(0, 0.015^2), "
                                "NUM_GROUPS=4 (4 Hessians of 28672^2 fp32), 128x2048 tokens, w4 asym "
                                "per-channel, act_order, B=128, GPTQ+ term on (alpha=0)")
                   if args.config == "cfg5" else
                   "configs[1]: q_proj 4096x4096, NUM_GROUPS=4, 128x2048 tokens, w4 asym "
                   "per-channel, act_order, B=128, GPTQ+ term on (alpha=0)",
                   "parallelism": "single GPU"},
        "roofline": hessian_roofline(flops, h_ms, args.hessian_math,
                                     {"traffic": load_traffic(args.hessian_math) if args.config == "cfg2" else None,
                                      "launch_ms": round(h_ms, 3), "launches": n_launch,
                                      "flops_per_launch": flops}),
    }
    if args.config == "cfg5":
        if args.cpu_baseline_sample:
            line["cpu_baseline"] = cpu_baseline_hessian_sample(X, s, cfg)
    elif not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(X, W, s, grad, cfg, args.cpu_chunks)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark: ms per linear (Hessian accumulation + GPTQ+ fasterquant) on one MI355X.

Default workload -- BASELINE.json configs[2], the configuration the metric and the target are
stated on: a full Llama-3-8B-shaped decoder layer, 7 linears (q/o 4096x4096, k/v 1024x4096,
gate/up 14336x4096, down 4096x14336), fp16 W ~ N(0, 0.02^2), calibration X = 128 samples x
2048 tokens per input width (N(0,1), 8 seeded outlier channels x20), NUM_GROUPS = 4 token
saliencies ~ LogNormal(0,1) clipped at their 0.99 quantile, GPTQ+ term on with
G ~ N(0, 1e-4^2) and alpha = 0, w4 asymmetric per-channel, act_order, BLOCKSIZE = 128,
percdamp = 0.01, 16-sample add_batch chunks; q/k/v and gate/up take their Hessians from one
launch over their shared input (add_batch_shared).  A step = one layer (Hessians of the 7
linears + finalize_hessian + fasterquant of each), inputs resident in HBM; value = layer / 7.
Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
  python bench.py --config cfg1|cfg2          # configs[0] / configs[1]: one 4096x4096 q_proj
  python bench.py --config cfg4               # configs[3]: the layer rotated, w4 sym, g128, atomic
  python bench.py --config cfg5 [--cpu-baseline-sample]   # configs[4]: Llama-3-70B down_proj
  python bench.py --alpha 0.05 --ref-loss 1e-3   # the GPTQ+ term with a non-zero beta

Report helpers that run no GPU work (their outputs are the summaries under profiles/):
  python bench.py --stats-table STATS_CSV --config cfgN --units U
  python bench.py --traffic FETCH_CSV WRITE_CSV CAL_FETCH_CSV CAL_WRITE_CSV --config cfgN
"""
from __future__ import annotations

import argparse
import csv
import hashlib
import json
import os
import platform
import re
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_MFMA_PEAK_TFLOPS = 157.3
FP16_MFMA_PEAK_TFLOPS = 2500.0      # dense fp16 / bf16 MFMA
FP64_MFMA_PEAK_TFLOPS = 78.6
HBM_PEAK_GBS = 8000.0
METRIC = "ms per linear (H-accum + fasterquant) at Llama-8B shapes; % fp32-MFMA peak"
PIECES = {"split16": 2, "split16x3": 3, "fp32": 1}     # 16-bit MFMA products per fp32 product (fp16 X)
# the arithmetic the Hessian (the dominant kernel) computes in, by --hessian-math and fp32 X;
# the Cholesky chain runs in fp64, every other kernel in fp32
DTYPE_TEXT = {
    ("split16x3", False): "f32 (fp16 inputs; Hessian: exact fp32 products, 3 fp16 MFMA products each, fp32 sums)",
    ("split16", False): "f32 (fp16 inputs; Hessian: fp32 products within 2^-23 relative, 2 fp16 MFMA products "
                        "each, fp32 sums)",
    ("fp32", False): "f32 (fp16 inputs; Hessian: fp32 MFMA)",
    ("split16x3", True): "f32 (fp32 inputs; Hessian: fp32 MFMA)",
    ("split16", True): "f32 (fp32 inputs; Hessian: fp32 products within 2^-20.5 relative, 3 fp16 MFMA "
                       "products each, fp32 sums)",
    ("fp32", True): "f32 (fp32 inputs; Hessian: fp32 MFMA)",
}
KERNEL = {"split16": "k_hessian_split<__half, 2>", "split16x3": "k_hessian_split<__half, 3>",
          "fp32": "k_hessian_accum<__half>"}
HESSIAN_SRC = os.path.join(ROOT, "gptq_plus_mp_quant_amd", "csrc", "hessian.hip")
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "hessian_traffic.json")

BASE = dict(R=4096, C=4096, G=4, N=128, T=2048, bsz=16, bits=4, sym=False, blocksize=128,
            percdamp=0.01, alpha=0.0, ref_loss=0.0, outliers=8, seed=20251201, wscale=0.02)
# cfgK = BASELINE.json configs[K-1] (numbered from 1)
CONFIGS = {
    "cfg1": dict(BASE, G=1, gptq_plus=False, kind="linear"),
    "cfg2": dict(BASE, kind="linear"),
    "cfg3": dict(BASE, kind="layer"),
    "cfg4": dict(BASE, sym=True, groupsize=128, actorder=False, atomic=True, rotate=True, kind="layer"),
    "cfg5": dict(BASE, R=8192, C=28672, wscale=0.015, kind="linear"),
}
WORKLOAD = {
    "cfg1": "configs[0]: q_proj 4096x4096, NUM_GROUPS=1, 128x2048 tokens, w4 asym per-channel, act_order, "
            "B=128, GPTQ+ term off",
    "cfg2": "configs[1]: q_proj 4096x4096, NUM_GROUPS=4, 128x2048 tokens, w4 asym per-channel, act_order, "
            "B=128, GPTQ+ term on (alpha={alpha})",
    "cfg3": "configs[2]: Llama-3-8B decoder layer, 7 linears (q/k/v and gate/up Hessians fused over their "
            "shared input), NUM_GROUPS=4, 128x2048 tokens, w4 asym per-channel, act_order, B=128, GPTQ+ term on "
            "(alpha={alpha}); value = layer time / 7, ms_per_step = layer",
    "cfg4": "configs[3]: Llama-3-8B decoder layer, seeded orthogonal (Hadamard-based) rotation of W and X, w4 "
            "sym, 128-column dynamic groups, BLOCK_ATOMIC_QUANT, NUM_GROUPS=4, 128x2048 tokens; value = layer "
            "time / 7, ms_per_step = layer",
    "cfg5": "configs[4]: Llama-3-70B down_proj 8192x28672, W ~ N(0, 0.015^2), NUM_GROUPS=4 (4 Hessians of "
            "28672^2 fp32), 128x2048 tokens, w4 asym per-channel, act_order, B=128, GPTQ+ term on (alpha={alpha})",
}
# the modules of a Llama-3-8B decoder layer; modules that read the same input share one X
LAYER8B = [("q_proj", 4096, 4096, "attn"), ("k_proj", 1024, 4096, "attn"), ("v_proj", 1024, 4096, "attn"),
           ("o_proj", 4096, 4096, "o"), ("gate_proj", 14336, 4096, "mlp"), ("up_proj", 14336, 4096, "mlp"),
           ("down_proj", 4096, 14336, "down")]
INPUT_WIDTH = {"attn": 4096, "o": 4096, "mlp": 4096, "down": 14336}


# ---------------------------------------------------------------------------------------------
# synthetic inputs (seeded, generated on the GPU)

def _saliency(gen, dev, N, T, G):
    import torch
    s = torch.exp(torch.randn((N, T, G), generator=gen, device=dev))
    for g in range(G):
        s[..., g].clamp_(max=float(torch.quantile(s[..., g].flatten(), 0.99)))   # linear interpolation
    return s


def make_inputs(dev, cfg):
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(cfg["seed"])
    N, T, C, R, G = cfg["N"], cfg["T"], cfg["C"], cfg["R"], cfg["G"]
    X = torch.empty((N, T, C), dtype=torch.float16, device=dev)
    for i in range(N):
        X[i] = torch.randn((T, C), generator=gen, device=dev, dtype=torch.float32).half()
    X[:, :, torch.randperm(C, generator=gen, device=dev)[: cfg["outliers"]]] *= 20
    W = (torch.randn((R, C), generator=gen, device=dev) * cfg["wscale"]).half()
    s = _saliency(gen, dev, N, T, G)
    grad = torch.randn((R, C), generator=gen, device=dev) * 1e-4
    return X, W, s, grad


def hadamard(n, dev):
    import torch
    H = torch.ones((1, 1), device=dev)
    while H.shape[0] < n:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return H


def rotation(C, gen, dev):
    """configs[3]'s seeded orthogonal rotation: diag(+-1) H_C / sqrt(C) for a power of two,
    Q_k (x) (diag(+-1) H_m / sqrt(m)) for C = k * m (QuaRot-style; C = 14336 = 7 * 2048)."""
    import torch
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


def make_layer_inputs(dev, cfg):
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(cfg["seed"] + 1)
    N, T, G = cfg["N"], cfg["T"], cfg["G"]
    xs, rots = {}, {}
    for key, C in INPUT_WIDTH.items():
        X = torch.empty((N, T, C), dtype=torch.float16, device=dev)
        for i in range(N):
            X[i] = torch.randn((T, C), generator=gen, device=dev, dtype=torch.float32).half()
        X[:, :, torch.randperm(C, generator=gen, device=dev)[: cfg["outliers"]]] *= 20
        if cfg.get("rotate"):
            rots[key] = rotation(C, gen, dev)
            for i in range(N):                                  # X <- X R, one sample at a time
                X[i] = (X[i].float() @ rots[key]).half()
        xs[key] = X
    mods = {}
    for name, R, C, key in LAYER8B:
        W = (torch.randn((R, C), generator=gen, device=dev) * cfg["wscale"]).half()
        if cfg.get("rotate"):
            W = (W.float() @ rots[key]).half()                 # W' = W R keeps X' W'^T = X W^T
        mods[name] = (W, _saliency(gen, dev, N, T, G), torch.randn((R, C), generator=gen, device=dev) * 1e-4, key)
    return xs, mods


# ---------------------------------------------------------------------------------------------
# the timed work

class KernelTimer:
    """HIP events recorded by the library around each Hessian product kernel
    (rq_hessian_timing_events), on the stream that kernel runs on."""

    def __init__(self):
        self.pairs = []

    def arm(self):
        import torch
        from gptq_plus_mp_quant_amd import _native as nat
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()          # creates the events; the library records them again around the kernel
        b.record()
        nat.call("rq_hessian_timing_events", a.cuda_event, b.cuda_event)
        self.pairs.append((a, b))

    def total_ms(self):
        import torch
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in self.pairs), len(self.pairs)


def fq_kwargs(cfg):
    """fasterquant arguments: act_order with static_groups = act_order like the driver (:7472);
    configs[3] dynamic 128-column groups + atomic; configs[0] without the GPTQ+ term."""
    act = cfg.get("actorder", True)
    return dict(blocksize=cfg["blocksize"], percdamp=cfg["percdamp"], groupsize=cfg.get("groupsize", -1),
                actorder=act, static_groups=act, block_atomic_quant=cfg.get("atomic", False),
                enable_gradient_update=cfg.get("gptq_plus", True))


def new_gptq(layer, W, s, grad, cfg):
    from gptq_plus_mp_quant_amd import GPTQPlus, WeightQuantizer
    layer.weight.data.copy_(W)
    g = GPTQPlus(layer, saliency=s, gradient=grad, num_groups=cfg["G"], alpha=cfg["alpha"],
                 reference_loss=cfg["ref_loss"])
    g.quantizer = WeightQuantizer()
    g.quantizer.configure(cfg["bits"], perchannel=True, sym=cfg["sym"], mse=False)
    return g


class PhaseMarks:
    """Events recorded on the current stream at the boundaries of a step's phases (no host
    synchronisation), read after the timed region: per-step times and per-phase means."""

    def __init__(self):
        self.steps = []

    def begin(self):
        import torch
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.steps.append([("begin", e)])

    def mark(self, name):
        import torch
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.steps[-1].append((name, e))

    def report(self):
        import torch
        torch.cuda.synchronize()
        per_step, phases = [], {}
        for marks in self.steps:
            per_step.append(marks[0][1].elapsed_time(marks[-1][1]))
            for (_, a), (name, b) in zip(marks, marks[1:]):
                phases[name] = phases.get(name, 0.0) + a.elapsed_time(b)
        n = max(len(self.steps), 1)
        return per_step, {k: v / n for k, v in phases.items()}


def one_linear(X, W, s, grad, cfg, layer, timer=None, keep=False, marks=None):
    if marks is not None:
        marks.begin()
    g = new_gptq(layer, W, s, grad, cfg)
    for j in range(0, cfg["N"], cfg["bsz"]):
        if timer is not None:
            timer.arm()
        g.add_batch(X[j:j + cfg["bsz"]], None)
    if marks is not None:
        marks.mark("hessian")
    g.finalize_hessian()
    if marks is not None:
        marks.mark("finalize")
    g.fasterquant(**fq_kwargs(cfg))
    if marks is not None:
        marks.mark("fasterquant")
    g.free()
    if marks is not None:
        marks.mark("free")
    return g


def one_layer(xs, mods, cfg, layers, timer=None, keep=False, marks=None):
    from gptq_plus_mp_quant_amd import add_batch_shared, fasterquant_shared
    if marks is not None:
        marks.begin()
    objs = {name: new_gptq(layers[name], W, s, grad, cfg) for name, (W, s, grad, _) in mods.items()}
    for key in INPUT_WIDTH:
        group = [objs[n] for n, _, _, k in LAYER8B if k == key]
        for j in range(0, cfg["N"], cfg["bsz"]):
            if timer is not None:
                timer.arm()
            add_batch_shared(group, xs[key][j:j + cfg["bsz"]])
    if marks is not None:
        marks.mark("hessian")
    for g in objs.values():
        g.finalize_hessian()
    if marks is not None:
        marks.mark("finalize")
    kept = {}
    if keep:
        kept = {name: (g.H.clone(), g.act_square.clone()) for name, g in objs.items()}
    # one fasterquant per linear, free() after each group (the reference's loop, free() emptying
    # the allocator cache like gptq_plus_utils.py:2357-2361); --shared-fasterquant runs the chains
    # of the linears that share an input as one batch (fasterquant_shared, bit-identical results)
    for key in INPUT_WIDTH:
        names = [n for n, _, _, k in LAYER8B if k == key]
        group = [objs[n] for n in names]
        if len(group) > 1 and cfg.get("shared_fq"):
            fasterquant_shared(group, **fq_kwargs(cfg))
        else:
            for g in group:
                g.fasterquant(**fq_kwargs(cfg))
        if marks is not None:
            marks.mark(f"fasterquant {'/'.join(names)}")
        for g in group:
            g.free()
        if marks is not None:
            marks.mark(f"free {'/'.join(names)}")
    return kept


def hessian_flops(cfg):
    """Algorithmic fp32 flops of one unit's Hessians: the upper triangle incl. the diagonal,
    2 per (token, i <= j) element of every Hessian (G * N * T * C * (C + 1) per linear)."""
    ntok = cfg["N"] * cfg["T"]
    if cfg["kind"] == "layer":
        return sum(cfg["G"] * ntok * C * (C + 1) for _, _, C, _ in LAYER8B)
    return cfg["G"] * ntok * cfg["C"] * (cfg["C"] + 1)


def hessian_calls(cfg):
    """add_batch product launches per unit (layer or linear): one per HESSIAN_ACCUM_BSZ-sample chunk
    and distinct input (the layer's q/k/v and gate/up read one X each).  The split kernel issues
    each call as several dispatches (one per round of whole items), so per-call figures are
    totals over the call's dispatches."""
    chunks = cfg["N"] // cfg["bsz"]
    return chunks * (len(INPUT_WIDTH) if cfg["kind"] == "layer" else 1)


def load_traffic(math, config):
    """Calibrated HBM bytes per product-kernel launch from the committed rocprofv3 measurement,
    used only when it was taken on this configuration with the current hessian.hip."""
    if not os.path.exists(TRAFFIC_JSON):
        return None, "no measurement"
    with open(TRAFFIC_JSON) as f:
        rec = (json.load(f).get(math) or {})
    if rec.get("config") != config:
        return None, f"measured on {rec.get('config')}"
    if rec.get("hessian_src_sha256") != source_sha():
        return None, "hessian.hip changed since the measurement"
    return rec.get("traffic_bytes_per_launch"), "profiles/hessian_traffic.json"


def source_sha():
    with open(HESSIAN_SRC, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def roofline(cfg, args, kernel_ms, launches, steps):
    """The dominant kernel (the Hessian product kernel) against the peak of the MFMA pipe it
    runs on: algorithmic fp32 flops per launch (the upper triangle of the reference's fp32
    products, each counted once) / measured launch time.  The split kernels form each fp32
    product from PIECES 16-bit MFMA products, so they are held to the fp16 / bf16 peak (2.5
    PF/s) and `executed` gives the pipe's use counting every product issued; the fp32 MFMA kernel
    is held to the fp32 peak.  `fp32_equivalent` states the same rate against the fp32 MFMA
    peak the metric names (a ratio, not a fraction of a pipe)."""
    flops_unit = hessian_flops(cfg)
    per_launch_flops = flops_unit * steps / launches
    ms = kernel_ms / launches
    ach = per_launch_flops / (ms * 1e-3) / 1e12
    traffic, tsrc = load_traffic(args.hessian_math, args.config)
    pieces = PIECES[args.hessian_math]
    kernel = KERNEL[args.hessian_math]
    if args.x_fp32:   # fp32 activations: exact on the fp32 kernel, or hi w0 + hi w1 + lo w0 (split16)
        traffic, tsrc = None, "fp32 activations: not measured"
        pieces = 3 if args.hessian_math == "split16" else 1
        kernel = "k_hessian_split32" if args.hessian_math == "split16" else "k_hessian_accum<float>"
    peak = FP16_MFMA_PEAK_TFLOPS if pieces > 1 else FP32_MFMA_PEAK_TFLOPS
    return {"bound": "mfma", "achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s",
            "frac": round(ach / peak, 4), "traffic": traffic,
            "pipe": "fp16 MFMA (v_mfma_f32_32x32x16_f16)" if pieces > 1 else "fp32 MFMA (v_mfma_f32_32x32x2_f32)",
            "kernel": kernel, "launch_ms": round(ms, 4), "launches": launches // steps,
            "flops_per_launch": int(per_launch_flops),
            "algorithmic": "fp32 flops of H_g += X^T diag(s_g) X, upper triangle incl. diagonal "
                           "(G*n*C*(C+1) per launch of n tokens)",
            "executed": {"products_per_fp32_product": pieces, "tflops": round(ach * pieces, 2),
                         "frac": round(ach * pieces / peak, 4)},
            "fp32_equivalent": {"peak": FP32_MFMA_PEAK_TFLOPS, "ratio": round(ach / FP32_MFMA_PEAK_TFLOPS, 4)},
            "traffic_source": tsrc}


# ---------------------------------------------------------------------------------------------
# the CPU baseline: the reference's op sequence (oracle/) on the host cores

def host_cpu():
    """Use every physical core this process may run on; describe the host."""
    import torch
    out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout if shutil_which("lscpu") else ""
    field = lambda k: (re.search(rf"^{k}:\s*(.+)$", out, re.M) or [None, "?"])[1].strip()
    model = field("Model name")
    try:
        sockets, cps, tpc = int(field(r"Socket\(s\)")), int(field(r"Core\(s\) per socket")), int(field(r"Thread\(s\) per core"))
    except ValueError:
        sockets, cps, tpc = 1, os.cpu_count() or 1, 1
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = max(1, min(sockets * cps, affinity // max(tpc, 1) if tpc > 1 else affinity))
    torch.set_num_threads(threads)
    cfg_txt = torch.__config__.show()
    blas = (re.search(r"BLAS_INFO=(\w+)", cfg_txt) or [None, "?"])[1]
    par = torch.__config__.parallel_info()
    backend = (re.search(r"ATen parallel backend: (.+)", par) or [None, "?"])[1].strip()
    return threads, {"model": model, "sockets": sockets, "cores_per_socket": cps, "threads_per_core": tpc,
                     "cpus_available": affinity, "threads_used": threads, "blas": blas,
                     "aten_parallel": backend, "isa": torch.backends.cpu.get_cpu_capability(),
                     "torch": torch.__version__}


def shutil_which(name):
    from shutil import which
    return which(name) is not None


def cpu_baseline_linear(X, W, s, grad, cfg, chunks=2):
    """`chunks` of the 8 add_batch calls timed (extrapolated by tokens)
    plus the full finalize_hessian + fasterquant of the same linear."""
    import torch
    from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
    threads, host = host_cpu()
    o = GPTQPlusOracle(W.cpu(), s.cpu(), grad.cpu(), cfg["G"], cfg["alpha"], cfg["ref_loss"])
    o.quantizer = make_quantizer(cfg["bits"], cfg["sym"])
    Xc = X[: chunks * cfg["bsz"]].cpu()
    t0 = time.perf_counter()
    for j in range(0, Xc.shape[0], cfg["bsz"]):
        o.add_batch(Xc[j:j + cfg["bsz"]])
    t_acc = time.perf_counter() - t0
    o.index, o.token_count = cfg["N"], cfg["N"] * cfg["T"]
    t1 = time.perf_counter()
    o.finalize_hessian()
    o.fasterquant(**{k: v for k, v in fq_kwargs(cfg).items()})
    t_fq = time.perf_counter() - t1
    nchunks = cfg["N"] // cfg["bsz"]
    total = t_acc * nchunks / chunks + t_fq
    return dict(value=round(total * 1e3, 1), unit="ms per linear (extrapolated)", cores=threads, kind="port",
                sample=(f"oracle (the reference's torch op sequence) on the host CPU: {chunks}/{nchunks} add_batch "
                        f"chunks timed ({t_acc:.1f} s, x{nchunks // chunks} by tokens) + full finalize_hessian + "
                        f"fasterquant ({t_fq:.1f} s)"), host=host)


def cpu_baseline_layer(xs, mods, kept, cfg):
    """configs[2] / configs[3] on a bounded sample.  add_batch: one full 16-sample chunk
    (32768 tokens, the reference's HESSIAN_ACCUM_BSZ call with its (G, 32768, C) fp32 `weighted`)
    per input width, through the reference's per-module call (x 8 chunks by tokens, per module
    of that width).  finalize_hessian + fasterquant: all 4 row subgroups of q_proj (4096 x 4096)
    and one of the 4 of each other distinct (rows, columns) shape (x 4: the subgroups are
    independent in the reference's loop, :1027-1162), on the GPU run's finalized Hessians.  The
    two parts make the layer."""
    import torch
    from oracle.gptqplus_cpu import GPTQPlusOracle, make_quantizer
    threads, host = host_cpu()
    N, G, bsz = cfg["N"], cfg["G"], cfg["bsz"]
    t_ab, parts = {}, []
    for key, C in (("attn", 4096), ("down", 14336)):
        name = next(n for n, _, c, k in LAYER8B if c == C)
        W, s, grad, _ = mods[name]
        o = GPTQPlusOracle(W.cpu(), s[:bsz].cpu(), grad.cpu(), G, cfg["alpha"], cfg["ref_loss"])
        x = xs[key][:bsz].cpu()
        t0 = time.perf_counter()
        o.add_batch(x)
        t_ab[C] = (time.perf_counter() - t0) * (N // bsz)
        parts.append(f"add_batch C={C}: 1 of {N // bsz} {bsz}-sample chunks {t_ab[C] / (N // bsz):.2f} s")
        print(f"cpu baseline add_batch C={C}: {t_ab[C] / (N // bsz):.2f} s per {bsz}-sample chunk", flush=True)
        del o, x
    t_fq = {}
    for name, R, C, key in LAYER8B:
        if (R, C) in t_fq:
            continue
        W, s, grad, _ = mods[name]
        nsub = G if (R, C) == (4096, 4096) else 1
        Rs = R // G
        H, act = kept[name]
        o = GPTQPlusOracle(W[:nsub * Rs].cpu(), s[:, :, :nsub].cpu(), grad[:nsub * Rs].cpu(), nsub,
                           cfg["alpha"], cfg["ref_loss"])
        o.quantizer = make_quantizer(cfg["bits"], cfg["sym"])
        o.H = H[:nsub].cpu()
        o.act_square = act.cpu()
        o.index, o.token_count, o._finalized = N, N * cfg["T"], True
        t0 = time.perf_counter()
        o.fasterquant(**fq_kwargs(cfg))
        t_fq[(R, C)] = (time.perf_counter() - t0) * G / nsub
        parts.append(f"fasterquant {R}x{C}: {nsub}/{G} subgroups {t_fq[(R, C)] * nsub / G:.2f} s")
        print(f"cpu baseline fasterquant {R}x{C}: {t_fq[(R, C)] / G:.2f} s per subgroup ({nsub} timed)",
              flush=True)
        del o
    total = sum(t_ab[C] + t_fq[(R, C)] for _, R, C, _ in LAYER8B)
    return dict(value=round(total * 1e3 / len(LAYER8B), 1), unit="ms per linear (layer / 7, extrapolated)",
                cores=threads, kind="port",
                sample=("oracle (the reference's torch op sequence) on the host CPU, extrapolated from a "
                        "bounded sample: " + "; ".join(parts) + f"; layer {total:.1f} s"), host=host)


def cpu_baseline_hessian_sample(X, s, cfg, samples=1):
    """configs[4] on the host is hours of work: the oracle's add_batch on `samples` of the 128
    calibration samples, extrapolated by tokens; a lower bound (finalize + fasterquant left out)."""
    import torch
    from oracle.gptqplus_cpu import GPTQPlusOracle
    threads, host = host_cpu()
    C, G = cfg["C"], cfg["G"]
    o = GPTQPlusOracle(torch.zeros(G, C), s[:samples].cpu(), torch.zeros(G, C), G, 0.0, 0.0)
    t0 = time.perf_counter()
    o.add_batch(X[:samples].cpu())
    t = time.perf_counter() - t0
    scale = cfg["N"] // samples
    return dict(value=round(t * scale * 1e3, 1), unit="ms per linear (Hessian accumulation only, extrapolated)",
                cores=threads, kind="port",
                sample=(f"oracle add_batch on {samples}/{cfg['N']} samples ({t:.1f} s, x{scale} by tokens); "
                        "finalize_hessian + fasterquant not timed, so this is a lower bound"), host=host)


# ---------------------------------------------------------------------------------------------
# report helpers (no GPU work)

def copy_calibration(dev, nbytes=1 << 30, reps=3):
    """A plain device-to-device copy of known size, profiled with the same FETCH_SIZE /
    WRITE_SIZE counters to calibrate them (bytes moved = nbytes read + nbytes written)."""
    import torch
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "reps": reps}), flush=True)


def gemm_calibration(dev):
    """Practical GEMM ceilings: torch.matmul (hipBLASLt / rocBLAS) on large square operands in
    fp16, fp32 (TF32 off) and fp64, as TFLOP/s."""
    import torch
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
    # fp64 rank-K updates C -= A B of the Cholesky chain's panel shapes (trailing rows x rows,
    # K = panel width): the practical ceiling the panel-update kernel is measured against
    out["fp64_rank_k"] = []
    for m, k in ((4096, 256), (13824, 512), (13824, 256), (27648, 512)):
        a = torch.randn(m, k, device=dev, dtype=torch.float64)
        b = torch.randn(k, m, device=dev, dtype=torch.float64)
        c = torch.randn(m, m, device=dev, dtype=torch.float64)
        for _ in range(2):
            c.addmm_(a, b, alpha=-1.0)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            c.addmm_(a, b, alpha=-1.0)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 5
        out["fp64_rank_k"].append({"m": m, "k": k, "ms": round(ms, 3), "tflops": round(2 * m * m * k / ms / 1e9, 1)})
        del a, b, c
    print(json.dumps({"gemm_calibration": out}), flush=True)


def _kernel_name(full):
    n = re.sub(r"\(anonymous namespace\)::", "", full)
    n = re.sub(r"\((?:[^()]|\([^()]*\))*\)\s*$", "", n).strip()
    return n[:60]


def algorithmic_work(cfg, lookahead=False):
    """Algorithmic work per unit (one linear, or one layer) of the kernels the table reports:
    (bytes, flops) by kernel-name prefix.  Bytes are those the operation must move at least once
    (inputs read, outputs written); flops count the reference's arithmetic (fp32 unless noted).
    With `lookahead` (the run used k_block_lookahead), k_quant_block quantises only each linear's
    first block, and k_block_lookahead does every other block's column loop plus the whole
    trailing update."""
    B = cfg["blocksize"]
    linears = [(R, C) for _, R, C, _ in LAYER8B] if cfg["kind"] == "layer" else [(cfg["R"], cfg["C"])]
    G, ntok = cfg["G"], cfg["N"] * cfg["T"]
    w = {}

    def add(k, b=0.0, f=0.0):
        ob, of = w.get(k, (0.0, 0.0))
        w[k] = (ob + b, of + f)
    for R, C in linears:
        nb = (C + B - 1) // B
        trail = sum(2.0 * R * B * (C - min(C, (k + 1) * B)) for k in range(nb))
        add("k_find_params", 2.0 * R * C + 8 * R)
        # row-staged gathers (params.hip): 1024 threads per workgroup for rows above 32 KB
        nt = lambda esize: 1024 if C * esize > 32 * 1024 else 256
        add(f"k_gather_rows<{nt(2)}, __half>", (2.0 + 4.0) * R * C)   # fp16 W read, permuted fp32 written
        add(f"k_gather_rows<{nt(4)}, float>", 8.0 * R * C)            # G read, permuted copy written
        # one H row per workgroup: 512 threads x 8 rows in flight from C = 8192 on (params.hip)
        add("k_gather_h_rows<512, 8>" if C >= 8192 else "k_gather_h_rows<256, 1>", 8.0 * G * C * C)
        f0 = min(B, C) / C if lookahead else 1.0             # share of the columns k_quant_block runs
        add("k_quant_block", 9.0 * R * C * f0, 2.0 * R * C * B * f0)   # W read, fp32 Q + int8 code written
        if lookahead:
            add("k_block_lookahead", 9.0 * R * C * (1.0 - f0) + 8.0 * R * C, trail + 2.0 * R * C * B * (1.0 - f0))
        else:
            add("k_trailing_w", 8.0 * R * C, trail)
        add("k_trailing_z", 20.0 * R * C, 3.0 * trail)         # GPTQ+ terms: three chains; W, GH, Z
        add("k_hessian_finalize64", 6.0 * G * C * C)           # upper triangle read, both halves written
        add(f"k_writeback_rows<{nt(2)}, __half>", 2.0 * R * C + 2.0 * R * C)   # int16 codes read, fp16 out
        add("k_panel_update", 0.0, G * (2.0 / 3.0) * C ** 3)   # fp64: trailing factor + L^-1 rows
    inputs = {4096: 0, 14336: 0}
    if cfg["kind"] == "layer":
        for key, C in INPUT_WIDTH.items():
            inputs[C] = inputs.get(C, 0) + 1
    else:
        inputs = {cfg["C"]: 1}
    for C, n in inputs.items():
        add("k_xprep", n * 4.0 * ntok * C)                      # X read, the blocked copy written
    add("k_hessian_split", 0.0, float(hessian_flops(cfg)))
    add("k_hessian_accum", 0.0, float(hessian_flops(cfg)))
    return w


def stats_table(path, cfg, units, config):
    """Markdown table of a rocprofv3 --stats kernel CSV (the 24 longest kernels and every kernel
    whose algorithmic work per unit is known), with achieved rates where that work is known."""
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            rows.append((_kernel_name(r["Name"]), int(r["Calls"]), float(r["TotalDurationNs"]) / 1e6,
                         float(r["AverageNs"]) / 1e3, float(r["Percentage"])))
    work = algorithmic_work(cfg, lookahead=any("k_block_lookahead" in r[0] for r in rows))
    rows.sort(key=lambda x: -x[2])
    print(f"| kernel | calls | total (ms) | per unit (ms) | average (us) | % | algorithmic work per unit | achieved |")
    print("|---|---:|---:|---:|---:|---:|---|---|")
    for rank, (name, calls, tot, avg, pct) in enumerate(rows):
        per = tot / units
        bare = name[5:] if name.startswith("void ") else name
        key = bare if bare in work else next((k for k in work if bare.split("<")[0] == k), None)
        if rank >= 24 and not key:     # the 24 longest kernels, then those with a known rate
            continue
        wtxt = ach = ""
        if key:
            b, fl = work[key]
            if fl:
                # the split Hessian kernels run on the fp16 pipe (algorithmic fp32 flops against
                # its peak), the fp32 one on the fp32 pipe, the Cholesky update on the fp64 pipe
                peak = FP64_MFMA_PEAK_TFLOPS if key == "k_panel_update" else (
                    FP16_MFMA_PEAK_TFLOPS if key == "k_hessian_split" else (
                        FP32_MFMA_PEAK_TFLOPS if key != "k_quant_block" else None))
                tf = fl / (per * 1e-3) / 1e12
                wtxt = f"{fl / 1e9:.1f} GFLOP" + (f", {b / 1e6:.0f} MB" if b else "")
                ach = f"{tf:.1f} TF/s" + (f" ({100 * tf / peak:.1f} % of {peak})" if peak else "")
                if key in ("k_hessian_split", "k_hessian_accum"):
                    # the live launch time covers one add_batch call, which may span dispatches
                    ach += f"; {per / hessian_calls(cfg):.3f} ms per add_batch call"
                if b and key in ("k_quant_block", "k_block_lookahead"):
                    ach += f"; {b / (per * 1e-3) / 1e9:.0f} GB/s"
            else:
                gbs = b / (per * 1e-3) / 1e9
                wtxt = f"{b / 1e6:.0f} MB"
                ach = f"{gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f} % of HBM)"
        print(f"| `{name}` | {calls} | {tot:.2f} | {per:.3f} | {avg:.1f} | {pct:.2f} | {wtxt} | {ach} |")


def counters_table(path, top=16):
    """Markdown table of a rocprofv3 --pmc CSV (one row per dispatch and counter), per kernel:
    MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE * 128) (the SQ counter sums the
    1024 SIMDs, GRBM_GUI_ACTIVE the 8 XCDs' busy cycles: busy SIMD-cycles over SIMD-cycles),
    VALU and LDS instructions per MFMA, LDS bank-conflict cycles per LDS instruction, and the
    sustained clock: GRBM_GUI_ACTIVE / 8 XCDs over the dispatches' summed durations (for kernels
    averaging 1 ms or more per dispatch)."""
    agg, disp, dur = {}, {}, {}
    with open(path) as f:
        for r in csv.DictReader(f):
            k = _kernel_name(r["Kernel_Name"])
            agg.setdefault(k, {}).setdefault(r["Counter_Name"], 0.0)
            agg[k][r["Counter_Name"]] += float(r["Counter_Value"])
            if (k, r["Dispatch_Id"]) not in disp:
                disp[(k, r["Dispatch_Id"])] = 1
                dur[k] = dur.get(k, 0.0) + (float(r["End_Timestamp"]) - float(r["Start_Timestamp"])) / 1e3
    rows = sorted(agg.items(), key=lambda kv: -dur.get(kv[0], 0.0))
    print("| kernel | dispatches | time (ms) | MFMA busy | clock (GHz) | VALU / MFMA | LDS / MFMA | LDS conflict cycles / LDS |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|")
    for k, c in rows[:top]:
        n = sum(1 for (kk, _d) in disp if kk == k)
        busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / max(c.get("GRBM_GUI_ACTIVE", 0.0) * 128, 1.0)
        mf = c.get("SQ_INSTS_MFMA", 0.0)
        per_mfma = lambda key: f"{c.get(key, 0.0) / mf:.2f}" if mf else "-"
        lds = c.get("SQ_INSTS_LDS", 0.0)
        conf = f"{c.get('SQ_LDS_BANK_CONFLICT', 0.0) / lds:.2f}" if lds else "-"
        # cycles per ns; the counter window exceeds a short dispatch, so only from 1 ms on average
        clk = c.get("GRBM_GUI_ACTIVE", 0.0) / 8 / max(dur.get(k, 0.0) * 1e3, 1.0)
        clk = f"{clk:.3f}" if dur.get(k, 0.0) >= 1e3 * n else "-"
        print(f"| `{k}` | {n} | {dur.get(k, 0.0) / 1e3:.2f} | {100 * busy:.1f} % | {clk} | {per_mfma('SQ_INSTS_VALU')} | "
              f"{per_mfma('SQ_INSTS_LDS')} | {conf} |")


def traffic_report(fetch_csv, write_csv, cal_fetch_csv, cal_write_csv, kernel_prefix, config, cfg, math):
    """HBM bytes per product-kernel launch from FETCH_SIZE / WRITE_SIZE passes (KiB per dispatch),
    each scaled by what the counter reads for a 1 GiB device copy; written to TRAFFIC_JSON with
    the source hash of hessian.hip so bench.py only reports it while the kernel is unchanged."""
    def per_dispatch(path, counter, pred, calls=None):
        vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(path))
                if r["Counter_Name"] == counter and pred(r["Kernel_Name"])]
        return sum(vals) / max(calls or len(vals), 1), len(vals)
    is_k = lambda n: kernel_prefix in n
    is_copy = lambda n: "copyBuffer" in n
    # per add_batch call (one profiled step: hessian_calls(cfg) calls, each one or more dispatches)
    ncalls = hessian_calls(cfg)
    fetch, nf = per_dispatch(fetch_csv, "FETCH_SIZE", is_k, ncalls)
    write, nw = per_dispatch(write_csv, "WRITE_SIZE", is_k, ncalls)
    cfetch, _ = per_dispatch(cal_fetch_csv, "FETCH_SIZE", is_copy)
    cwrite, _ = per_dispatch(cal_write_csv, "WRITE_SIZE", is_copy)
    gib = float(1 << 30)
    rf, wf = cfetch * 1024 / gib, cwrite * 1024 / gib          # counter bytes per real byte
    traffic = fetch * 1024 / rf + write * 1024 / wf
    flops = hessian_flops(cfg)
    rec = {"kernel": kernel_prefix, "config": config, "dispatches": [nf, nw], "calls": ncalls,
           "fetch_size_kib_per_call": round(fetch, 1), "write_size_kib_per_call": round(write, 1),
           "copy_calibration": {"fetch_kib": round(cfetch, 1), "write_kib": round(cwrite, 1),
                                "read_factor": round(rf, 3), "write_factor": round(wf, 3)},
           "traffic_bytes_per_launch": int(traffic), "hessian_src_sha256": source_sha(),
           "flops_per_unit": flops}
    data = json.load(open(TRAFFIC_JSON)) if os.path.exists(TRAFFIC_JSON) else {}
    data[math] = rec
    with open(TRAFFIC_JSON, "w") as f:
        json.dump(data, f, indent=1)
    print(json.dumps(rec))


# ---------------------------------------------------------------------------------------------

def run(args):
    import torch
    from gptq_plus_mp_quant_amd import _native as nat
    dev = torch.device("cuda:0")
    nat.load().rq_hessian_math({"split16": nat.RQ_HMATH_SPLIT16, "split16x3": nat.RQ_HMATH_SPLIT16X3,
                                "fp32": nat.RQ_HMATH_FP32}[args.hessian_math])
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.copy_calibration:
        copy_calibration(dev)
        return
    if args.gemm_calibration:
        gemm_calibration(dev)
        return
    cfg = dict(CONFIGS[args.config], alpha=args.alpha, ref_loss=args.ref_loss, shared_fq=args.shared_fasterquant)
    layer_mode = cfg["kind"] == "layer"
    if layer_mode:
        xs, mods = make_layer_inputs(dev, cfg)
        if args.x_fp32:
            xs = {k: v.float() for k, v in xs.items()}
        layers = {n: torch.nn.Linear(C, R, bias=False).to(dev, torch.float16) for n, R, C, _ in LAYER8B}
        step = lambda timer=None, keep=False, marks=None: one_layer(xs, mods, cfg, layers, timer, keep, marks)
    else:
        X, W, s, grad = make_inputs(dev, cfg)
        if args.x_fp32:
            X = X.float()
        layer = torch.nn.Linear(cfg["C"], cfg["R"], bias=False).to(dev, torch.float16)
        step = lambda timer=None, keep=False, marks=None: one_linear(X, W, s, grad, cfg, layer, timer, keep, marks)
    torch.cuda.synchronize()
    kept = None
    for i in range(args.warmup):
        out = step(keep=(layer_mode and i == args.warmup - 1))
        kept = out if layer_mode and i == args.warmup - 1 else kept
    timer = KernelTimer()
    marks = PhaseMarks()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(timer, marks=marks)
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    kernel_ms, launches = timer.total_ms()
    step_ms, phase_ms = marks.report()
    per = len(LAYER8B) if layer_mode else 1
    print("per-step ms: " + " ".join(f"{t:.1f}" for t in step_ms), file=sys.stderr, flush=True)
    print("per-phase ms (mean per step): " + "; ".join(f"{k} {v:.2f}" for k, v in phase_ms.items()),
          file=sys.stderr, flush=True)
    srt = sorted(step_ms)
    line = {
        "metric": METRIC, "value": round(ms_step / per, 2), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 2), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": DTYPE_TEXT[(args.hessian_math, bool(args.x_fp32))],
        "data": "synthetic (seeded, generated on the GPU)",
        "config": {"workload": WORKLOAD[args.config].format(alpha=cfg["alpha"]), "parallelism": "single GPU",
                   "hessian_math": args.hessian_math},
        "roofline": roofline(cfg, args, kernel_ms, launches, args.steps),
        "step_ms": {"min": round(srt[0], 2), "median": round(srt[len(srt) // 2], 2), "max": round(srt[-1], 2)},
        "phase_ms": {k: round(v, 2) for k, v in phase_ms.items()},
    }
    if not args.no_cpu_baseline:
        if layer_mode:
            if kept is None:
                kept = step(keep=True)
            line["cpu_baseline"] = cpu_baseline_layer(xs, mods, kept, cfg)
        elif args.config == "cfg5":
            if args.cpu_baseline_sample:
                line["cpu_baseline"] = cpu_baseline_hessian_sample(X, s, cfg)
        else:
            line["cpu_baseline"] = cpu_baseline_linear(X, W, s, grad, cfg, args.cpu_chunks)
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", choices=sorted(CONFIGS), default="cfg3",
                    help="cfgK = BASELINE.json configs[K-1]; default cfg3 (the Llama-3-8B layer)")
    ap.add_argument("--alpha", type=float, default=0.0, help="GPTQ+ alpha (with --ref-loss > 0: beta != 0)")
    ap.add_argument("--ref-loss", type=float, default=0.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-chunks", type=int, default=2)
    ap.add_argument("--cpu-baseline-sample", action="store_true",
                    help="with --config cfg5: time the CPU oracle's Hessian accumulation on one sample")
    ap.add_argument("--hessian-math", choices=sorted(PIECES), default="split16x3",
                    help="Hessian kernel for fp16 inputs: split16x3 (default: three fp16 MFMA products per fp32 "
                         "product, exact), split16 (two: within 2^-23 relative), fp32 (fp32 MFMA)")
    ap.add_argument("--shared-fasterquant", action="store_true",
                    help="layer configs: fasterquant_shared for the linears that share an input (their Cholesky "
                         "chains as one batch) instead of one fasterquant call per linear")
    ap.add_argument("--x-fp32", action="store_true",
                    help="fp32 activations (the reference's add_batch takes any float dtype): the same inputs "
                         "converted to fp32")
    ap.add_argument("--copy-calibration", action="store_true", help="only run a 1 GiB device copy (counter calibration)")
    ap.add_argument("--gemm-calibration", action="store_true", help="only time torch.matmul in fp16 / fp32 / fp64")
    ap.add_argument("--stats-table", metavar="STATS_CSV", help="print a rocprofv3 kernel-stats CSV as a table")
    ap.add_argument("--units", type=float, default=1.0, help="with --stats-table: units (linears or layers) profiled")
    ap.add_argument("--counters-table", metavar="PMC_CSV", help="print a rocprofv3 --pmc CSV as a per-kernel table")
    ap.add_argument("--traffic", nargs=4, metavar=("FETCH", "WRITE", "CAL_FETCH", "CAL_WRITE"),
                    help="counter CSVs of the product kernel and of the copy calibration -> profiles/hessian_traffic.json")
    args = ap.parse_args()
    if args.stats_table:
        stats_table(args.stats_table, CONFIGS[args.config], args.units, args.config)
        return
    if args.counters_table:
        counters_table(args.counters_table)
        return
    if args.traffic:
        cfg = CONFIGS[args.config]
        traffic_report(*args.traffic, "k_hessian_split" if args.hessian_math != "fp32" else "k_hessian_accum",
                       args.config, cfg, args.hessian_math)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs the GPTQ+ hot path on one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding is a design note, not a launched path.", file=sys.stderr)
        sys.exit(2)
    run(args)


if __name__ == "__main__":
    main()

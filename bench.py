"""Benchmark: ms per linear (Hessian accumulation + GPTQ+ fasterquant) on one MI355X.

Workload: one 4096x4096 q_proj linear, fp16 W ~ N(0, 0.02^2);
calibration X = 128 samples x 2048 tokens x 4096 fp16 ~ N(0,1) with 8 outlier channels x20;
NUM_GROUPS = 4 token saliencies ~ LogNormal(0,1) clipped at their 0.99 quantile; GPTQ+
first-order term on with G ~ N(0, 1e-4^2) and alpha = 0; w4 asymmetric per-channel,
act_order, BLOCKSIZE = 128, percdamp = 0.01; 16-sample add_batch chunks.
A step = one linear: 8 add_batch calls + finalize_hessian + fasterquant, inputs resident in
HBM.  Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
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

CFG = dict(R=4096, C=4096, G=4, N=128, T=2048, bsz=16, bits=4, sym=False, blocksize=128,
           percdamp=0.01, alpha=0.0, outliers=8, seed=20251201)


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
    W = (torch.randn((R, C), generator=gen, device=dev) * 0.02).half()
    s = torch.exp(torch.randn((N, T, G), generator=gen, device=dev))
    for g in range(G):
        q = torch.quantile(s[..., g].flatten(), 0.99)          # linear interpolation
        s[..., g].clamp_(max=float(q))
    grad = torch.randn((R, C), generator=gen, device=dev) * 1e-4
    return X, W, s, grad


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
    g.fasterquant(blocksize=cfg["blocksize"], percdamp=cfg["percdamp"], groupsize=-1, actorder=True,
                  static_groups=True)
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
    o.fasterquant(blocksize=cfg["blocksize"], percdamp=cfg["percdamp"], groupsize=-1, actorder=True,
                  static_groups=True)
    t_fq = time.perf_counter() - t1
    nchunks = cfg["N"] // cfg["bsz"]
    total_s = t_acc * nchunks / chunks + t_fq
    return dict(value=round(total_s * 1e3, 1), unit="ms per linear (extrapolated)", cores=threads,
                kind="port",
                sample=(f"oracle (reference torch op sequence) on host CPU: {chunks}/{nchunks} add_batch "
                        f"chunks timed ({t_acc:.1f} s, x{nchunks // chunks} by tokens) + full "
                        f"finalize_hessian+fasterquant ({t_fq:.1f} s); {platform.processor() or platform.machine()}"))


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


def load_traffic():
    path = os.path.join(ROOT, "profiles", "hessian_traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-chunks", type=int, default=2)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (counter calibration for the traffic figure)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs the GPTQ+ hot path on one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding is a design note, not a launched path.", file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        copy_calibration(dev)
        return
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = dict(CFG)
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
    achieved = flops / (h_ms * 1e-3) / 1e12

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
        "dtype": "fp32 (fp16 inputs)",
        "data": "synthetic (seeded, generated on the GPU)",
        "config": {"workload": "configs[1]: q_proj 4096x4096, NUM_GROUPS=4, 128x2048 tokens, w4 asym "
                               "per-channel, act_order, B=128, GPTQ+ term on (alpha=0)",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                     "traffic": load_traffic(),
                     "kernel": "k_hessian_accum", "launch_ms": round(h_ms, 3), "launches": n_launch,
                     "flops_per_launch": flops},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(X, W, s, grad, cfg, args.cpu_chunks)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

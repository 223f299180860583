"""E-step throughput on one MI355X: samples/s and fraction of the fp32 MFMA peak.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline]

Workload: the isotropic E-step at N=1,000,000, K=1024, D=128, float32, on the
clustered synthetic data of flash_gmm.data.iso_clustered (seed 1), generated
on the GPU so X is resident in HBM before timing.  One step = one full E-step
(constant prologue + log-normaliser pass + accumulation pass + reduction)
through the C ABI on torch's current stream.  Prints one JSON line.
"""

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "flash-gmm_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "E-step samples/sec @K=1024,D=128 fp32 + % of fp32 MFMA peak (1 GPU)"
PEAK_FP32_MFMA_TFLOPS = 157.3       # MI355X dense fp32 matrix, published
PEAK_HBM_GBS = 8000.0
A100_SAMPLES_PER_S = 1_000_000 / 0.152   # README.md:116 (A100 80GB, N=1M, 152 ms)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def cpu_baseline(inp, K, D, min_s=10.0, max_s=30.0, rows=16384):
    """The oracle's float32 restatement on the host cores, on a bounded sample."""
    import torch
    from oracle import gmm_oracle as O

    threads = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(threads)
    X = inp["X"][:rows].cpu()
    mu, lss, lpi = (inp[k].cpu() for k in ("mu", "log_sigma_sq", "log_pi"))
    O.estep_iso(X[:1024], mu, lss, lpi, dtype=torch.float32)  # warm
    done, t0 = 0, time.perf_counter()
    reps = 0
    while True:
        O.estep_iso(X, mu, lss, lpi, dtype=torch.float32, chunk=rows)
        done += rows
        reps += 1
        el = time.perf_counter() - t0
        if el >= min_s or el >= max_s:
            break
    return {
        "value": done / el, "unit": "samples/s", "cores": threads, "kind": "port",
        "sample": f"{rows} rows of the same workload (K={K}, D={D}) x {reps} repetitions, "
                  f"{el:.1f} s, float32 oracle (torch CPU) on {cpu_model()}",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--atomic-reduce", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures a single GPU; --gpus {args.gpus} is not supported "
              "(the E-step shards by rows with one all-reduce of O(K*D) statistics, "
              "which is not built here).", file=sys.stderr)
        sys.exit(2)

    import torch
    from flash_gmm import data, iso_estep_into
    from flash_gmm import _lib

    dev = torch.device("cuda:0")
    N, K, D = 1_000_000, 1024, 128
    log(f"generating workload iso_n1m_k1024_d128 on {torch.cuda.get_device_name(dev)}")
    inp = data.iso_clustered(N, K, D, seed=1, device=dev)
    X, mu, lss, lpi = (inp[k] for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    logZ = torch.empty(N, device=dev)
    Nk = torch.empty(K, device=dev)
    mu_acc = torch.empty(K, D, device=dev)
    sig = torch.empty(K, device=dev)
    ws = torch.empty(int(_lib.lib().fgmm_iso_workspace_bytes(N, K, D)), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)

    def step(ev=None):
        if ev is not None:
            ev[0].record(stream)
        iso_estep_into(X, mu, lss, lpi, logZ, Nk, mu_acc, sig, workspace=ws, phase=1,
                       atomic_reduce=args.atomic_reduce)
        if ev is not None:
            ev[1].record(stream)
        iso_estep_into(X, mu, lss, lpi, logZ, Nk, mu_acc, sig, workspace=ws, phase=2,
                       atomic_reduce=args.atomic_reduce)
        if ev is not None:
            ev[2].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"warmup done; sum Nk = {Nk.double().sum().item():.3f} (N = {N})")

    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(args.steps):
        step(evs[i])
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    ms = total_ms / args.steps
    p1 = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    p2 = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
    log(f"timed {args.steps} steps: {ms:.3f} ms/step (phase1 {p1:.3f} ms, phase2 {p2:.3f} ms)")

    half_flop = 2.0 * N * K * D          # x.mu^T (phase 1) or r^T X (phase 2), algorithmic
    step_tflops = 2 * half_flop / (ms * 1e-3) / 1e12
    dom, dom_ms = ("iso_accum (accumulation pass + slab reduction)", p2) if p2 >= p1 else \
        ("iso_lse (log-normaliser pass + prologue)", p1)
    dom_tflops = half_flop / (dom_ms * 1e-3) / 1e12
    executed = (6.0 * N * K * D) / (ms * 1e-3) / 1e12

    out = {
        "metric": METRIC,
        "value": N / (ms * 1e-3),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (N / (ms * 1e-3)) / A100_SAMPLES_PER_S,
        "baseline_note": "reference's published A100 80GB figure for this shape: 152 ms at N=1M "
                         "(README.md:116), TF32 dot",
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "iso_n1m_k1024_d128", "N": N, "K": K, "D": D,
                   "generator": "flash_gmm.data.iso_clustered(seed=1), generated on device",
                   "reduce": "atomic" if args.atomic_reduce else "deterministic"},
        "fraction_of_fp32_mfma_peak": step_tflops / PEAK_FP32_MFMA_TFLOPS,
        "step_tflops_algorithmic": step_tflops,
        "executed_mfma_tflops": executed,
        "phase_ms": {"phase1_lse": p1, "phase2_accum": p2},
        "roofline": {
            "bound": "mfma",
            "kernel": dom,
            "achieved": dom_tflops,
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": dom_tflops / PEAK_FP32_MFMA_TFLOPS,
            "traffic": None,
            "algorithmic_flop_per_launch": half_flop,
            "avg_launch_ms": dom_ms,
        },
    }
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (bounded sample)")
        out["cpu_baseline"] = cpu_baseline({k: v for k, v in inp.items()}, K, D)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

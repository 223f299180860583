"""E-step throughput on one MI355X: samples/s and fraction of the fp32 MFMA peak.

    python bench.py [--gpus 1] [--steps 20] [--warmup 20] [--no-cpu-baseline]
                    [--workload iso_n1m_k1024_d128|diag_n1m_k1024_d96|full_n250k_k256_d64]

Default workload (the headline): the isotropic E-step at N=1,000,000, K=1024,
D=128, float32, on the clustered synthetic data of flash_gmm.data.iso_clustered
(seed 1), generated on the GPU so X is resident in HBM before timing.  One step
= one full E-step (constant prologue + log-normaliser pass + accumulation pass +
reduction) through the C ABI on torch's current stream.  Prints one JSON line.
The diagonal and full-covariance workloads are measured the same way.
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
PEAK_BF16_MFMA_TFLOPS = 2500.0      # MI355X dense bf16 matrix, published
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


def cpu_baseline(inp, kind, K, D, min_s=10.0, max_s=30.0, rows=16384):
    """The oracle's float32 restatement on the host cores, on a bounded sample."""
    import torch
    from oracle import gmm_oracle as O

    threads = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(threads)
    if kind == "full":
        rows = 4096
    X = inp["X"][:rows].cpu()
    third = "prec_chol" if kind == "full" else "log_sigma_sq"
    mu, p3, lpi = (inp[k].cpu() for k in ("mu", third, "log_pi"))
    fn = {"iso": O.estep_iso, "diag": O.estep_diag, "full": O.estep_full}[kind]
    fn(X[:512], mu, p3, lpi, dtype=torch.float32)  # warm
    done, t0 = 0, time.perf_counter()
    reps = 0
    while True:
        fn(X, mu, p3, lpi, dtype=torch.float32, chunk=rows)
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


# HBM bytes per launch of each pass's main kernel with the stored log-joint (the
# default): rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (separate runs) on this
# bench command, scaled by what the counters read for a 512 MiB device copy (x2.0
# for FETCH_SIZE, x1.0 for WRITE_SIZE); the counter values and commands are in
# profiles/<kind>_estep_<shape>.md.  Not reported with --recompute.
TRAFFIC_BYTES = {
    "iso_n1m_k1024_d128": {"phase1": 3_140_715_520, "phase2": 799_602_688},
    "diag_n1m_k1024_d96": {"phase1": 4_374_549_504, "phase2": 656_783_360},
    "full_n250k_k256_d64": {"phase1": 836_218_880, "phase2": 414_390_272},
}

WORKLOADS = {
    # name: (N, K, D)
    "iso_n1m_k1024_d128": (1_000_000, 1024, 128),
    "diag_n1m_k1024_d96": (1_000_000, 1024, 96),
    "full_n250k_k256_d64": (250_000, 256, 64),
    "diag_n1m_k256_d256": (1_000_000, 256, 256),
    "full_n100k_k64_d128": (100_000, 64, 128),
}


def algorithmic_flop(kind, N, K, D):
    """Per-step algorithmic flops and the (phase 1, phase 2) split.

    iso:  4NKD  = x.mu^T (2NKD, phase 1) + r^T X (2NKD, phase 2)
    diag: 8NKD  = [x^2, x].[-w, 2v]^T (4NKD, phase 1) + r^T [X, X^2] (4NKD, phase 2)
    full: 4NKD^2 + 2NKD = X.L_k whitening (2NKD^2, phase 1) + sum r x x^T (2NKD^2)
          + r^T X (2NKD) in phase 2 (dense-equivalent count)
    """
    if kind == "iso":
        return 4.0 * N * K * D, 2.0 * N * K * D, 2.0 * N * K * D
    if kind == "diag":
        return 8.0 * N * K * D, 4.0 * N * K * D, 4.0 * N * K * D
    return 4.0 * N * K * D * D + 2.0 * N * K * D, 2.0 * N * K * D * D, 2.0 * N * K * D * D + 2.0 * N * K * D


def algorithmic_bytes(kind, N, K, D, lj):
    """Per-step HBM bytes each phase must move (phase 1, phase 2).

    Phase 1 reads X and writes logZ, the per-row state (iso: ||x||^2 and logZ2 in
    fp64; diag, full: logZ2) and, when pass 2 reads it, the fp32 log-joint.
    Phase 2 reads X, the per-row state and the log-joint.  O(K*D) operands and the
    slab partials are left out (under 1% here).

    The isotropic log-joint, and the diagonal one up to D = 128, are sparse: phase 1
    writes it whole at most (rows the running max already rules out are left
    unwritten) with per-row block maxima and need masks per tile (iso: one maximum
    per row and one mask word; diag: one per half block, 64 maxima and two words),
    and phase 2 reads X, the row state and the masks, plus only the log-joint rows
    whose need bit is set, a data-dependent share that is not counted here (the
    measured traffic includes it).
    """
    KB = -(-K // 32)
    if kind == "full":
        lj_bytes = (-(-N // 128) * 4) * (-(-K // 4) * 4) * 32 * 4
    else:
        lj_bytes = (-(-N // 128) * 4) * KB * 4096
    lj_bytes = lj_bytes if lj else 0
    row = 16 if kind == "iso" else 8
    x = 4.0 * N * D
    if lj and (kind == "iso" or (kind == "diag" and D <= 128)):
        per_tile = (128, 4) if kind == "iso" else (256, 8)   # maxima, mask words
        tiles = lj_bytes / 4096
        return (x + 4.0 * N + row * N + lj_bytes + tiles * sum(per_tile),
                x + row * N + tiles * per_tile[1])
    return x + 4.0 * N + row * N + lj_bytes, x + row * N + lj_bytes


def stream_main(args):
    """Streaming EM over host-generated rows (pinned double buffers, copy/compute overlap)."""
    import numpy as np
    import torch
    from flash_gmm import SynthIsoSource, data, stream_em_iso

    dev = torch.device("cuda:0")
    N, K, D = args.rows or 1_000_000_000, 1024, 128
    chunk = 16 << 20
    iters = 3
    # Centres and starting parameters of the clustered isotropic model (seed 4);
    # rows x_n = c[a_n] + N(0, I) come from the native counter-based generator.
    model = data.iso_clustered(1, K, D, seed=4)
    g = torch.Generator().manual_seed(4)
    centres = torch.randn(K, D, generator=g) * 2.0
    mu = (centres + 0.5 * torch.randn(K, D, generator=g)).to(dev)
    lss = torch.zeros(K, device=dev)
    lpi = model["log_pi"].to(dev)
    threads = min(len(os.sched_getaffinity(0)), 16)
    src = SynthIsoSource(centres.numpy(), seed=4, threads=threads)
    log(f"streaming EM: N={N} rows, K={K}, D={D}, chunks of {chunk} rows, {iters} iterations, "
        f"{threads} host threads")
    # Device-wide used memory, sampled while the driver runs (the ctypes call
    # releases the GIL); the driver's own allocation total is reported beside it.
    import threading
    free0, total_mem = torch.cuda.mem_get_info(dev)
    peak_used = [total_mem - free0]
    done = threading.Event()

    def sample():
        while not done.wait(0.25):
            f, t = torch.cuda.mem_get_info(dev)
            peak_used[0] = max(peak_used[0], t - f)

    th = threading.Thread(target=sample, daemon=True)
    th.start()
    try:
        rep = stream_em_iso(src, N, mu, lss, lpi, iterations=iters, chunk_rows=chunk,
                            exact_variance=True)
    finally:
        done.set()
        th.join()
    total_s = rep["total_ms"] / 1e3
    out = {
        "metric": f"streaming EM end-to-end rows/s (N={N}, K={K}, D={D}, {iters} iterations, fp32)",
        "value": N * iters / total_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": iters,
        "warmup": 0,
        "ms_per_step": rep["total_ms"] / iters,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "baseline_note": "reference: ~28 min for one pass over N=1B on an A100 (README.md:103)",
        "dtype": "f32",
        "data": "synthetic (host generator, Philox4x32-10 + Box-Muller)",
        "config": {"workload": "stream_em_n1b_k1024_d128", "N": N, "K": K, "D": D, "chunk_rows": chunk,
                   "iterations": iters, "host_threads": threads},
        "end_to_end_s": total_s,
        "setup_s": rep["setup_ms"] / 1e3,
        "host_generation_s": rep["source_ms"] / 1e3,
        "h2d_device_s": rep["h2d_ms"] / 1e3,
        "estep_device_s": rep["estep_ms"] / 1e3,
        "mstep_device_s": rep["mstep_ms"] / 1e3,
        "h2d_GBps": (N * iters * D * 4) / max(rep["h2d_ms"], 1e-9) / 1e6,
        "peak_device_bytes_driver": rep["device_bytes"],
        "device_used_bytes_before": total_mem - free0,
        "device_used_bytes_peak": peak_used[0],
        "pinned_host_bytes": rep["pinned_bytes"],
        "loglik_per_iteration": rep["loglik"],
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--atomic-reduce", action="store_true")
    ap.add_argument("--dense", action="store_true",
                    help="also run accumulation steps whose responsibilities are all zero")
    ap.add_argument("--no-dense-run", action="store_true",
                    help="skip the dense comparison run (profiling the default launches alone)")
    ap.add_argument("--workload", default="iso_n1m_k1024_d128",
                    choices=sorted(WORKLOADS) + ["stream_em_n1b_k1024_d128"])
    ap.add_argument("--rows", type=int, default=0, help="override N of the streaming workload")
    ap.add_argument("--precision", choices=["fp32", "bf16"], default="fp32",
                    help="bf16 runs the H100 variants' bf16 operand contract (FGMM_FLAG_BF16) "
                         "and is rated against the bf16 matrix peak")
    ap.add_argument("--store-log-joint", action="store_true",
                    help="pass 1 stores the N x K log-joint and pass 2 reads it "
                         "(FGMM_FLAG_STORE_LOGJOINT; O(N*K) workspace) instead of the default plan")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB five times (scales the "
                         "FETCH_SIZE / WRITE_SIZE counters to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures a single GPU; --gpus {args.gpus} is not supported "
              "(the E-step shards by rows with one all-reduce of O(K*D) statistics, "
              "which is not built here).", file=sys.stderr)
        sys.exit(2)

    if args.workload.startswith("stream_em"):
        stream_main(args)
        return
    if args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 4
        a = torch.ones(n, device="cuda:0")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4, "launches": 5}), flush=True)
        return

    import torch
    from flash_gmm import _lib, data, diag_estep_into, full_estep_into, iso_estep_into

    dev = torch.device("cuda:0")
    N, K, D = WORKLOADS[args.workload]
    kind = args.workload.split("_")[0]
    bf16 = args.precision == "bf16"
    peak = PEAK_BF16_MFMA_TFLOPS if bf16 else PEAK_FP32_MFMA_TFLOPS
    log(f"generating workload {args.workload} on {torch.cuda.get_device_name(dev)}")
    inp = data.make(args.workload, device=dev)
    L = _lib.lib()
    logZ = torch.empty(N, device=dev)
    Nk = torch.empty(K, device=dev)
    mu_acc = torch.empty(K, D, device=dev)
    if kind == "iso":
        args4 = (inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"])
        sig = torch.empty(K, device=dev)
        fn = lambda ph, dense=args.dense: iso_estep_into(*args4, logZ, Nk, mu_acc, sig, workspace=ws,
                                                         phase=ph, atomic_reduce=args.atomic_reduce,
                                                         dense=dense, store_log_joint=args.store_log_joint,
                                                         precision=args.precision)
    elif kind == "diag":
        args4 = (inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"])
        sig = torch.empty(K, D, device=dev)
        fn = lambda ph, dense=args.dense: diag_estep_into(*args4, logZ, Nk, mu_acc, sig, workspace=ws,
                                                          phase=ph, dense=dense, store_log_joint=args.store_log_joint,
                                                          precision=args.precision)
    else:
        args4 = (inp["X"], inp["mu"], inp["prec_chol"], inp["log_pi"])
        sig = torch.empty(K, D, D, device=dev)
        fn = lambda ph, dense=args.dense: full_estep_into(*args4, logZ, Nk, mu_acc, sig, workspace=ws,
                                                          phase=ph, dense=dense, store_log_joint=args.store_log_joint,
                                                          precision=args.precision)
    ws_fn = getattr(L, f"fgmm_{kind}_workspace_bytes_ex")
    pflag = _lib.FLAG_BF16 if bf16 else 0
    flags = (_lib.FLAG_STORE_LOGJOINT if args.store_log_joint else 0) | pflag
    ws = torch.empty(int(ws_fn(N, K, D, flags)), dtype=torch.uint8, device=dev)
    # Pass 2 reads the log-joint that pass 1 stores whenever the plan sizes it in.
    stored_lj = (int(ws_fn(N, K, D, pflag)) != int(ws_fn(N, K, D, pflag | _lib.FLAG_STORE_LOGJOINT))
                 and args.store_log_joint)
    stream = torch.cuda.current_stream(dev)

    def step(ev=None):
        if ev is not None:
            ev[0].record(stream)
        fn(1)
        if ev is not None:
            ev[1].record(stream)
        fn(2)
        if ev is not None:
            ev[2].record(stream)

    def dense_step():
        fn(1, True)
        fn(2, True)

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

    dense_ms = None
    if not args.dense and not args.no_dense_run:
        # The same steps with every accumulation step executed (identical outputs):
        # the dense cost, reported beside the default.
        for _ in range(2):
            dense_step()
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(args.steps):
            dense_step()
        end.record(stream)
        torch.cuda.synchronize()
        dense_ms = start.elapsed_time(end) / args.steps
        log(f"dense accumulation: {dense_ms:.3f} ms/step")

    flop, f1, f2 = algorithmic_flop(kind, N, K, D)
    b1, b2 = algorithmic_bytes(kind, N, K, D, stored_lj)
    step_tflops = flop / (ms * 1e-3) / 1e12
    p2_kernel = {"iso": "iso_accum", "diag": "diag_accum", "full": "full_accum"}[kind] + (
        "_lj" if stored_lj and kind != "full" else "")
    if kind == "iso" and stored_lj and D % 32 == 0 and D <= 128:
        p2_kernel = "iso_accum_sparse or iso_accum_lj, picked on device by mask density"
    if kind == "diag" and stored_lj and D <= 128:
        p2_kernel = ("diag_accum_sparse or diag_accum_lj2, picked on device by mask density"
                     if D % 32 == 0 else "diag_accum_lj2")
    split_p1 = (kind in ("iso", "diag") and D <= 128) or (kind == "full" and stored_lj)
    p1_kernel = f"{kind}_lse" + ("_x6" if split_p1 and kind != "iso" else "")
    names = (f"{p1_kernel} (log-normaliser pass + prologue"
             + (", split-bf16 products" if split_p1 else "")
             + (", stores the log-joint)" if stored_lj else ")"),
             f"{p2_kernel} (accumulation pass + slab reduction"
             + (", reads the stored log-joint)" if stored_lj else ", recomputes the log-joint)"))
    if bf16:
        names = (f"{kind}_bf16_lse (log-normaliser pass + prologue, bf16 operands"
                 + (", stores the log-joint)" if kind == "full" else ")"),
                 f"{kind}_bf16_accum (accumulation pass + slab reduction, "
                 + ("reads the stored log-joint)" if kind == "full" else "recomputes in bf16)"))
    traffic_tab = {} if (not args.store_log_joint or bf16) else TRAFFIC_BYTES.get(args.workload, {})
    phases = {}
    for ph, name, t, f, b in (("phase1", names[0], p1, f1, b1), ("phase2", names[1], p2, f2, b2)):
        phases[ph] = {"kernel": name, "ms": t, "algorithmic_flop": f,
                      "tflops": f / (t * 1e-3) / 1e12, "algorithmic_bytes": b,
                      "gbs": b / (t * 1e-3) / 1e9, "traffic": traffic_tab.get(ph)}
    dom_phase = "phase2" if p2 >= p1 else "phase1"
    dom = phases[dom_phase]
    # Phase 1 and the recomputing phase 2 are matrix-core bound.  Reading the stored
    # log-joint, phase 2 moves ~8 bytes per (row, component) and skips the steps whose
    # responsibilities are all zero: it is HBM bound.
    hbm_bound = dom_phase == "phase2" and stored_lj and not args.dense
    if hbm_bound:
        roof = {"bound": "hbm", "achieved": dom["gbs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": dom["gbs"] / PEAK_HBM_GBS, "algorithmic_bytes_per_launch": dom["algorithmic_bytes"]}
    else:
        roof = {"bound": "mfma", "achieved": dom["tflops"], "peak": peak,
                "unit": "TFLOP/s", "frac": dom["tflops"] / peak,
                "algorithmic_flop_per_launch": dom["algorithmic_flop"]}
    roof.update({"kernel": dom["kernel"], "traffic": dom["traffic"],
                 "traffic_unit": "bytes per launch (HBM read + write, rocprofv3 counters)",
                 "avg_launch_ms": dom["ms"]})
    # Phase 1 forms its fp32 contraction from split-bf16 products on the bf16 matrix
    # cores: 7 steps (6 products + 1 centring offset) per chunk and 32x32 tile, each
    # step 32 bf16 flop per (row, output).  Per (row, component):
    #   iso:  16-dimension chunks, 1 output:          14 D bf16 flop (2 D algorithmic)
    #   diag: 8-dimension chunks of [x^2, x]:         28 D               (4 D)
    #   full: 16-dimension chunks, D outputs:         14 D^2             (2 D^2)
    # (D padded: iso to 16, diag and full to 32.)  Full recomputation keeps fp32 steps.
    ex = None
    if not bf16 and dom_phase == "phase1":
        if kind == "iso" and D <= 128:
            ex = 14.0 * N * K * (D + (-D) % 16)
        elif kind == "diag" and D <= 128:
            ex = 28.0 * N * K * (D + (-D) % 32)
        elif kind == "full" and stored_lj:
            ex = 14.0 * N * K * (D + (-D) % 32) ** 2
    if ex is not None:
        roof["executed"] = {"arithmetic": "split-bf16 (bf16x6) products, fp32 accumulation, fp64 "
                                          "combination; fp32 inputs and outputs",
                            "bf16_flop_per_launch": ex,
                            "bf16_tflops": ex / (dom["ms"] * 1e-3) / 1e12,
                            "bf16_peak": PEAK_BF16_MFMA_TFLOPS,
                            "bf16_frac": ex / (dom["ms"] * 1e-3) / 1e12 / PEAK_BF16_MFMA_TFLOPS}

    out = {
        "metric": (METRIC if kind == "iso" and not bf16 else
                   f"E-step samples/sec ({args.workload}) bf16 operands, fp32 accumulation "
                   "+ % of bf16 MFMA peak (1 GPU)" if bf16 else
                   f"E-step samples/sec ({args.workload}) fp32 + % of fp32 MFMA peak (1 GPU)"),
        "value": N / (ms * 1e-3),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (N / (ms * 1e-3)) / A100_SAMPLES_PER_S if kind == "iso" and not bf16 else None,
        "baseline_note": "reference's published A100 80GB figure for this shape: 152 ms at N=1M "
                         "(README.md:116), TF32 dot" if kind == "iso" else
                         "no published reference number for this workload",
        "dtype": "bf16 operands, f32 accumulation" if bf16 else "f32",
        "data": "synthetic",
        "config": {"workload": args.workload, "N": N, "K": K, "D": D,
                   "generator": f"flash_gmm.data.make({args.workload!r}), generated on device",
                   "reduce": "atomic" if args.atomic_reduce else "deterministic",
                   "log_joint": "stored by phase 1, read by phase 2" if stored_lj else "recomputed by phase 2"},
        "fraction_of_fp32_mfma_peak": step_tflops / PEAK_FP32_MFMA_TFLOPS,
        "fraction_of_matrix_peak": step_tflops / peak,
        "fraction_basis": "dense-equivalent algorithmic flops per step / step time; phase 2 executes "
                          "only the accumulation steps whose responsibilities are not all zero"
                          + (" and reads the log-joint instead of recomputing it" if stored_lj else "")
                          + ", so the matrix work executed is lower: the dense run and the per-phase "
                            "rates below are the executed figures",
        "step_tflops_algorithmic": step_tflops,
        "phase_ms": {"phase1": p1, "phase2": p2},
        "phases": phases,
        "accumulation": "dense" if args.dense else
                        "skips steps whose responsibilities are all exactly zero (bitwise-identical outputs)",
        "dense_ms_per_step": dense_ms if dense_ms is not None else (ms if args.dense else None),
        "dense_fraction_of_fp32_mfma_peak": (flop / (dense_ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS)
                                            if dense_ms is not None else None,
        "dense_fraction_of_matrix_peak": (flop / (dense_ms * 1e-3) / 1e12 / peak)
                                         if dense_ms is not None else None,
        "roofline": roof,
    }
    if not args.no_cpu_baseline and not bf16:
        log("timing the CPU baseline (bounded sample)")
        out["cpu_baseline"] = cpu_baseline({k: v for k, v in inp.items()}, kind, K, D)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

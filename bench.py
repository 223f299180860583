"""E-step throughput on one MI355X: samples/s and the dominant kernel's roofline fraction.

    python bench.py [--gpus 1] [--steps 20] [--warmup 20] [--no-cpu-baseline]
                    [--workload iso_n1m_k1024_d128|iso_ref_n1m_k1024_d128|diag_n1m_k1024_d96|
                                full_n250k_k256_d64|stream_em_n1b_k1024_d128|...]
                    [--precision fp32|bf16] [--store-log-joint] [--no-extra-runs]
    python bench.py --sweep iso:1000000:1024:32,64,96,128,192,256   (one JSON line per D)
    python bench.py --reduce-compare                                (tree vs atomic finish)

Default workload (the headline): the isotropic E-step at N=1,000,000, K=1024,
D=128, float32, on the clustered synthetic data of flash_gmm.data.iso_clustered
(seed 1), generated on the GPU so X is resident in HBM before timing.  One step
= one full E-step on the default O(N + K*D) plan (constant prologue +
log-normaliser pass + accumulation pass + reduction) through the C ABI on
torch's current stream.  Prints one JSON line.  The other workloads are measured
the same way; the stored log-joint plan (FGMM_FLAG_STORE_LOGJOINT) and the dense
accumulation are timed after the headline and reported as extra keys.
"""

import argparse
import json
import math
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
LJ_NEED_GAP = 160.0                 # log2 units: a (row, block) below this under logZ2 is skipped

WORKLOADS = {
    # name: (N, K, D)
    "iso_n1m_k1024_d128": (1_000_000, 1024, 128),
    "iso_ref_n1m_k1024_d128": (1_000_000, 1024, 128),
    "diag_n1m_k1024_d96": (1_000_000, 1024, 96),
    # the reference's dense data (X, mu ~ N(0, I)) for the diagonal and full models
    "diag_ref_n1m_k1024_d96": (1_000_000, 1024, 96),
    "full_ref_n250k_k256_d64": (250_000, 256, 64),
    "full_n250k_k256_d64": (250_000, 256, 64),
    "diag_n1m_k256_d256": (1_000_000, 256, 256),
    "full_n100k_k64_d128": (100_000, 64, 128),
    # widths above 128 (component-tiled pass 1, dimension-range pass 2; full up to 256)
    "iso_n1m_k1024_d256": (1_000_000, 1024, 256),
    "iso_n1m_k1024_d960": (1_000_000, 1024, 960),
    "diag_n1m_k1024_d960": (1_000_000, 1024, 960),
    "full_n100k_k64_d256": (100_000, 64, 256),
}

# HBM traffic per launch from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (separate runs)
# on this bench command (--steps 10 --warmup 2 --no-cpu-baseline --no-extra-runs), each
# scaled by what the counter reads for a 512 MiB device copy (bench.py
# --copy-calibration 512: FETCH_SIZE x2.0, WRITE_SIZE x1.0).  Per kernel of one step:
# (FETCH_SIZE KiB, WRITE_SIZE KiB); the commands and tables are in profiles/.
TRAFFIC_KIB = {
    # (workload, plan, precision): {kernel: (fetch KiB, write KiB)}; "phase1" names pass 1's
    # The drop-in's mode (store_log_joint="auto"): on this clustered data the probe keeps
    # the default plan, and iso_accum_ljt returns at once.
    ("iso_n1m_k1024_d128", "default", "fp32"): {
        "phase1": "iso_lse_pipe<128, 1>",
        "iso_prep": (311, 1_104), "iso_store_probe<128>": (2_680, 2), "iso_lse_pipe<128, 1>": (310_281, 24_414),
        "iso_accum_ljt<128>": (18, 0), "iso_accum_gather<128>": (268_569, 33_280),
        "iso_accum_tiles2<128>": (16, 0), "iso_reduce": (20_842, 664)},
    # The reference's N(0, I) data: the probe selects the stored branch (pass 1 writes the
    # log-joint, the X parts and the logZ pairs; iso_accum_ljt reads them back).
    ("iso_ref_n1m_k1024_d128", "default", "fp32"): {
        "phase1": "iso_lse_pipe<128, 1>",
        "iso_prep": (310, 1_104), "iso_store_probe<128>": (2_679, 2),
        "iso_lse_pipe<128, 1>": (316_772, 4_534_764), "iso_accum_ljt<128>": (2_289_322, 33_280),
        "iso_accum_gather<128>": (22, 0), "iso_accum_tiles2<128>": (13, 0), "iso_reduce": (20_835, 664)},
    ("diag_n1m_k1024_d96", "default", "fp32"): {
        "phase1": "diag_lse_x6<96, 2, 0>",
        "diag_x6_prep": (457, 1_552), "diag_lse_x6<96, 2, 0>": (193_991, 19_532),
        "diag_accum_gather<96>": (207_844, 49_408), "diag_reduce": (25_823, 780)},
    # The drop-in's mode: on this clustered data the probe keeps the default plan, and
    # the stored branch's pass-1 instance and full_accum_ljt return at once.
    ("full_n250k_k256_d64", "default", "fp32"): {
        "phase1": "full_lse_x6<64, 2, 0, 2>",
        "full_x6_prep": (2_134, 8_328), "full_probe_ll<64>": (5_285, 2_048), "full_probe_count": (1_045, 2),
        "full_lse_x6<64, 2, 0, 2>": (177_976, 67_765), "full_lse_x6<64, 2, 1, 0>": (17, 0),
        "full_accum_ljt<64>": (23, 0), "full_accum_gather<64, 0, 0>": (68_174, 25_150),
        "full_reduce_sig": (12_328, 4_096), "full_reduce": (286, 65)},
    # N(0, I) data: the probe selects the stored branch.
    ("full_ref_n250k_k256_d64", "default", "fp32"): {
        "phase1": "full_lse_x6<64, 2, 1, 0>",
        "full_x6_prep": (2_134, 8_328), "full_probe_ll<64>": (5_285, 2_048), "full_probe_count": (1_045, 2),
        "full_lse_x6<64, 2, 0, 2>": (23, 0), "full_lse_x6<64, 2, 1, 0>": (152_892, 253_042),
        "full_accum_ljt<64>": (157_397, 25_096), "full_accum_gather<64, 0, 0>": (15, 0),
        "full_reduce_sig": (12_328, 4_096), "full_reduce": (286, 65)},
    ("full_n100k_k64_d128", "default", "fp32"): {
        "phase1": "full_lse_x6<128, 2, 0, 2>",
        "full_x6_prep": (2_112, 8_258), "full_lse_x6<128, 2, 0, 2>": (135_236, 1_984),
        "full_accum_gather<128, 0, 0>": (94_705, 82_968), "full_reduce_sig": (41_000, 4_096),
        "full_reduce": (542, 32)},
}


def _kib_bytes(fw):
    return fw[0] * 2048 + fw[1] * 1024


TRAFFIC_BYTES = {
    key: {"phase1": _kib_bytes(v[v["phase1"]]),
          "step": sum(_kib_bytes(fw) for k, fw in v.items() if k != "phase1"),
          "step_kernels": {k: _kib_bytes(fw) for k, fw in v.items() if k != "phase1"}}
    for key, v in TRAFFIC_KIB.items()
}


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


def rup(a, b):
    return -(-a // b) * b


def padded_dim(kind, D):
    """D as the kernels pad it: to 32 up to 128, then to 64 (iso, diag); to 32 (full)."""
    if kind == "full":
        return rup(D, 32)
    return rup(D, 32) if D <= 128 else rup(D, 64)


def algorithmic(kind, N, K, D):
    """Per-step algorithmic flops (total, pass 1, pass 2) and pass-1 bytes.

    iso:  4NKD  = x.mu^T (2NKD, pass 1) + r^T X (2NKD, pass 2)
    diag: 8NKD  = [x^2, x].[-w, 2v]^T (4NKD, pass 1) + r^T [X, X^2] (4NKD, pass 2)
    full: 4NKD^2 + 2NKD (dense-equivalent) = whitening (2NKD^2, pass 1)
          + sum r x x^T (2NKD^2) + r^T X (2NKD), pass 2
    Bytes: X read once + logZ written + the O(K*D) parameters (the per-row state and
    need bits the passes exchange are O(N) and O(N K / 32) bits, listed apart).
    """
    if kind == "iso":
        f = (4.0 * N * K * D, 2.0 * N * K * D, 2.0 * N * K * D)
        par = K * (D + 2) * 4
    elif kind == "diag":
        f = (8.0 * N * K * D, 4.0 * N * K * D, 4.0 * N * K * D)
        par = K * (2 * D + 1) * 4
    else:
        f = (4.0 * N * K * D * D + 2.0 * N * K * D, 2.0 * N * K * D * D, 2.0 * N * K * D * D + 2.0 * N * K * D)
        par = K * (D * D + D + 1) * 4
    return f, 4.0 * N * D + 4.0 * N + par


def pass1_executed(kind, N, K, D, precision, stored):
    """Matrix-core flops pass 1 executes per launch, and the unit that runs them.

    Split-bf16 ("bf16x6") passes form each fp32 product from 7 bf16 matrix steps
    (6 products of the three-way splits + 1 centring offset) per chunk, each step
    32 bf16 flop per (row, output), at every width:
      iso:   16-dimension chunks, 1 output:   14 DP bf16 flop per (row, component)
      diag:  8-dimension chunks of [x^2, x]:  28 DP
      full:  16-dimension chunks, DP outputs: 14 DP^2
    The bf16 contract runs one bf16 step per product (2 DP, 4 DP, 2 DP^2 bf16 flop).
    """
    DP = padded_dim(kind, D)
    if precision == "bf16":
        per = {"iso": 2 * DP, "diag": 4 * DP, "full": 2 * DP * DP}[kind]
        return per * float(N) * K, "bf16", PEAK_BF16_MFMA_TFLOPS
    per = {"iso": 14 * DP, "diag": 28 * DP, "full": 14 * DP * DP}[kind]
    return per * float(N) * K, "bf16", PEAK_BF16_MFMA_TFLOPS


def iso_need_pairs(inp, logZ, chunk=65536):
    """Needed (row, 32-component block) pairs, from the inputs and the kernel's logZ:
    a pair is needed when its largest log-joint is within LJ_NEED_GAP (log2 units) of
    logZ2, the kernels' test.  float32 here, so pairs within ~1 unit of the edge may
    be miscounted: an estimate of the gathering pass's work."""
    import torch
    X, mu, lss, lpi = (inp[k] for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    N, D = X.shape
    K = mu.shape[0]
    KB = -(-K // 32)
    b = 0.5 * torch.exp(-lss.double()) * 1.4426950408889634
    C = (lpi.double() - 0.5 * D * (1.8378770664093453 + lss.double())) * 1.4426950408889634
    musq = (mu.double() ** 2).sum(1)
    C0, b, musq = C.float(), b.float(), musq.float()
    total = 0
    for n0 in range(0, N, chunk):
        x = X[n0:n0 + chunk]
        ll2 = C0[None, :] - b[None, :] * ((x * x).sum(1)[:, None] - 2.0 * (x @ mu.T) + musq[None, :])
        pad = KB * 32 - K
        if pad:
            ll2 = torch.nn.functional.pad(ll2, (0, pad), value=-math.inf)
        bm = ll2.view(ll2.shape[0], KB, 32).amax(dim=2)
        lz2 = logZ[n0:n0 + chunk].float() * 1.4426950408889634
        total += int((bm - lz2[:, None] >= -LJ_NEED_GAP).sum())
    return total


def iso_bf16_rtx_pairs(inp, logZ, chunk=65536):
    """(16-row group, 32-component block) pairs of the bf16 contract's pass 2 whose
    bf16(r) is not all zero: the r^T X steps it executes (a step of zeros is skipped).
    The contract's log-joint from bf16-rounded X and mu in float32; r rounds to a
    nonzero bf16 above 2^-134.  Slabs start at multiples of 64 rows, so the groups are
    the rows' 16-row blocks."""
    import torch
    X, mu, lss, lpi = (inp[k] for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    N, D = X.shape
    K = mu.shape[0]
    KB = -(-K // 32)
    ish = (0.5 * torch.exp(-lss.double()) * 1.4426950408889634).float()
    musq = (mu.double() ** 2).sum(1)
    c0 = ((lpi.double() - 0.5 * D * (1.8378770664093453 + lss.double())) * 1.4426950408889634
          - ish.double() * musq).float()
    mub = mu.bfloat16().float()
    total = 0
    for n0 in range(0, N, chunk):
        xb = X[n0:n0 + chunk].bfloat16().float()
        ll2 = c0[None, :] - ish[None, :] * (xb * xb).sum(1)[:, None] + 2.0 * ish[None, :] * (xb @ mub.T)
        lz2 = logZ[n0:n0 + chunk].float() * 1.4426950408889634
        nz = (ll2 - lz2[:, None]) > -134.0
        pad_k, rows = KB * 32 - K, nz.shape[0]
        pad_n = -rows % 16
        if pad_k or pad_n:
            nz = torch.nn.functional.pad(nz, (0, pad_k, 0, pad_n), value=False)
        total += int(nz.view(-1, 16, KB, 32).any(dim=3).any(dim=1).sum())
    return total


def cpu_baseline(inp, kind, K, D, gpu_logZ, min_s=10.0, max_s=30.0, rows=16384):
    """The oracle's float32 restatement on every host core this process may use, on a
    bounded sample of the workload's rows; beside it, the float64 oracle on the same
    rows checks the CPU restatement and the GPU's logZ."""
    import torch
    from oracle import gmm_oracle as O

    threads = len(os.sched_getaffinity(0))
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
        out32 = fn(X, mu, p3, lpi, dtype=torch.float32, chunk=rows)
        done += rows
        reps += 1
        el = time.perf_counter() - t0
        if el >= min_s or el >= max_s:
            break
    ref = fn(X, mu, p3, lpi, dtype=torch.float64)
    lz64 = ref[0]
    return {
        "value": done / el, "unit": "samples/s", "cores": threads, "kind": "port",
        "sample": f"the first {rows} rows of the same workload (K={K}, D={D}) x {reps} passes, "
                  f"{el:.1f} s, float32 oracle (torch CPU) on {threads} threads of {cpu_model()}",
        "max_abs_logZ_err_vs_fp64": {
            "cpu_fp32": float((out32[0].double() - lz64).abs().max()),
            "gpu": float((gpu_logZ[:rows].double().cpu() - lz64).abs().max()),
            "rows": rows,
        },
    }


def make_runner(kind, inp, N, K, D, dev, precision="fp32", store=False, atomic=False):
    """Return (step(phase, dense), workspace bytes) for one plan."""
    import torch
    from flash_gmm import _lib, diag_estep_into, full_estep_into, iso_estep_into

    L = _lib.lib()
    logZ = torch.empty(N, device=dev)
    Nk = torch.empty(K, device=dev)
    mu_acc = torch.empty(K, D, device=dev)
    flags = ((_lib.FLAG_STORE_LOGJOINT_AUTO if store == "auto" else _lib.FLAG_STORE_LOGJOINT if store else 0) |
             (_lib.FLAG_BF16 if precision == "bf16" else 0))
    ws = torch.empty(max(1, int(getattr(L, f"fgmm_{kind}_workspace_bytes_ex")(N, K, D, flags))),
                     dtype=torch.uint8, device=dev)
    if kind == "iso":
        args = (inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"])
        sig = torch.empty(K, device=dev)
        call = lambda ph, dense: iso_estep_into(*args, logZ, Nk, mu_acc, sig, workspace=ws, phase=ph,
                                                atomic_reduce=atomic, dense=dense, store_log_joint=store,
                                                precision=precision)
    elif kind == "diag":
        args = (inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"])
        sig = torch.empty(K, D, device=dev)
        call = lambda ph, dense: diag_estep_into(*args, logZ, Nk, mu_acc, sig, workspace=ws, phase=ph,
                                                 atomic_reduce=atomic, dense=dense, store_log_joint=store,
                                                 precision=precision)
    else:
        args = (inp["X"], inp["mu"], inp["prec_chol"], inp["log_pi"])
        sig = torch.empty(K, D, D, device=dev)
        call = lambda ph, dense: full_estep_into(*args, logZ, Nk, mu_acc, sig, workspace=ws, phase=ph,
                                                 atomic_reduce=atomic, dense=dense, store_log_joint=store,
                                                 precision=precision)
    return call, ws.numel(), (logZ, Nk, mu_acc, sig)


def time_steps(call, steps, warmup, stream, dense=False):
    """W untimed steps, then K timed ones between two synchronisations; each step is
    PHASE1 then PHASE2 with HIP events on the launch stream around each phase."""
    import torch
    for _ in range(warmup):
        call(1, dense)
        call(2, dense)
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(steps):
        evs[i][0].record(stream)
        call(1, dense)
        evs[i][1].record(stream)
        call(2, dense)
        evs[i][2].record(stream)
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    p1 = sum(e[0].elapsed_time(e[1]) for e in evs) / steps
    p2 = sum(e[1].elapsed_time(e[2]) for e in evs) / steps
    return ms, p1, p2


def time_dropin(kind, inp, steps, warmup, stream):
    """The reference's own call, timed as a whole: flash_gmm_estep (or its diagonal /
    full counterpart) on device-resident inputs, with its output allocation, argument
    checks and workspace (torch's caching allocator) inside the timing.  W untimed calls,
    then K timed ones between two synchronisations, HIP events on the stream around
    each call; returns (mean ms per call over the K calls, median per-call ms)."""
    import torch
    from flash_gmm import flash_gmm_estep, flash_gmm_estep_diag, flash_gmm_estep_full
    fn = {"iso": flash_gmm_estep, "diag": flash_gmm_estep_diag, "full": flash_gmm_estep_full}[kind]
    third = "prec_chol" if kind == "full" else "log_sigma_sq"
    args = (inp["X"], inp["mu"], inp[third], inp["log_pi"])
    for _ in range(warmup):
        fn(*args)
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    evs[0].record(stream)
    for i in range(steps):
        fn(*args)
        evs[i + 1].record(stream)
    end.record(stream)
    torch.cuda.synchronize()
    per = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(steps))
    return start.elapsed_time(end) / steps, per[len(per) // 2]


KERNELS = {
    # (kind, plan) -> (pass-1 kernel, pass-2 kernel)
    ("iso", "default"): ("iso_lse_pipe (need masks)", "iso_accum_gather / iso_accum_tiles (by the needed-pair count)"),
    ("iso", "auto"): ("iso_store_probe, iso_lse_pipe (need masks; stores the log-joint where the probe selects it)",
                      "iso_accum_ljt where the probe selected the stored branch, else iso_accum_gather / "
                      "iso_accum_tiles2 (by the needed-pair count)"),
    ("iso", "default_wide"): ("iso_lse_ctile (need masks)", "iso_accum_drange"),
    ("iso", "stored"): ("iso_lse_pipe (stores the log-joint, bf16 X parts, logZ pairs)",
                        "iso_accum_sparse / iso_accum_ljt (by the needed-pair count)"),
    ("iso", "stored_wide"): ("iso_lse_ctile (stores the log-joint)", "iso_accum_lj"),
    ("diag", "default"): ("diag_lse_x6 (need masks)", "diag_accum_gather"),
    ("diag", "auto"): ("diag_store_probe, diag_lse_x6 (need masks; the instance that also stores the "
                       "log-joint, the rows' feature parts and logZ pairs runs where the probe selects it)",
                       "diag_accum_ljt where the probe selected the stored branch, else diag_accum_gather"),
    ("diag", "default_wide"): ("diag_lse_ctile (need masks)", "diag_accum_drange"),
    ("diag", "stored"): ("diag_lse_x6 (stores the log-joint)", "diag_accum_sparse / diag_accum_lj2"),
    ("diag", "stored_wide"): ("diag_lse_ctile (stores the log-joint)", "diag_accum_lj"),
    ("full", "default"): ("full_lse_x6 (need masks)", "full_accum_gather"),
    ("full", "auto"): ("full_probe_ll, full_probe_count, full_lse_x6 (need masks; the instance that also keeps the "
                       "log-joint runs where the probe selects it)",
                       "full_accum_ljt where the probe selected the stored branch, else full_accum_gather"),
    ("full", "stored"): ("full_lse_x6 (stores the log-joint)", "full_accum"),
}


# Widths up to which the drop-in call runs with store_log_joint="auto" (the
# device-selected stored branch; the full model also needs K <= 512).
AUTO_MAX_D = {"iso": 128, "diag": 96, "full": 64}


def dropin_mode(kind, K, D, precision):
    """store_log_joint of the drop-in call for this shape."""
    if precision != "fp32" or D > AUTO_MAX_D[kind] or (kind == "full" and K > 512):
        return False
    return "auto"


def kernel_names(kind, D, precision, stored):
    if precision == "bf16":
        return f"{kind}_bf16_lse", f"{kind}_bf16_accum"
    if stored == "auto":
        return KERNELS[(kind, "auto")] if D <= AUTO_MAX_D[kind] else kernel_names(kind, D, precision, False)
    wide = kind != "full" and D > 128
    if stored and (D > 256 or (kind == "full" and D > 128)):
        stored = False          # the stored plan's widths; above them the call runs the default plan
    plan = ("stored" if stored else "default") + ("_wide" if wide else "")
    return KERNELS[(kind, plan)]


def measure(args, workload, precision, store, dev, inp=None):
    """One plan of one workload: the headline-style record (without the CPU leg)."""
    import torch
    from flash_gmm import data

    N, K, D = WORKLOADS[workload]
    kind = workload.split("_")[0]
    if inp is None:
        inp = data.make(workload, device=dev)
    call, ws_bytes, outs = make_runner(kind, inp, N, K, D, dev, precision, store)
    stream = torch.cuda.current_stream(dev)
    ms, p1, p2 = time_steps(call, args.steps, args.warmup, stream)
    return inp, outs, dict(ms=ms, p1=p1, p2=p2, ws=ws_bytes, call=call)


def main_workload(args):
    import torch

    dev = torch.device("cuda:0")
    workload = args.workload
    N, K, D = WORKLOADS[workload]
    kind = workload.split("_")[0]
    bf16 = args.precision == "bf16"
    log(f"generating workload {workload} on {torch.cuda.get_device_name(dev)}")
    # The phases run the plan the drop-in call takes: store_log_joint="auto" (iso up
    # to D = 128, diag to 96, full to 64), else the default plan.
    mode = True if args.store_log_joint else dropin_mode(kind, K, D, args.precision)
    inp, outs, r = measure(args, workload, args.precision, mode, dev)
    split_ms, p1, p2 = r["ms"], r["p1"], r["p2"]
    log(f"timed {args.steps} steps as two phase calls: {split_ms:.3f} ms/step (phase1 {p1:.3f} ms, "
        f"phase2 {p2:.3f} ms)")
    logZ = outs[0].clone()
    stream = torch.cuda.current_stream(dev)
    # The step: the whole drop-in call (outputs allocated, arguments checked, one C call)
    # for the default fp32 plan; the opt-in plans time their preallocated calls.
    dropin = not bf16 and not args.store_log_joint
    if dropin:
        ms, med = time_dropin(kind, inp, args.steps, args.warmup, stream)
        log(f"timed {args.steps} drop-in calls: {ms:.3f} ms/step (median call {med:.3f} ms)")
    else:
        ms, med = split_ms, None

    (flop, f1, f2), alg_bytes = algorithmic(kind, N, K, D)
    k1, k2 = kernel_names(kind, D, args.precision, mode)
    ex1, unit1, peak1 = pass1_executed(kind, N, K, D, args.precision, args.store_log_joint)
    phases = {
        "phase1": {"kernel": k1 + " + prologue", "ms": p1, "fp32_algorithmic_flop": f1,
                   "fp32_equivalent_tflops": f1 / (p1 * 1e-3) / 1e12,
                   "executed_matrix_flop": ex1, "executed_unit": unit1,
                   "executed_tflops": ex1 / (p1 * 1e-3) / 1e12},
        "phase2": {"kernel": k2 + " + slab reduction", "ms": p2, "fp32_algorithmic_flop": f2,
                   "fp32_equivalent_tflops": f2 / (p2 * 1e-3) / 1e12},
    }
    need = None
    if kind == "iso" and not bf16 and not args.store_log_joint and D <= 128:
        pairs = iso_need_pairs(inp, logZ)
        KB = -(-K // 32)
        DP = padded_dim(kind, D)
        # gathered tiles of 32 rows; per tile the split-bf16 recompute (7 steps per
        # 16 dimensions) and r^T X (3 products, DP/32 column tiles, 2 row steps)
        ex2 = pairs / 32.0 * (7 * DP // 16 + 3 * 2 * DP // 32) * 32768.0
        need = {"needed_row_block_pairs": pairs, "fraction": pairs / (N * KB),
                "basis": "estimated from the inputs and the kernel's logZ (float32)"}
        if mode == "auto" and pairs >= 0.5 * N * KB:
            # The stored branch: r^T X only (3 products, 2 row steps, DP / 32 column
            # tiles) for every (32-row tile, block) with a needed row.
            ex2 = (-(-N // 32)) * KB * 3 * 2 * (DP // 32) * 32768.0
            need["branch"] = "stored (iso_accum_ljt)"
        phases["phase2"].update(executed_matrix_flop=ex2, executed_unit="bf16",
                                executed_tflops=ex2 / (p2 * 1e-3) / 1e12, needed_pairs=need)
    if kind == "iso" and bf16 and not args.store_log_joint:
        DP = padded_dim(kind, D)
        groups = iso_bf16_rtx_pairs(inp, logZ)
        # recomputed S: one step per 16 dimensions for every (32 rows, 32 components);
        # r^T X: DP / 32 steps per needed (16 rows, 32 components)
        ex2 = 2.0 * DP * N * K + groups * (DP // 32) * 32768.0
        phases["phase2"].update(executed_matrix_flop=ex2, executed_unit="bf16",
                                executed_tflops=ex2 / (p2 * 1e-3) / 1e12,
                                rtx_steps={"nonzero_16row_block_pairs": groups,
                                           "fraction": groups / ((-(-N // 16)) * (-(-K // 32))),
                                           "basis": "estimated from the inputs and the kernel's logZ"})
    dom = "phase1" if p1 >= p2 else "phase2"
    d = phases[dom]
    if "executed_matrix_flop" in d:
        unit = d["executed_unit"]
        peak = PEAK_BF16_MFMA_TFLOPS if unit == "bf16" else PEAK_FP32_MFMA_TFLOPS
        roof = {"bound": "mfma", "achieved": d["executed_tflops"], "peak": peak, "unit": "TFLOP/s",
                "frac": d["executed_tflops"] / peak, "kernel": d["kernel"], "avg_launch_ms": d["ms"],
                "achieved_basis": f"matrix flops executed per launch on the {unit} matrix cores / the "
                                  "phase's mean duration (HIP events on the launch stream)",
                "fp32_equivalent_tflops": d["fp32_equivalent_tflops"]}
    else:
        # The executed matrix work of this pass is not modelled here: report no fraction
        # rather than rate dense-equivalent fp32 flops against a peak they do not run on.
        roof = {"bound": "mfma", "achieved": None, "peak": PEAK_BF16_MFMA_TFLOPS, "unit": "TFLOP/s",
                "frac": None, "kernel": d["kernel"], "avg_launch_ms": d["ms"],
                "achieved_basis": "executed matrix work of this pass not modelled; see "
                                  "dense_equivalent_tflops",
                "dense_equivalent_tflops": d["fp32_equivalent_tflops"]}
    traffic = TRAFFIC_BYTES.get((workload, "stored" if args.store_log_joint else "default", args.precision),
                                {}).get(dom)
    roof.update({"traffic": traffic, "traffic_unit": "HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE)",
                 "algorithmic_bytes": alg_bytes if dom == "phase1" else None,
                 "traffic_over_algorithmic": (traffic / alg_bytes) if (traffic and dom == "phase1") else None})

    out = {
        "metric": (METRIC if workload == "iso_n1m_k1024_d128" and not bf16 else
                   f"E-step samples/sec ({workload}) bf16 operands, fp32 accumulation (1 GPU)" if bf16 else
                   f"E-step samples/sec ({workload}) fp32 (1 GPU)"),
        "value": N / (ms * 1e-3),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (N / (ms * 1e-3)) / A100_SAMPLES_PER_S
                       if kind == "iso" and D == 128 and K == 1024 and not bf16 else None,
        "baseline_note": "reference's published A100 80GB figure for this shape: 152 ms at N=1M "
                         "(README.md:116), TF32 dot; context, not the same hardware"
                         if kind == "iso" and K == 1024 and D == 128 else
                         "no published reference number for this workload",
        "dtype": "bf16 operands, f32 accumulation" if bf16 else "f32",
        "data": "synthetic",
        "config": {"workload": workload, "N": N, "K": K, "D": D,
                   "generator": f"flash_gmm.data.make({workload!r}), generated on device",
                   "reduce": "deterministic fixed-order tree",
                   "log_joint": "stored by phase 1, read by phase 2 (opt-in)" if args.store_log_joint
                   else "the default plan with a device-selected stored branch (store_log_joint='auto', "
                        "the drop-in's mode): a row-sample probe chooses per call; need bits from "
                        "phase 1 and gathered rows in phase 2 where few pairs are needed, the stored "
                        "log-joint where most are" if mode == "auto"
                   else "recomputed (default O(N + K*D) plan: need bits from phase 1, gathered rows "
                        "in phase 2)" if (D <= 128 and not bf16)
                   else "recomputed (default O(N + K*D) plan)",
                   "workspace_bytes": r["ws"]},
        "fp32_equivalent_tflops": flop / (ms * 1e-3) / 1e12,
        "fp32_equivalent_basis": "the workload's algorithmic flops (iso 4NKD, diag 8NKD, full 4NKD^2 + 2NKD) per step / step time. Not a "
                                 "roofline: pass 1 forms its fp32 products from split-bf16 steps on the "
                                 "bf16 matrix cores and pass 2 skips the work whose responsibilities are "
                                 "zero; roofline.frac rates the executed work against the peak of the unit "
                                 "that runs it",
        "phases": phases,
        "roofline": roof,
        "step_definition": ("one drop-in call (flash_gmm_estep and its diagonal / full counterparts: "
                            "outputs allocated, arguments checked, both passes and the reduction)"
                            if dropin else "one preallocated call per phase (opt-in plan)"),
        "timing_paths": {"dropin_ms_per_call": ms if dropin else None,
                         "dropin_median_call_ms": med,
                         "phase_split_ms_per_step": split_ms,
                         "note": "phase_split: the same work as two preallocated C calls "
                                 "(FGMM_FLAG_PHASE1, then PHASE2) with HIP events between them; "
                                 "the phases above come from it"},
    }
    st = TRAFFIC_BYTES.get((workload, "stored" if args.store_log_joint else "default", args.precision), {})
    if "step" in st:
        out["step_traffic"] = {"bytes": st["step"], "algorithmic_bytes": alg_bytes,
                               "over_algorithmic": st["step"] / alg_bytes,
                               "kernels": st.get("step_kernels"),
                               "basis": "HBM bytes of every kernel of one step, rocprofv3 FETCH_SIZE x2.0 "
                                        "+ WRITE_SIZE x1.0 (calibrated on a device copy), profiles/"}
    if not args.no_extra_runs:
        call = r["call"]
        dms, d1, d2 = time_steps(call, args.steps, 2, stream, dense=True)
        out["dense_accumulation"] = {"ms_per_step": dms, "phase1_ms": d1, "phase2_ms": d2,
                                     "note": "every row and accumulation step executed (FGMM_FLAG_DENSE)"}
        log(f"dense: {dms:.3f} ms/step")
        if not bf16 and not args.store_log_joint:
            del call, r
            torch.cuda.empty_cache()
            _, _, rs = measure(args, workload, "fp32", True, dev, inp=inp)
            out["stored_log_joint_plan"] = {
                "ms_per_step": rs["ms"], "phase1_ms": rs["p1"], "phase2_ms": rs["p2"],
                "workspace_bytes": rs["ws"], "note": "opt-in FGMM_FLAG_STORE_LOGJOINT: pass 1 stores the "
                                                     "N x K fp32 log-joint, pass 2 reads it"}
            log(f"stored log-joint plan: {rs['ms']:.3f} ms/step")
            del rs
            torch.cuda.empty_cache()
    if workload == "iso_n1m_k1024_d128" and not bf16 and not args.store_log_joint and not args.no_extra_runs:
        # The reference's own benchmark data (flash_gmm.py:228-234: X, mu ~ N(0, I),
        # lss = 0, uniform log pi), where every responsibility is nonzero.
        ref_wl = "iso_ref_n1m_k1024_d128"
        torch.cuda.empty_cache()
        rinp, _, rr = measure(args, ref_wl, "fp32", "auto", dev)
        rms, rmed = time_dropin("iso", rinp, args.steps, args.warmup, stream)
        del rr["call"]
        torch.cuda.empty_cache()
        _, _, rd = measure(args, ref_wl, "fp32", False, dev, inp=rinp)
        out["reference_smoke_workload"] = {
            "workload": ref_wl, "N": N, "K": K, "D": D, "value": N / (rms * 1e-3), "unit": "samples/s",
            "ms_per_step": rms, "median_call_ms": rmed, "phase1_ms": rr["p1"], "phase2_ms": rr["p2"],
            "plan": "the drop-in call (store_log_joint='auto': the probe selects the stored branch here)",
            "default_plan": {"ms_per_step": rd["ms"], "phase1_ms": rd["p1"], "phase2_ms": rd["p2"],
                             "note": "the O(N + K*D) plan on the same data (pass 2 recomputes the "
                                     "contraction for every pair)"},
            "vs_baseline": (N / (rms * 1e-3)) / A100_SAMPLES_PER_S,
            "data": "X, mu ~ N(0, I), lss = 0, log pi = -log K (flash_gmm.py:228-234), generated on device"}
        log(f"reference smoke workload: {rms:.3f} ms/step (phase1 {rr['p1']:.3f}, phase2 {rr['p2']:.3f}); "
            f"default plan {rd['ms']:.3f} ms")
        del rinp, rr, rd
        torch.cuda.empty_cache()
        # The same dense regime for the diagonal and full models at their benchmark
        # shapes: the drop-in call (the probe selects the stored branch) beside the
        # default plan, whose pass 2 recomputes every pair.
        dense = {}
        for dwl in ("diag_ref_n1m_k1024_d96", "full_ref_n250k_k256_d64"):
            dN, dK, dD = WORKLOADS[dwl]
            dkind = dwl.split("_")[0]
            dinp, _, da = measure(args, dwl, "fp32", "auto", dev)
            dms, dmed = time_dropin(dkind, dinp, args.steps, args.warmup, stream)
            del da["call"]
            torch.cuda.empty_cache()
            _, _, dd = measure(args, dwl, "fp32", False, dev, inp=dinp)
            del dd["call"]
            dense[dwl] = {"N": dN, "K": dK, "D": dD, "ms_per_step": dms, "median_call_ms": dmed,
                          "value": dN / (dms * 1e-3), "unit": "samples/s",
                          "phase1_ms": da["p1"], "phase2_ms": da["p2"],
                          "plan": "the drop-in call (store_log_joint='auto': the probe selects the stored "
                                  "branch here)",
                          "default_plan": {"ms_per_step": dd["ms"], "phase1_ms": dd["p1"], "phase2_ms": dd["p2"]}}
            log(f"{dwl}: drop-in {dms:.3f} ms/step (phase1 {da['p1']:.3f}, phase2 {da['p2']:.3f}); "
                f"default plan {dd['ms']:.3f} ms (phase2 {dd['p2']:.3f})")
            del dinp, da, dd
            torch.cuda.empty_cache()
        out["dense_regime_diag_full"] = dense
    if not args.no_cpu_baseline and not bf16:
        log("timing the CPU baseline (bounded sample)")
        out["cpu_baseline"] = cpu_baseline(inp, kind, K, D, logZ)
    print(json.dumps(out), flush=True)


def sweep_main(args):
    """One JSON line per D: default plan, stored log-joint and dense, ms per step."""
    import torch
    from flash_gmm import data

    kind, N, K, Ds = args.sweep.split(":")
    N, K = int(N), int(K)
    dev = torch.device("cuda:0")
    gen = {"iso": data.iso_clustered, "diag": data.diag_clustered, "full": data.full_clustered}[kind]
    stream = torch.cuda.current_stream(dev)
    for D in (int(d) for d in Ds.split(",")):
        inp = gen(N, K, D, seed=1, device=dev)
        res = {"sweep": kind, "N": N, "K": K, "D": D}
        for name, store in (("default", False), ("stored", True)):
            call, ws, _ = make_runner(kind, inp, N, K, D, dev, "fp32", store)
            ms, p1, p2 = time_steps(call, args.steps, 3, stream)
            res[name] = {"ms": round(ms, 3), "phase1_ms": round(p1, 3), "phase2_ms": round(p2, 3),
                         "workspace_MB": round(ws / 2**20, 1)}
            if name == "default":
                dms, _, _ = time_steps(call, args.steps, 2, stream, dense=True)
                res["default"]["dense_ms"] = round(dms, 3)
            del call
            torch.cuda.empty_cache()
        print(json.dumps(res), flush=True)
        del inp
        torch.cuda.empty_cache()


def reduce_compare_main(args):
    """Deterministic fixed-order tree against float atomics for the finish, per workload."""
    import torch
    from flash_gmm import data

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    for workload in ("iso_n1m_k1024_d128", "diag_n1m_k1024_d96", "full_n250k_k256_d64"):
        N, K, D = WORKLOADS[workload]
        kind = workload.split("_")[0]
        inp = data.make(workload, device=dev)
        res = {"reduce_compare": workload}
        for name, atomic in (("tree", False), ("atomic", True)):
            call, _, _ = make_runner(kind, inp, N, K, D, dev, "fp32", False, atomic)
            ms, p1, p2 = time_steps(call, args.steps, 3, stream)
            res[name] = {"ms": round(ms, 4), "phase2_ms": round(p2, 4)}
            del call
            torch.cuda.empty_cache()
        print(json.dumps(res), flush=True)
        del inp
        torch.cuda.empty_cache()


def stream_main(args):
    """Streaming EM over host-generated rows (pinned double buffers, copy/compute overlap)."""
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
    threads = len(os.sched_getaffinity(0))
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
    ap.add_argument("--no-extra-runs", action="store_true",
                    help="time only the selected plan (no dense and stored-log-joint runs)")
    ap.add_argument("--workload", default="iso_n1m_k1024_d128",
                    choices=sorted(WORKLOADS) + ["stream_em_n1b_k1024_d128"])
    ap.add_argument("--rows", type=int, default=0, help="override N of the streaming workload")
    ap.add_argument("--precision", choices=["fp32", "bf16"], default="fp32",
                    help="bf16 runs the H100 variants' bf16 operand contract (FGMM_FLAG_BF16)")
    ap.add_argument("--store-log-joint", action="store_true",
                    help="time the opt-in plan that stores the N x K log-joint (FGMM_FLAG_STORE_LOGJOINT)")
    ap.add_argument("--sweep", default="", metavar="KIND:N:K:D1,D2,...",
                    help="time the default, stored and dense plans over several D")
    ap.add_argument("--reduce-compare", action="store_true",
                    help="time the fixed-order tree finish against float atomics at the benchmark shapes")
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
    elif args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 4
        a = torch.ones(n, device="cuda:0")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4, "launches": 5}), flush=True)
    elif args.sweep:
        sweep_main(args)
    elif args.reduce_compare:
        reduce_compare_main(args)
    else:
        main_workload(args)


if __name__ == "__main__":
    main()

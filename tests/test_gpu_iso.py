"""GPU parity of the isotropic E-step against the CPU oracle (tolerances in parity.py)."""

import math
import os
import sys

import numpy as np
import pytest
import torch

from flash_gmm import FlashGMMError, data, flash_gmm_estep, iso_estep_into
from oracle import gmm_oracle as O

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden  # noqa: E402
from parity import LOGZ_ATOL, assert_close_stats, assert_dense_agrees, logz_atol_fp32, logz_err  # noqa: E402

pytestmark = pytest.mark.gpu

def run_gpu(inp, dev, **kw):
    args = [inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    out = flash_gmm_estep(*args, **kw)
    torch.cuda.synchronize()
    return out


def oracle(inp, dtype=torch.float64):
    return O.estep_iso(inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"], dtype=dtype)


def check_wide(got, inp, what, D, ref=None):
    """All four outputs against the float64 oracle.  The logZ bound is 1e-4 up to
    D = 128; above, max(1e-4, the error of the float32 restatement of the reference's
    arithmetic on the same rows), measured here."""
    ref = oracle(inp) if ref is None else ref
    atol = logz_atol_fp32(oracle(inp, torch.float32)[0] if D > 128 else None, ref[0], D)
    print(f"{what}: max |logZ - oracle| {logz_err(got[0], ref[0]):.2e}, bound {atol:.2e}", flush=True)
    assert_close_stats(got, ref, what, logz_atol=atol)


@pytest.mark.parametrize("name", ["iso_n10k_k64_d32", "iso_clustered_n4096_k96_d40"])
def test_golden_vectors(name, gpu_device):
    inp, kind = make_golden.make_inputs(name)
    fx = np.load(os.path.join(os.path.dirname(make_golden.__file__), name + ".npz"))
    assert str(fx["sha256"]) == make_golden.input_digest(inp), "input generator changed"
    got = run_gpu(inp, gpu_device)
    assert_close_stats(got, (fx["logZ"], fx["Nk"], fx["mu_acc"], fx["sig"]), name)


SHAPES = [
    # (N, K, D)
    (1, 1, 1), (31, 3, 5), (33, 17, 3), (129, 33, 32), (1000, 100, 96), (257, 64, 100),
    (300, 40, 128), (200, 32, 129), (150, 7, 256), (2048, 1, 64), (4097, 70, 64),
    (3000, 150, 160), (2500, 260, 192), (1800, 130, 250),
]


@pytest.mark.parametrize("N,K,D", SHAPES)
def test_edge_shapes(N, K, D, gpu_device):
    inp = data.iso_clustered(N, K, D, seed=N + K + D)
    check_wide(run_gpu(inp, gpu_device), inp, f"N={N} K={K} D={D}", D)


def test_empty_rows(gpu_device):
    inp = data.iso_plain(0, 8, 16, seed=3)
    lz, nk, mu_acc, sig = run_gpu(inp, gpu_device)
    assert lz.shape == (0,)
    assert torch.all(nk == 0) and torch.all(mu_acc == 0) and torch.all(sig == 0)


def test_no_components(gpu_device):
    inp = data.iso_plain(40, 1, 8, seed=4)
    inp["mu"] = inp["mu"][:0]
    inp["log_sigma_sq"] = inp["log_sigma_sq"][:0]
    inp["log_pi"] = inp["log_pi"][:0]
    lz, nk, mu_acc, sig = run_gpu(inp, gpu_device)
    assert torch.all(torch.isneginf(lz)) and nk.numel() == 0 and mu_acc.shape == (0, 8)


def test_zero_weight_components(gpu_device):
    inp = data.iso_clustered(500, 20, 24, seed=5)
    inp["log_pi"][[0, 3, 19]] = -math.inf
    got = run_gpu(inp, gpu_device)
    assert_close_stats(got, oracle(inp), "lpi=-inf")
    assert float(got[1][0]) == 0.0 and float(got[1][19]) == 0.0


def test_strided_inputs(gpu_device):
    inp = data.iso_clustered(700, 30, 40, seed=6)
    ref = oracle(inp)
    big = torch.zeros(700, 57, device=gpu_device)
    big[:, 3:43] = inp["X"].to(gpu_device)
    Xv = big[:, 3:43]                                        # row stride 57, misaligned
    Xt = inp["X"].to(gpu_device).t().contiguous().t()       # column-major
    mu_t = inp["mu"].to(gpu_device).t().contiguous().t()
    for X in (Xv, Xt):
        got = flash_gmm_estep(X, mu_t, inp["log_sigma_sq"].to(gpu_device), inp["log_pi"].to(gpu_device))
        torch.cuda.synchronize()
        assert_close_stats(got, ref, "strided")


@pytest.mark.parametrize("dtype", [torch.float64, torch.bfloat16, torch.float16])
def test_other_float_dtypes_compute_in_float32(dtype, gpu_device):
    """Non-float32 X / mu are converted (the reference assumes float32 inputs)."""
    inp = data.iso_clustered(3000, 40, 24, seed=13)
    dev = gpu_device
    X, mu, lss, lpi = (inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    Xd, mud = X.to(dtype), mu.to(dtype)
    got = flash_gmm_estep(Xd, mud, lss, lpi)
    ref = flash_gmm_estep(Xd.float(), mud.float(), lss, lpi)
    torch.cuda.synchronize()
    for u, v in zip(got, ref):
        assert u.dtype == torch.float32 and torch.equal(u, v)


def test_block_kwargs_are_accepted(gpu_device):
    inp = data.iso_plain(100, 8, 16, seed=7)
    a = run_gpu(inp, gpu_device)
    b = run_gpu(inp, gpu_device, BLOCK_N=128, BLOCK_K=32, BLOCK_D=16)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_deterministic_bitwise(gpu_device):
    inp = data.iso_clustered(20000, 256, 64, seed=8)
    a = run_gpu(inp, gpu_device)
    b = run_gpu(inp, gpu_device)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def _into(inp, dev, **kw):
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, device=dev)]
    iso_estep_into(*[inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")], *out, **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("case", ["clustered_d128", "clustered_d64_ragged", "plain_d32", "clustered_d256"])
def test_zero_step_skip_is_bitwise_dense(case, stored, gpu_device):
    """Skipping all-zero responsibility steps (and, on the default plan, the rows whose
    need bit is clear) changes no bit of any output."""
    if case == "clustered_d128":
        inp = data.iso_clustered(12000, 1024, 128, seed=1)   # mostly zero steps
    elif case == "clustered_d64_ragged":
        inp = data.iso_clustered(7777, 300, 61, seed=5)
    elif case == "clustered_d256":
        inp = data.iso_clustered(6000, 512, 256, seed=6)   # component-tiled pass 1, range pass 2
    else:
        inp = data.iso_plain(10000, 64, 32, seed=0)          # no zero steps
    a = _into(inp, gpu_device, store_log_joint=stored)
    b = _into(inp, gpu_device, dense=True, store_log_joint=stored)
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    from flash_gmm import _lib
    L = _lib.lib()
    applies = stored and L.fgmm_iso_workspace_bytes_ex(N, K, D, _lib.FLAG_STORE_LOGJOINT) != \
        L.fgmm_iso_workspace_bytes(N, K, D)
    # Up to D = 128 the stored plan's sparse masks take iso_accum_sparse (fp32 pair
    # products) and the dense run iso_accum_ljt (split-bf16 tiles): the same terms,
    # other roundings.
    assert_dense_agrees(a, b, bitwise=applies and D > 128)
    check_wide(a, inp, case, D)
    check_wide(b, inp, case + " dense", D)


# Clustered shapes whose need masks are sparse (K >= 512): the accumulation pass
# takes its sparse form (register-row pairs fetched per tile, with the overflow path
# for tiles of more than three pairs at K=512), which must give the dense pass's bits.
SPARSE_SHAPES = [(20000, 1024, 64), (20000, 512, 96), (40000, 512, 128), (30001, 1024, 128)]


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("N,K,D", SPARSE_SHAPES)
def test_sparse_accumulation_is_bitwise_dense(N, K, D, stored, gpu_device):
    """Sparse accumulation against the dense one (FGMM_FLAG_DENSE) and the oracle, on the
    default plan (gathered rows) and the stored log-joint (iso_accum_sparse's fp32 pair
    products against iso_accum_ljt's split-bf16 tiles): logZ bitwise, the statistics
    to 1e-5 of each output's largest magnitude."""
    inp = data.iso_clustered(N, K, D, seed=N % 101)
    a = _into(inp, gpu_device, store_log_joint=stored)
    b = _into(inp, gpu_device, dense=True, store_log_joint=stored)
    assert_dense_agrees(a, b, bitwise=False)
    assert_close_stats(a, oracle(inp), f"sparse N={N} K={K} D={D}")


# Shapes on the stored log-joint path (D > 32 and K > 96), including row counts
# that leave partial 32-row tiles and slabs, and both column splits of pass 2.
LJ_SHAPES = [(33, 128, 128), (65, 257, 96), (1000, 130, 64), (777, 300, 61), (4097, 129, 100),
             (2500, 260, 192), (1800, 300, 250), (9001, 512, 128), (3000, 150, 160), (700, 200, 256)]


@pytest.mark.parametrize("N,K,D", LJ_SHAPES)
def test_stored_and_recomputed_log_joint(N, K, D, gpu_device):
    """Pass 2 from the log-joint stored by pass 1, and recomputed, both against the oracle."""
    from flash_gmm import _lib
    L = _lib.lib()
    # The two plans differ (stored tiles, pass-2 work split), so these shapes take the stored path.
    assert L.fgmm_iso_workspace_bytes(N, K, D) != L.fgmm_iso_workspace_bytes_ex(N, K, D, _lib.FLAG_STORE_LOGJOINT)
    inp = data.iso_clustered(N, K, D, seed=N + 3 * K + D)
    ref = oracle(inp)
    stored = _into(inp, gpu_device, store_log_joint=True)
    recomputed = _into(inp, gpu_device)
    assert torch.equal(stored[0], recomputed[0])          # pass 1 is the same kernel math
    check_wide(stored, inp, f"stored N={N} K={K} D={D}", D, ref=ref)
    check_wide(recomputed, inp, f"recomputed N={N} K={K} D={D}", D, ref=ref)


def test_stored_log_joint_zero_weight_components(gpu_device):
    """log_pi = -inf components on the stored path: r = 0 and finite sig_acc."""
    inp = data.iso_clustered(3000, 200, 48, seed=15)
    inp["log_pi"][[0, 7, 199]] = -math.inf
    got = _into(inp, gpu_device, store_log_joint=True)
    assert_close_stats(got, oracle(inp), "stored lpi=-inf")
    assert float(got[1][0]) == 0.0 and float(got[3][199]) == 0.0
    assert torch.isfinite(got[3]).all()


@pytest.mark.parametrize("stored", [False, True])
def test_phase_split_equals_one_call(stored, gpu_device):
    """PHASE1 then PHASE2 on one workspace gives the single call's outputs bitwise."""
    inp = data.iso_clustered(5000, 256, 96, seed=16)
    dev = gpu_device
    ref = _into(inp, dev, store_log_joint=stored)
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    from flash_gmm import _lib
    L = _lib.lib()
    flags = _lib.FLAG_STORE_LOGJOINT if stored else 0
    ws = torch.empty(L.fgmm_iso_workspace_bytes_ex(N, K, D, flags), dtype=torch.uint8, device=dev)
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, device=dev)]
    args = [inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    iso_estep_into(*args, *out, workspace=ws, phase=1, store_log_joint=stored)
    iso_estep_into(*args, None, *out[1:], workspace=ws, phase=2, store_log_joint=stored)
    torch.cuda.synchronize()
    for u, v in zip(out, ref):
        assert torch.equal(u, v)


def test_atomic_reduce_matches(gpu_device):
    inp = data.iso_clustered(5000, 200, 48, seed=9)
    ref = run_gpu(inp, gpu_device)
    dev = gpu_device
    K, D = 200, 48
    out = [torch.empty(5000, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, device=dev)]
    args = [inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    iso_estep_into(*args, *out, atomic_reduce=True)
    torch.cuda.synchronize()
    assert torch.equal(out[0], ref[0])
    for u, v in zip(out[1:], ref[1:]):
        torch.testing.assert_close(u, v, rtol=1e-5, atol=1e-5 * float(v.abs().max()))


def test_accumulate_over_chunks_equals_one_call(gpu_device):
    inp = data.iso_clustered(9000, 128, 64, seed=10)
    dev = gpu_device
    args = [inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    ref = flash_gmm_estep(*args)
    K, D = 128, 64
    nk = torch.zeros(K, device=dev)
    mu_acc = torch.zeros(K, D, device=dev)
    sig = torch.zeros(K, device=dev)
    for n0 in range(0, 9000, 2500):
        iso_estep_into(args[0][n0:n0 + 2500], *args[1:], None, nk, mu_acc, sig, accumulate=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(nk, ref[1], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(mu_acc, ref[2], rtol=1e-5, atol=1e-5 * float(ref[2].abs().max()))
    torch.testing.assert_close(sig, ref[3], rtol=1e-5, atol=1e-4)


def test_auto_store_accumulate_over_chunks(gpu_device):
    """FGMM_FLAG_ACCUMULATE with the stored branch selected (dense data): three row
    chunks added into the outputs equal one call over all rows (to float32 rounding)."""
    inp = data.reference_smoke(9000, 256, 128, seed=10)
    dev = gpu_device
    args = [inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    ref = _into(inp, dev, store_log_joint="auto")
    K, D = 256, 128
    nk, mu_acc, sig = torch.zeros(K, device=dev), torch.zeros(K, D, device=dev), torch.zeros(K, device=dev)
    for n0 in range(0, 9000, 3000):
        iso_estep_into(args[0][n0:n0 + 3000], *args[1:], None, nk, mu_acc, sig, accumulate=True,
                       store_log_joint="auto")
    torch.cuda.synchronize()
    torch.testing.assert_close(nk, ref[1], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(mu_acc, ref[2], rtol=1e-5, atol=1e-5 * float(ref[2].abs().max()))
    torch.testing.assert_close(sig, ref[3], rtol=1e-5, atol=1e-5 * float(ref[3].abs().max()))


def test_headline_shape_mid_size(gpu_device):
    """K=1024, D=128 clustered data at N=65,536 against the float64 oracle."""
    inp = data.iso_clustered(65536, 1024, 128, seed=1)
    assert_close_stats(run_gpu(inp, gpu_device), oracle(inp), "K1024 D128 N65536")


@pytest.mark.parametrize("kind", ["clustered", "dense"])
def test_pass1_tail_groups(kind, gpu_device):
    """Pass 1 (D <= 128) runs whole rounds of 8-tile workgroups, one per compute unit,
    then the tiles left in smaller groups whose spare waves only load and meet the
    barriers.  At an N that leaves 531 tiles after one round (groups of 3, the last
    tile partial): all four outputs against the oracle, the default plan against
    dense=True, and store_log_joint='auto' (on the dense data the stored branch, which
    reads the log-joint tiles, X parts and logZ pairs pass 1 wrote)."""
    cus = torch.cuda.get_device_properties(gpu_device).multi_processor_count
    N = 8 * cus * 32 + 530 * 32 + 17
    print(f"tail groups {kind} N={N} CUs={cus}", flush=True)
    inp = (data.iso_clustered(N, 256, 128, seed=5) if kind == "clustered"
           else data.reference_smoke(N, 256, 128, seed=5))
    ref = oracle(inp)
    base = _into(inp, gpu_device)
    assert_close_stats(base, ref, f"tail groups {kind} N={N}")
    auto = _into(inp, gpu_device, store_log_joint="auto")
    assert torch.equal(auto[0], base[0])
    assert_close_stats(auto, ref, f"tail groups auto {kind} N={N}")
    dense = _into(inp, gpu_device, dense=True)
    assert_dense_agrees(base, dense, bitwise=False)


@pytest.mark.parametrize("N,K,D", [(50_000, 48, 64), (30_000, 20, 30), (40_000, 64, 96)])
def test_small_k_mid_size(N, K, D, gpu_device):
    """Few component blocks: pass 2 runs 1 or 2 blocks per workgroup with more row groups."""
    inp = data.iso_clustered(N, K, D, seed=N % 97)
    got = run_gpu(inp, gpu_device)
    assert_close_stats(got, oracle(inp), f"small K N={N} K={K} D={D}")
    dev = gpu_device
    dense = _into(inp, dev, dense=True)
    assert_dense_agrees(got, dense, bitwise=False)


def test_wide_shape_mid_size(gpu_device):
    """D=256 (component-tiled pass 1, dimension-range pass 2) at N=16,384, K=512 against
    the float64 oracle."""
    inp = data.iso_clustered(16384, 512, 256, seed=7)
    check_wide(run_gpu(inp, gpu_device), inp, "K512 D256 N16384", 256)


def test_phase2_requires_the_phase1_workspace(gpu_device):
    inp = data.iso_clustered(300, 64, 32, seed=17)
    dev = gpu_device
    args = [inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    out = [torch.empty(64, device=dev), torch.empty(64, 32, device=dev), torch.empty(64, device=dev)]
    with pytest.raises(FlashGMMError):
        iso_estep_into(*args, None, *out, phase=2)
    with pytest.raises(FlashGMMError):
        iso_estep_into(*args, None, *out, phase=2, workspace=torch.empty(16, dtype=torch.uint8, device=dev))


def test_stored_plan_falls_back_when_its_workspace_cannot_be_allocated(gpu_device, monkeypatch):
    """store_log_joint=True whose O(N*K) workspace fails to allocate runs the default plan."""
    from flash_gmm import _lib, estep
    inp = data.iso_clustered(4000, 256, 64, seed=18)
    dev = gpu_device
    ref = _into(inp, dev)
    L = _lib.lib()
    lean = L.fgmm_iso_workspace_bytes(4000, 256, 64)
    real = estep._empty_workspace

    def small_only(nbytes, device):
        if nbytes > lean:
            raise torch.cuda.OutOfMemoryError("simulated")
        return real(nbytes, device)

    monkeypatch.setattr(estep, "_empty_workspace", small_only)
    got = _into(inp, dev, store_log_joint=True)
    for u, v in zip(got, ref):
        assert torch.equal(u, v)


@pytest.mark.parametrize("N,K,D", [(3000, 2100, 128), (2000, 6200, 64), (1500, 9000, 32)])
def test_need_masks_from_the_running_max(N, K, D, gpu_device):
    """More component blocks than pass 1 keeps maxima for in LDS: the need masks come
    from the running-max bound instead; results against the dense pass and the oracle."""
    inp = data.iso_clustered(N, K, D, seed=K % 89)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device, dense=True)
    assert_dense_agrees(a, b, bitwise=False)
    assert_close_stats(a, oracle(inp), f"running-max masks N={N} K={K} D={D}")


def _full_size_against_oracle(inp, dev, what):
    got = flash_gmm_estep(inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"])
    torch.cuda.synchronize()
    logZ, Nk, mu_acc, sig = got
    N = inp["X"].shape[0]
    assert abs(Nk.double().sum().item() - N) <= 1e-5 * N
    xs = inp["X"].double().sum(0)
    torch.testing.assert_close(mu_acc.double().sum(0), xs, rtol=0, atol=1e-5 * float(mu_acc.abs().sum(0).max()))
    assert torch.all(sig >= 0)
    print(f"{what}: full-size oracle (float64, CPU)", flush=True)
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    ref = O.estep_iso(*[inp[k].cpu() for k in ("X", "mu", "log_sigma_sq", "log_pi")])
    print(f"{what}: max |logZ - oracle| = {(logZ.cpu().double() - ref[0]).abs().max().item():.3e}", flush=True)
    assert_close_stats(got, ref, what)
    return got


def test_reference_smoke_workload_full_size(gpu_device):
    """The reference's own benchmark workload (flash_gmm.py:228-234: X ~ N(0, I),
    mu ~ N(0, I), lss = 0, uniform log pi; N=1M, K=1024, D=128), where nearly every
    responsibility is nonzero, against the float64 oracle over every row."""
    inp = data.reference_smoke(1_000_000, 1024, 128, seed=0, device=gpu_device)
    _full_size_against_oracle(inp, gpu_device, "reference smoke N=1M")


def test_headline_shape_second_seed(gpu_device):
    """The headline shape on another seed: the logZ margin is not one seed's luck."""
    inp = data.iso_clustered(1_000_000, 1024, 128, seed=2, device=gpu_device)
    _full_size_against_oracle(inp, gpu_device, "K1024 D128 N=1M seed 2")


def test_headline_shape_full_size_against_oracle(gpu_device):
    """N=1M, K=1024, D=128 (the benchmark workload): size-independent properties, and
    all four outputs against the float64 oracle over every row (about 15 s of CPU)."""
    dev = gpu_device
    inp = data.iso_clustered(1_000_000, 1024, 128, seed=1, device=dev)
    stored = _into(inp, dev, store_log_joint=True)
    got = flash_gmm_estep(inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"])
    torch.cuda.synchronize()
    logZ, Nk, mu_acc, sig = got
    N = inp["X"].shape[0]
    assert abs(Nk.double().sum().item() - N) <= 1e-5 * N
    xs = inp["X"].double().sum(0)
    torch.testing.assert_close(mu_acc.double().sum(0), xs, rtol=0, atol=1e-5 * float(mu_acc.abs().sum(0).max()))
    assert torch.all(sig >= 0)
    # The gathered accumulation agrees with the dense one, and pass 1 with the stored plan's.
    dense = _into(inp, dev, dense=True)
    assert_dense_agrees(got, dense, bitwise=False)
    assert torch.equal(stored[0], got[0])
    print("full-size oracle (float64, CPU)", flush=True)
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    ref = O.estep_iso(*[inp[k].cpu() for k in ("X", "mu", "log_sigma_sq", "log_pi")])
    print(f"N=1M max |logZ - oracle| = {(logZ.cpu().double() - ref[0]).abs().max().item():.3e}", flush=True)
    assert_close_stats(got, ref, "K1024 D128 N=1M")


def test_wide_row_stride(gpu_device):
    """A row stride of X above 2^20 floats, past the stored path's 32-bit buffer offsets:
    the call recomputes instead, with results to the same bar."""
    inp = data.iso_clustered(200, 128, 64, seed=21)
    big = torch.zeros(200, (1 << 20) + 64, device=gpu_device)
    big[:, :64] = inp["X"].to(gpu_device)
    got = flash_gmm_estep(big[:, :64], *[inp[k].to(gpu_device) for k in ("mu", "log_sigma_sq", "log_pi")])
    torch.cuda.synchronize()
    assert_close_stats(got, oracle(inp), "iso wide row stride")


def test_rejects_bad_shapes(gpu_device):
    inp = data.iso_plain(10, 4, 8, seed=11)
    X, mu, lss, lpi = (inp[k].to(gpu_device) for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    with pytest.raises(AssertionError):
        flash_gmm_estep(X, mu[:, :4], lss, lpi)
    with pytest.raises(FlashGMMError):
        flash_gmm_estep(X, mu, lss[:2], lpi)
    with pytest.raises(FlashGMMError):   # not floating point
        flash_gmm_estep(X.int(), mu, lss, lpi)


# FGMM_FLAG_STORE_LOGJOINT_AUTO (store_log_joint="auto"): the device-selected stored
# branch on dense data, the default plan elsewhere.
AUTO_DENSE_SHAPES = [(20000, 256, 128), (9000, 300, 96), (5000, 130, 61), (3000, 64, 32), (777, 40, 100)]


@pytest.mark.parametrize("N,K,D", AUTO_DENSE_SHAPES)
def test_auto_store_dense_takes_stored_branch(N, K, D, gpu_device):
    """On the reference's dense data (X, mu ~ N(0, I)) the probe selects the stored
    branch: the statistics come from iso_accum_ljt, whose roundings differ from the
    default plan's in the last bits, and agree with the oracle; logZ is pass 1's,
    bitwise the default plan's."""
    inp = data.reference_smoke(N, K, D, seed=N % 97)
    auto = _into(inp, gpu_device, store_log_joint="auto")
    base = _into(inp, gpu_device)
    assert torch.equal(auto[0], base[0])
    assert any(not torch.equal(u, v) for u, v in zip(auto[1:], base[1:]))
    check_wide(auto, inp, f"auto dense N={N} K={K} D={D}", D)


@pytest.mark.parametrize("N,K,D", [(20000, 1024, 128), (9000, 300, 96), (5000, 512, 64), (4000, 512, 100)])
def test_auto_store_clustered_is_the_default_plan(N, K, D, gpu_device):
    """On clustered data with many components (few pairs needed) the probe keeps the
    default plan: every output bitwise equal to a call without the flag.  (With a
    few blocks or few dimensions, as at K = 512, D = 33, most (row, block) pairs can
    be needed and the stored branch is the probe's choice.)"""
    inp = data.iso_clustered(N, K, D, seed=K % 13)
    auto = _into(inp, gpu_device, store_log_joint="auto")
    base = _into(inp, gpu_device)
    for u, v in zip(auto, base):
        assert torch.equal(u, v)


@pytest.mark.parametrize("kind", ["dense", "clustered"])
def test_auto_store_phase_split_and_reuse(kind, gpu_device):
    """PHASE1 then PHASE2 on one workspace equals the single call bitwise, and calls
    alternating between dense and clustered data on that workspace each select their
    own branch (the probe's counters start from zero every call)."""
    from flash_gmm import _lib
    L = _lib.lib()
    dev = gpu_device
    dense_inp = data.reference_smoke(6000, 256, 96, seed=4)
    clus_inp = data.iso_clustered(6000, 256, 96, seed=5)
    inp = dense_inp if kind == "dense" else clus_inp
    other = clus_inp if kind == "dense" else dense_inp
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    ws = torch.empty(L.fgmm_iso_workspace_bytes_ex(N, K, D, _lib.FLAG_STORE_LOGJOINT_AUTO), dtype=torch.uint8,
                     device=dev)
    ref = _into(inp, dev, store_log_joint="auto")
    ref_other = _into(other, dev, store_log_joint="auto")
    for _ in range(2):
        for cur, want in ((inp, ref), (other, ref_other)):
            out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
                   torch.empty(K, device=dev)]
            args = [cur[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
            iso_estep_into(*args, *out, workspace=ws, phase=1, store_log_joint="auto")
            iso_estep_into(*args, None, *out[1:], workspace=ws, phase=2, store_log_joint="auto")
            torch.cuda.synchronize()
            for u, v in zip(out, want):
                assert torch.equal(u, v)

"""GPU parity of the diagonal-covariance E-step against the CPU oracle (tolerances in parity.py)."""

import os
import sys

import numpy as np
import pytest
import torch

from flash_gmm import data, diag_estep_into, flash_gmm_estep, flash_gmm_estep_diag
from oracle import gmm_oracle as O

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden  # noqa: E402
from parity import LOGZ_ATOL, assert_close_stats, assert_dense_agrees, logz_atol_fp32, logz_err  # noqa: E402

pytestmark = pytest.mark.gpu


def run_gpu(inp, dev):
    out = flash_gmm_estep_diag(*[inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")])
    torch.cuda.synchronize()
    return out


def oracle(inp, dtype=torch.float64):
    return O.estep_diag(inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"], dtype=dtype)


def check_wide(got, inp, what, D, ref=None):
    """All four outputs against the float64 oracle.  The logZ bound is 1e-4 up to
    D = 128; above, max(1e-4, the error of the float32 restatement of the reference's
    arithmetic on the same rows), measured here."""
    ref = oracle(inp) if ref is None else ref
    atol = logz_atol_fp32(oracle(inp, torch.float32)[0] if D > 128 else None, ref[0], D)
    print(f"{what}: max |logZ - oracle| {logz_err(got[0], ref[0]):.2e}, bound {atol:.2e}", flush=True)
    assert_close_stats(got, ref, what, logz_atol=atol)


def test_golden_vectors(gpu_device):
    name = "diag_n3000_k40_d24"
    inp, kind = make_golden.make_inputs(name)
    fx = np.load(os.path.join(os.path.dirname(make_golden.__file__), name + ".npz"))
    assert str(fx["sha256"]) == make_golden.input_digest(inp)
    assert_close_stats(run_gpu(inp, gpu_device), (fx["logZ"], fx["Nk"], fx["mu_acc"], fx["sig"]), name)


@pytest.mark.parametrize("N,K,D", [(1, 1, 1), (33, 5, 3), (500, 40, 24), (1000, 70, 96),
                                   (300, 33, 128), (129, 3, 64), (2000, 130, 50),
                                   (700, 37, 129), (1500, 70, 192), (900, 65, 200), (800, 97, 256),
                                   (5, 2, 255)])
def test_edge_shapes(N, K, D, gpu_device):
    inp = data.diag_clustered(N, K, D, seed=N + K + D)
    check_wide(run_gpu(inp, gpu_device), inp, f"diag N={N} K={K} D={D}", D)


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("N,K,D,seed", [(9000, 512, 96, 2), (3001, 77, 45, 3), (4000, 130, 256, 4),
                                        (5000, 300, 128, 6)])
def test_zero_step_skip_is_bitwise_dense(N, K, D, seed, stored, gpu_device):
    """Skipping all-zero responsibility steps changes no bit of any output."""
    inp = data.diag_clustered(N, K, D, seed=seed)
    dev = gpu_device
    args = [inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    outs = []
    for dense in (False, True):
        o = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
             torch.empty(K, D, device=dev)]
        diag_estep_into(*args, *o, dense=dense, store_log_joint=stored)
        outs.append(o)
    torch.cuda.synchronize()
    assert_dense_agrees(outs[0], outs[1], bitwise=_stored_applies(N, K, D, stored))
    check_wide(outs[0], inp, "diag skip", D)
    check_wide(outs[1], inp, "diag dense", D)


@pytest.mark.parametrize("N,K,D", [(40_000, 30, 16), (30_000, 60, 40), (20_000, 50, 96)])
def test_small_k_mid_size(N, K, D, gpu_device):
    """Few component blocks: pass 2 runs 1 or 2 blocks per workgroup with more row groups."""
    inp = data.diag_clustered(N, K, D, seed=N % 89)
    assert_close_stats(run_gpu(inp, gpu_device), oracle(inp), f"diag small K N={N} K={K} D={D}")


def _stored_applies(N, K, D, stored):
    """Whether store_log_joint=True takes the stored plan here (it needs K > 96)."""
    from flash_gmm import _lib
    L = _lib.lib()
    return stored and L.fgmm_diag_workspace_bytes_ex(N, K, D, _lib.FLAG_STORE_LOGJOINT) != \
        L.fgmm_diag_workspace_bytes(N, K, D)


def _into(inp, dev, **kw):
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, device=dev)]
    diag_estep_into(*[inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")], *out, **kw)
    torch.cuda.synchronize()
    return out


# Shapes on the stored log-joint path (K > 96), with partial tiles and slabs, every
# padded width and both column splits of pass 2 (8 or 4 blocks per workgroup).
LJ_SHAPES = [(33, 128, 40), (65, 257, 96), (1000, 130, 64), (777, 300, 61), (4097, 129, 100),
             (2500, 260, 192), (1800, 300, 250), (9001, 512, 128), (3000, 150, 128), (700, 200, 256)]


@pytest.mark.parametrize("N,K,D", LJ_SHAPES)
def test_stored_and_recomputed_log_joint(N, K, D, gpu_device):
    """Pass 2 from the log-joint stored by pass 1, and recomputed, both against the oracle."""
    from flash_gmm import _lib
    L = _lib.lib()
    # The two plans differ (stored tiles, pass-2 work split), so these shapes take the stored path.
    assert L.fgmm_diag_workspace_bytes(N, K, D) != L.fgmm_diag_workspace_bytes_ex(N, K, D, _lib.FLAG_STORE_LOGJOINT)
    inp = data.diag_clustered(N, K, D, seed=N + 3 * K + D)
    ref = oracle(inp)
    stored = _into(inp, gpu_device, store_log_joint=True)
    recomputed = _into(inp, gpu_device)
    assert torch.equal(stored[0], recomputed[0])
    check_wide(stored, inp, f"stored N={N} K={K} D={D}", D, ref=ref)
    check_wide(recomputed, inp, f"recomputed N={N} K={K} D={D}", D, ref=ref)


# Shapes of the sparse stored log-joint (32 < D <= 128): sparse masks (D = 64 .. 128)
# and widths that are not a multiple of 32 (mask-driven dense kernel only).  Each
# half block of a row is stored by its own pass-1 wave, so a row may hold one
# stored and one left-out half.
SPARSE_SHAPES = [(20000, 1024, 64), (20000, 512, 96), (40000, 512, 128), (30001, 1024, 96),
                 (20000, 300, 40), (20000, 512, 90)]


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("N,K,D", SPARSE_SHAPES)
def test_sparse_accumulation_is_bitwise_dense(N, K, D, stored, gpu_device):
    """Accumulation (default plan, and from the sparse stored log-joint) against
    FGMM_FLAG_DENSE and the oracle."""
    inp = data.diag_clustered(N, K, D, seed=N % 97 + D)
    a = _into(inp, gpu_device, store_log_joint=stored)
    b = _into(inp, gpu_device, dense=True, store_log_joint=stored)
    assert_dense_agrees(a, b, bitwise=_stored_applies(N, K, D, stored))
    assert_close_stats(a, oracle(inp), f"sparse N={N} K={K} D={D}")


@pytest.mark.parametrize("stored", [False, True])
def test_phase_split_equals_one_call(stored, gpu_device):
    """PHASE1 then PHASE2 on one workspace gives the single call's outputs bitwise."""
    from flash_gmm import _lib
    inp = data.diag_clustered(5000, 256, 80, seed=16)
    dev = gpu_device
    ref = _into(inp, dev, store_log_joint=stored)
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    L = _lib.lib()
    flags = _lib.FLAG_STORE_LOGJOINT if stored else 0
    ws = torch.empty(L.fgmm_diag_workspace_bytes_ex(N, K, D, flags), dtype=torch.uint8, device=dev)
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, device=dev)]
    args = [inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    diag_estep_into(*args, *out, workspace=ws, phase=1, store_log_joint=stored)
    diag_estep_into(*args, None, *out[1:], workspace=ws, phase=2, store_log_joint=stored)
    torch.cuda.synchronize()
    for u, v in zip(out, ref):
        assert torch.equal(u, v)


def test_equal_variances_match_isotropic(gpu_device):
    inp = data.iso_clustered(3000, 50, 40, seed=12)
    dev = gpu_device
    X, mu, lss, lpi = (inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    a = flash_gmm_estep(X, mu, lss, lpi)
    b = flash_gmm_estep_diag(X, mu, lss[:, None].expand(50, 40).contiguous(), lpi)
    torch.cuda.synchronize()
    assert (a[0] - b[0]).abs().max().item() <= 2 * LOGZ_ATOL
    torch.testing.assert_close(b[1], a[1], rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(b[2], a[2], rtol=1e-4, atol=1e-4 * float(a[2].abs().max()))
    torch.testing.assert_close(b[3].sum(1), a[3], rtol=1e-4, atol=1e-3)


def test_accumulate_over_chunks(gpu_device):
    inp = data.diag_clustered(7000, 100, 48, seed=13)
    dev = gpu_device
    args = [inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    ref = flash_gmm_estep_diag(*args)
    nk = torch.zeros(100, device=dev)
    ma = torch.zeros(100, 48, device=dev)
    sg = torch.zeros(100, 48, device=dev)
    for n0 in range(0, 7000, 3000):
        diag_estep_into(args[0][n0:n0 + 3000], *args[1:], None, nk, ma, sg, accumulate=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(nk, ref[1], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(ma, ref[2], rtol=1e-5, atol=1e-5 * float(ref[2].abs().max()))
    torch.testing.assert_close(sg, ref[3], rtol=1e-5, atol=1e-5 * float(ref[3].abs().max()))


def test_diag_shape_mid_size(gpu_device):
    """K=1024, D=96 axis-aligned clusters at N=32,768 against the float64 oracle."""
    inp = data.diag_clustered(32768, 1024, 96, seed=2)
    assert_close_stats(run_gpu(inp, gpu_device), oracle(inp), "diag K1024 D96 N32768")


def test_diag_wide_mid_size(gpu_device):
    """D=256 (component-tiled pass 1, dimension-range pass 2) at N=8192, K=256 against
    the float64 oracle."""
    inp = data.diag_clustered(8192, 256, 256, seed=5)
    check_wide(run_gpu(inp, gpu_device), inp, "diag K256 D256 N8192", 256)


def test_diag_full_size_properties(gpu_device):
    """N=1M, K=1024, D=96 (the diagonal benchmark workload): every row counted once,
    the gathered accumulation against the dense one, and all four outputs against the
    float64 oracle over every row (about 15 s of CPU)."""
    dev = gpu_device
    inp = data.diag_clustered(1_000_000, 1024, 96, seed=2, device=dev)
    logZ, Nk, mu_acc, sig = flash_gmm_estep_diag(inp["X"], inp["mu"], inp["log_sigma_sq"], inp["log_pi"])
    torch.cuda.synchronize()
    N = 1_000_000
    assert abs(Nk.double().sum().item() - N) <= 1e-5 * N
    torch.testing.assert_close(mu_acc.double().sum(0), inp["X"].double().sum(0), rtol=0,
                               atol=1e-5 * float(mu_acc.abs().sum(0).max()))
    assert torch.all(sig >= -1e-3)
    # The gathered accumulation this data takes agrees with the dense one.
    dense = _into(inp, dev, dense=True)
    assert_dense_agrees((logZ, Nk, mu_acc, sig), dense, bitwise=False)
    print("diag N=1M: full-size oracle (float64, CPU)", flush=True)
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    ref = O.estep_diag(*[inp[k].cpu() for k in ("X", "mu", "log_sigma_sq", "log_pi")])
    print(f"diag N=1M max |logZ - oracle| = {(logZ.cpu().double() - ref[0]).abs().max().item():.3e}", flush=True)
    assert_close_stats((logZ, Nk, mu_acc, sig), ref, "diag K1024 D96 N=1M")


def test_wide_row_stride(gpu_device):
    """A row stride of X above 2^20 floats, past the stored path's 32-bit buffer offsets:
    the call recomputes instead, with results to the same bar."""
    inp = data.diag_clustered(200, 128, 64, seed=21)
    big = torch.zeros(200, (1 << 20) + 64, device=gpu_device)
    big[:, :64] = inp["X"].to(gpu_device)
    got = flash_gmm_estep_diag(big[:, :64], *[inp[k].to(gpu_device) for k in ("mu", "log_sigma_sq", "log_pi")])
    torch.cuda.synchronize()
    assert_close_stats(got, oracle(inp), "diag wide row stride")


def test_rejects_bad_variance_shape(gpu_device):
    inp = data.diag_clustered(10, 4, 8, seed=14)
    X, mu, lss, lpi = (inp[k].to(gpu_device) for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    with pytest.raises(AssertionError):
        flash_gmm_estep_diag(X, mu, lss[:, :4], lpi)


def test_atomic_reduce_matches_the_tree(gpu_device):
    """FGMM_FLAG_ATOMIC_REDUCE: the partials added with float atomics agree with the
    fixed-order tree to float32 rounding (accumulate included)."""
    inp = data.diag_clustered(5000, 200, 48, seed=9)
    ref = _into(inp, gpu_device)
    got = _into(inp, gpu_device, atomic_reduce=True)
    assert torch.equal(got[0], ref[0])
    for u, v in zip(got[1:], ref[1:]):
        torch.testing.assert_close(u, v, rtol=1e-5, atol=1e-5 * float(v.abs().max()))
    acc = [t.clone() for t in got]
    acc_out = [None] + [t.clone() for t in got[1:]]
    diag_estep_into(*[inp[k].to(gpu_device) for k in ("X", "mu", "log_sigma_sq", "log_pi")], None,
                    *acc_out[1:], accumulate=True, atomic_reduce=True)
    torch.cuda.synchronize()
    for u, v in zip(acc_out[1:], acc[1:]):
        torch.testing.assert_close(u, 2 * v, rtol=1e-5, atol=1e-5 * float(v.abs().max()))


# FGMM_FLAG_STORE_LOGJOINT_AUTO (store_log_joint="auto", D <= 96): the device-selected
# stored branch (diag_accum_ljt) on dense data, the default plan elsewhere.
DIAG_AUTO_DENSE_SHAPES = [(20000, 256, 96), (9000, 300, 64), (5000, 130, 61), (3000, 64, 32), (777, 40, 90),
                          (4099, 520, 80)]


@pytest.mark.parametrize("N,K,D", DIAG_AUTO_DENSE_SHAPES)
def test_auto_store_dense_takes_stored_branch(N, K, D, gpu_device):
    """On dense data (X, mu ~ N(0, I), per-dimension variances near 1) the probe selects
    the stored branch: its statistics differ from the default plan's in the last bits
    (another summation) and agree with the oracle."""
    inp = data.diag_reference_smoke(N, K, D, seed=N % 97)
    auto = _into(inp, gpu_device, store_log_joint="auto")
    base = _into(inp, gpu_device)
    assert any(not torch.equal(u, v) for u, v in zip(auto[1:], base[1:]))
    ref = oracle(inp)
    check_wide(auto, inp, f"diag auto dense N={N} K={K} D={D}", D, ref=ref)
    check_wide(base, inp, f"diag default dense N={N} K={K} D={D}", D, ref=ref)


@pytest.mark.parametrize("N,K,D", [(20000, 1024, 96), (9000, 300, 64), (5000, 512, 90), (3000, 300, 128)])
def test_auto_store_clustered_is_the_default_plan(N, K, D, gpu_device):
    """On clustered data with many components the probe keeps the default plan, and
    above D = 96 the flag does not apply: every output bitwise equal to a call
    without the flag.  (At D = 32 the axis-aligned clusters overlap enough that most
    (row, block) pairs are needed, and the stored branch is the probe's choice.)"""
    inp = data.diag_clustered(N, K, D, seed=K % 13 + D)
    auto = _into(inp, gpu_device, store_log_joint="auto")
    base = _into(inp, gpu_device)
    for u, v in zip(auto, base):
        assert torch.equal(u, v)


@pytest.mark.parametrize("kind", ["dense", "clustered"])
def test_auto_store_phase_split_and_reuse(kind, gpu_device):
    """PHASE1 then PHASE2 on one workspace equals the single call bitwise, and calls
    alternating between dense and clustered data on that workspace each select their
    own branch."""
    from flash_gmm import _lib
    L = _lib.lib()
    dev = gpu_device
    dense_inp = data.diag_reference_smoke(6000, 256, 96, seed=4)
    clus_inp = data.diag_clustered(6000, 256, 96, seed=5)
    inp = dense_inp if kind == "dense" else clus_inp
    other = clus_inp if kind == "dense" else dense_inp
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    ws = torch.empty(L.fgmm_diag_workspace_bytes_ex(N, K, D, _lib.FLAG_STORE_LOGJOINT_AUTO), dtype=torch.uint8,
                     device=dev)
    ref = _into(inp, dev, store_log_joint="auto")
    ref_other = _into(other, dev, store_log_joint="auto")
    for _ in range(2):
        for cur, want in ((inp, ref), (other, ref_other)):
            out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
                   torch.empty(K, D, device=dev)]
            args = [cur[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
            diag_estep_into(*args, *out, workspace=ws, phase=1, store_log_joint="auto")
            diag_estep_into(*args, None, *out[1:], workspace=ws, phase=2, store_log_joint="auto")
            torch.cuda.synchronize()
            for u, v in zip(out, want):
                assert torch.equal(u, v)


def test_auto_store_full_size_dense(gpu_device):
    """The dense regime at the benchmark shape (N = 1M, K = 1024, D = 96) through the
    drop-in call, which takes the stored branch: invariants over all rows (sum Nk = N,
    sum mu_acc = sum X, the sig identity against sum X^2 - ...) and all four outputs
    against the oracle on a 32,768-row prefix run on its own."""
    dev = gpu_device
    inp = data.make("diag_ref_n1m_k1024_d96", device=dev)
    X = inp["X"]
    got = flash_gmm_estep_diag(X, inp["mu"], inp["log_sigma_sq"], inp["log_pi"])
    base = _into({k: v for k, v in inp.items()}, dev)
    torch.cuda.synchronize()
    N = X.shape[0]
    assert abs(got[1].double().sum().item() - N) <= 1e-4 * N
    torch.testing.assert_close(got[2].double().sum(0), X.double().sum(0), rtol=1e-4, atol=1e-3 * N ** 0.5)
    # The stored branch and the default plan agree on all rows: logZ (pass 1 of both,
    # another instance of the kernel) to 1e-5, the statistics to 1e-5 of each
    # output's largest magnitude.
    assert float((got[0] - base[0]).abs().max()) <= 1e-5
    for u, v in zip(got[1:], base[1:]):
        assert float((u - v).abs().max()) <= 1e-5 * float(v.abs().max())
    sub = {k: (v[:32768].cpu() if k == "X" else v.cpu()) for k, v in inp.items()}
    part = flash_gmm_estep_diag(*[sub[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")])
    torch.cuda.synchronize()
    check_wide(part, sub, "diag auto N=32768 K=1024 D=96 dense", 96)


def test_auto_store_accumulate_over_chunks(gpu_device):
    """FGMM_FLAG_ACCUMULATE with the stored branch selected: three row chunks added
    into the outputs equal one call over all rows (to float32 rounding)."""
    dev = gpu_device
    inp = data.diag_reference_smoke(9000, 256, 96, seed=7)
    args = [inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    ref = _into(inp, dev, store_log_joint="auto")
    K, D = 256, 96
    nk, ma, sg = torch.zeros(K, device=dev), torch.zeros(K, D, device=dev), torch.zeros(K, D, device=dev)
    for n0 in range(0, 9000, 3000):
        diag_estep_into(args[0][n0:n0 + 3000], *args[1:], None, nk, ma, sg, accumulate=True, store_log_joint="auto")
    torch.cuda.synchronize()
    torch.testing.assert_close(nk, ref[1], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(ma, ref[2], rtol=1e-5, atol=1e-5 * float(ref[2].abs().max()))
    torch.testing.assert_close(sg, ref[3], rtol=1e-5, atol=1e-5 * float(ref[3].abs().max()))

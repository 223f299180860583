"""GPU parity of the full-covariance E-step against the CPU oracle (tolerances in parity.py;
sig_outer element-wise against sqrt(S_ii S_jj) of its component)."""

import os
import sys

import numpy as np
import pytest
import torch

from flash_gmm import data, flash_gmm_estep_diag, flash_gmm_estep_full, full_estep_into
from oracle import gmm_oracle as O

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden  # noqa: E402
from parity import LOGZ_ATOL, assert_close_stats, assert_dense_agrees  # noqa: E402

pytestmark = pytest.mark.gpu

KEYS = ("X", "mu", "prec_chol", "log_pi")


def run_gpu(inp, dev):
    out = flash_gmm_estep_full(*[inp[k].to(dev) for k in KEYS])
    torch.cuda.synchronize()
    return out


def oracle(inp):
    return O.estep_full(*[inp[k] for k in KEYS])


def _into(inp, dev, **kw):
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, D, device=dev)]
    full_estep_into(*[inp[k].to(dev) for k in KEYS], *out, **kw)
    torch.cuda.synchronize()
    return out


def test_golden_vectors(gpu_device):
    name = "full_n2000_k12_d16"
    inp, kind = make_golden.make_inputs(name)
    fx = np.load(os.path.join(os.path.dirname(make_golden.__file__), name + ".npz"))
    assert str(fx["sha256"]) == make_golden.input_digest(inp)
    assert_close_stats(run_gpu(inp, gpu_device), (fx["logZ"], fx["Nk"], fx["mu_acc"], fx["sig"]), name)


@pytest.mark.parametrize("N,K,D", [(1, 1, 1), (33, 5, 3), (500, 12, 16), (300, 7, 64),
                                   (1000, 33, 40), (129, 4, 32), (2000, 9, 63),
                                   (400, 9, 65), (600, 11, 96), (300, 5, 100), (500, 7, 128),
                                   (3, 2, 127)])
@pytest.mark.parametrize("stored", [False, True])
def test_edge_shapes(N, K, D, stored, gpu_device):
    """Pass 2 recomputing (default), and from the log-joint stored by pass 1."""
    inp = data.full_clustered(N, K, D, seed=N + K + D)
    assert_close_stats(_into(inp, gpu_device, store_log_joint=stored), oracle(inp),
                       f"full N={N} K={K} D={D} stored={stored}")


def test_diagonal_factor_matches_diag_entry(gpu_device):
    inp = data.diag_clustered(3000, 20, 24, seed=15)
    dev = gpu_device
    X, mu, lss, lpi = (inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    L = torch.diag_embed(torch.exp(-0.5 * lss.double()).float())
    a = flash_gmm_estep_diag(X, mu, lss, lpi)
    b = flash_gmm_estep_full(X, mu, L, lpi)
    torch.cuda.synchronize()
    assert (a[0] - b[0]).abs().max().item() <= 2 * LOGZ_ATOL
    torch.testing.assert_close(b[1], a[1], rtol=2e-4, atol=1e-4)
    torch.testing.assert_close(b[2], a[2], rtol=2e-4, atol=2e-4 * float(a[2].abs().max()))
    # diag sig_acc from sig_outer: diag(S) - 2 mu mu_acc + mu^2 Nk
    s = b[3].diagonal(dim1=1, dim2=2) - 2 * mu * b[2] + mu * mu * b[1][:, None]
    torch.testing.assert_close(s, a[3], rtol=1e-3, atol=1e-3 * float(a[3].abs().max()))


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("N,K,D,seed", [(6000, 128, 64, 3), (2501, 19, 29, 4), (3000, 24, 128, 5)])
def test_zero_step_skip_is_bitwise_dense(N, K, D, seed, stored, gpu_device):
    """Skipping all-zero responsibility steps changes no bit of any output."""
    inp = data.full_clustered(N, K, D, seed=seed)
    dev = gpu_device
    args = [inp[k].to(dev) for k in KEYS]
    outs = []
    for dense in (False, True):
        o = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
             torch.empty(K, D, D, device=dev)]
        full_estep_into(*args, *o, dense=dense, store_log_joint=stored)
        outs.append(o)
    torch.cuda.synchronize()
    # The default plan's gathering pass 2 adds the needed rows in its own tiles.
    assert_dense_agrees(outs[0], outs[1], bitwise=stored)
    assert_close_stats(outs[0], oracle(inp), "full skip")
    assert_close_stats(outs[1], oracle(inp), "full dense")


@pytest.mark.parametrize("N,K,D", [(8192, 256, 64), (3000, 40, 128), (3000, 1100, 32),
                                   (2000, 600, 64), (1500, 1100, 64)])
def test_default_plan_on_dense_data(N, K, D, gpu_device):
    """The default plan where nearly every pair is needed (the reference's N(0, I) data).
    Pass 1 forms its need masks from per-row candidate lists where they fit in LDS (the
    first three shapes: the lists overflow and set bits directly), else from bounds in
    the workspace (K = 600, D = 64) or the running maximum (K = 1100, D = 64).  Every
    form must give the oracle's outputs, and agree with dense=True."""
    inp = data.full_reference_smoke(N, K, D, seed=11)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device, dense=True)
    assert_dense_agrees(a, b, bitwise=False)
    assert_close_stats(a, oracle(inp), f"full default plan dense data N={N} K={K} D={D}")


@pytest.mark.parametrize("D", [72, 48])
@pytest.mark.parametrize("stored", [False, True])
def test_phase_split_equals_one_call(stored, D, gpu_device):
    """PHASE1 then PHASE2 on one workspace gives the single call's outputs bitwise."""
    from flash_gmm import _lib
    inp = data.full_clustered(3000, 40, D, seed=17)
    dev = gpu_device
    ref = _into(inp, dev, store_log_joint=stored)
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    L = _lib.lib()
    flags = _lib.FLAG_STORE_LOGJOINT if stored else 0
    ws_default = L.fgmm_full_workspace_bytes(N, K, D)
    ws = torch.empty(L.fgmm_full_workspace_bytes_ex(N, K, D, flags), dtype=torch.uint8, device=dev)
    assert (ws.numel() != ws_default) == stored
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, D, device=dev)]
    args = [inp[k].to(dev) for k in KEYS]
    full_estep_into(*args, *out, workspace=ws, phase=1, store_log_joint=stored)
    full_estep_into(*args, None, *out[1:], workspace=ws, phase=2, store_log_joint=stored)
    torch.cuda.synchronize()
    for u, v in zip(out, ref):
        assert torch.equal(u, v)


def test_accumulate_over_chunks(gpu_device):
    inp = data.full_clustered(5000, 16, 32, seed=16)
    dev = gpu_device
    args = [inp[k].to(dev) for k in KEYS]
    ref = flash_gmm_estep_full(*args)
    nk = torch.zeros(16, device=dev)
    ma = torch.zeros(16, 32, device=dev)
    so = torch.zeros(16, 32, 32, device=dev)
    for n0 in range(0, 5000, 1700):
        full_estep_into(args[0][n0:n0 + 1700], *args[1:], None, nk, ma, so, accumulate=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(nk, ref[1], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(ma, ref[2], rtol=1e-5, atol=1e-5 * float(ref[2].abs().max()))
    torch.testing.assert_close(so, ref[3], rtol=1e-5, atol=1e-5 * float(ref[3].abs().max()))


def test_full_shape_mid_size(gpu_device):
    """K=256, D=64 at N=8,192 against the float64 oracle."""
    inp = data.full_clustered(8192, 256, 64, seed=3)
    assert_close_stats(run_gpu(inp, gpu_device), oracle(inp), "full K256 D64 N8192")


def test_full_wide_mid_size(gpu_device):
    """D=128 (one component per workgroup in pass 2) at N=4,096, K=48 against the float64 oracle."""
    inp = data.full_clustered(4096, 48, 128, seed=6)
    assert_close_stats(run_gpu(inp, gpu_device), oracle(inp), "full K48 D128 N4096")


def test_full_size_properties(gpu_device):
    """N=250K, K=256, D=64 (the full-covariance benchmark workload): sum_k Nk = N,
    sum_k mu_acc = sum x, sum_k sig_outer = X^T X, and all four outputs (sig_outer
    included) against the float64 oracle over every row (about 25 s of CPU)."""
    dev = gpu_device
    inp = data.full_clustered(250_000, 256, 64, seed=3, device=dev)
    logZ, Nk, mu_acc, so = flash_gmm_estep_full(*[inp[k] for k in KEYS])
    torch.cuda.synchronize()
    N = 250_000
    X = inp["X"].double()
    assert abs(Nk.double().sum().item() - N) <= 1e-5 * N
    torch.testing.assert_close(mu_acc.double().sum(0), X.sum(0), rtol=0,
                               atol=1e-5 * float(mu_acc.abs().sum(0).max()))
    xtx = X.T @ X
    torch.testing.assert_close(so.double().sum(0), xtx, rtol=0, atol=1e-5 * float(xtx.abs().max()))
    assert torch.all(so.diagonal(dim1=1, dim2=2) >= 0)
    print("full N=250K: full-size oracle (float64, CPU)", flush=True)
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    ref = O.estep_full(*[inp[k].cpu() for k in KEYS])
    print(f"full N=250K max |logZ - oracle| = {(logZ.cpu().double() - ref[0]).abs().max().item():.3e}", flush=True)
    assert_close_stats((logZ, Nk, mu_acc, so), ref, "full K256 D64 N=250K")


def test_rejects_bad_factor_shape(gpu_device):
    inp = data.full_clustered(10, 3, 8, seed=17)
    X, mu, L, lpi = (inp[k].to(gpu_device) for k in KEYS)
    with pytest.raises(AssertionError):
        flash_gmm_estep_full(X, mu, L[:, :4, :4], lpi)


def test_atomic_reduce_matches_the_tree(gpu_device):
    """FGMM_FLAG_ATOMIC_REDUCE: the partials added with float atomics agree with the
    fixed-order tree to float32 rounding (accumulate included)."""
    inp = data.full_clustered(5000, 200, 48, seed=9)
    ref = _into(inp, gpu_device)
    got = _into(inp, gpu_device, atomic_reduce=True)
    assert torch.equal(got[0], ref[0])
    for u, v in zip(got[1:], ref[1:]):
        torch.testing.assert_close(u, v, rtol=1e-5, atol=1e-5 * float(v.abs().max()))
    acc = [t.clone() for t in got]
    acc_out = [None] + [t.clone() for t in got[1:]]
    full_estep_into(*[inp[k].to(gpu_device) for k in KEYS], None,
                    *acc_out[1:], accumulate=True, atomic_reduce=True)
    torch.cuda.synchronize()
    for u, v in zip(acc_out[1:], acc[1:]):
        torch.testing.assert_close(u, 2 * v, rtol=1e-5, atol=1e-5 * float(v.abs().max()))


# FGMM_FLAG_STORE_LOGJOINT_AUTO (store_log_joint="auto", D <= 64, K <= 512): the
# device-selected stored branch (pass 1 keeps the log-joint, full_accum_ljt reads r
# from it) on dense data, the default plan elsewhere.
FULL_AUTO_DENSE_SHAPES = [(8000, 128, 64), (6000, 64, 64), (3001, 130, 61), (3000, 40, 32), (777, 20, 50),
                          (4099, 257, 33)]


@pytest.mark.parametrize("N,K,D", FULL_AUTO_DENSE_SHAPES)
def test_auto_store_dense_takes_stored_branch(N, K, D, gpu_device):
    """On dense data (X, mu ~ N(0, I), covariances near I) the probe selects the
    stored branch: its statistics differ from the default plan's in the last bits
    (another summation) and agree with the oracle."""
    inp = data.full_reference_smoke(N, K, D, seed=N % 97)
    auto = _into(inp, gpu_device, store_log_joint="auto")
    base = _into(inp, gpu_device)
    assert any(not torch.equal(u, v) for u, v in zip(auto[1:], base[1:]))
    ref = oracle(inp)
    assert_close_stats(auto, ref, f"full auto dense N={N} K={K} D={D}")
    assert_close_stats(base, ref, f"full default dense N={N} K={K} D={D}")


@pytest.mark.parametrize("N,K,D", [(20000, 256, 64), (5000, 512, 48), (3000, 100, 96), (2000, 600, 32)])
def test_auto_store_clustered_is_the_default_plan(N, K, D, gpu_device):
    """On clustered data the probe keeps the default plan, and above D = 64 or
    K = 512 the flag does not apply: every output bitwise equal to a call without
    the flag."""
    inp = data.full_clustered(N, K, D, seed=K % 13 + D)
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
    dense_inp = data.full_reference_smoke(6000, 128, 64, seed=4)
    clus_inp = data.full_clustered(6000, 128, 64, seed=5)
    inp = dense_inp if kind == "dense" else clus_inp
    other = clus_inp if kind == "dense" else dense_inp
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    ws = torch.empty(L.fgmm_full_workspace_bytes_ex(N, K, D, _lib.FLAG_STORE_LOGJOINT_AUTO), dtype=torch.uint8,
                     device=dev)
    ref = _into(inp, dev, store_log_joint="auto")
    ref_other = _into(other, dev, store_log_joint="auto")
    for _ in range(2):
        for cur, want in ((inp, ref), (other, ref_other)):
            out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
                   torch.empty(K, D, D, device=dev)]
            args = [cur[k].to(dev) for k in KEYS]
            full_estep_into(*args, *out, workspace=ws, phase=1, store_log_joint="auto")
            full_estep_into(*args, None, *out[1:], workspace=ws, phase=2, store_log_joint="auto")
            torch.cuda.synchronize()
            for u, v in zip(out, want):
                assert torch.equal(u, v)


def test_auto_store_full_size_dense(gpu_device):
    """The dense regime at the benchmark shape (N = 250K, K = 256, D = 64) through the
    drop-in call, which takes the stored branch: sum Nk = N, sum mu_acc = sum X,
    sum sig_outer = X^T X over all rows, agreement with the default plan, and all
    four outputs against the oracle on an 8,192-row prefix run on its own."""
    dev = gpu_device
    inp = data.make("full_ref_n250k_k256_d64", device=dev)
    got = flash_gmm_estep_full(*[inp[k] for k in KEYS])
    base = _into(inp, dev)
    torch.cuda.synchronize()
    N = inp["X"].shape[0]
    X = inp["X"].double()
    assert abs(got[1].double().sum().item() - N) <= 1e-5 * N
    torch.testing.assert_close(got[2].double().sum(0), X.sum(0), rtol=0,
                               atol=1e-5 * float(got[2].abs().sum(0).max()))
    xtx = X.T @ X
    torch.testing.assert_close(got[3].double().sum(0), xtx, rtol=0, atol=1e-5 * float(xtx.abs().max()))
    assert float((got[0] - base[0]).abs().max()) <= 1e-5
    for u, v in zip(got[1:], base[1:]):
        assert float((u - v).abs().max()) <= 1e-5 * float(v.abs().max())
    sub = {k: (v[:8192].cpu() if k == "X" else v.cpu()) for k, v in inp.items()}
    part = run_gpu(sub, dev)
    assert_close_stats(part, oracle(sub), "full auto N=8192 K=256 D=64 dense")


def test_auto_store_accumulate_over_chunks(gpu_device):
    """FGMM_FLAG_ACCUMULATE with the stored branch selected: three row chunks added
    into the outputs equal one call over all rows (to float32 rounding)."""
    dev = gpu_device
    inp = data.full_reference_smoke(6000, 128, 64, seed=7)
    args = [inp[k].to(dev) for k in KEYS]
    ref = _into(inp, dev, store_log_joint="auto")
    K, D = 128, 64
    nk, ma, so = torch.zeros(K, device=dev), torch.zeros(K, D, device=dev), torch.zeros(K, D, D, device=dev)
    for n0 in range(0, 6000, 2000):
        full_estep_into(args[0][n0:n0 + 2000], *args[1:], None, nk, ma, so, accumulate=True, store_log_joint="auto")
    torch.cuda.synchronize()
    torch.testing.assert_close(nk, ref[1], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(ma, ref[2], rtol=1e-5, atol=1e-5 * float(ref[2].abs().max()))
    torch.testing.assert_close(so, ref[3], rtol=1e-5, atol=1e-5 * float(ref[3].abs().max()))

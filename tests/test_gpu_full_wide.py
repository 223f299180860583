"""GPU parity of the full-covariance E-step above D = 128, against the float64 oracle.
Up to D = 256 pass 1 runs at one wave per SIMD and the gathering pass 2 deals the
upper blocks of sig_outer to several waves per (slab, component); above 256 pass 1
(full_lse_wide) re-splits the rows per group of coordinate blocks and stores the
log-joint, and pass 2 (full_accum_wide) reads r from it.  The reference pads any D
to a power of two (flash_gmm_full_h100.py:268)."""

import os
import sys

import pytest
import torch

from flash_gmm import data, full_estep_into
from oracle import gmm_oracle as O

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from parity import assert_close_stats, assert_dense_agrees, logz_atol_fp32, logz_err  # noqa: E402

pytestmark = pytest.mark.gpu

KEYS = ("X", "mu", "prec_chol", "log_pi")


def oracle(inp, dtype=torch.float64):
    return O.estep_full(*[inp[k] for k in KEYS], dtype=dtype)


def check_wide(got, inp, what, D, ref=None):
    """All four outputs against the float64 oracle.  The logZ bound is 1e-4 up to
    D = 128; above, max(1e-4, the error of the float32 restatement of the reference's
    arithmetic on the same rows), measured here."""
    ref = oracle(inp) if ref is None else ref
    atol = logz_atol_fp32(oracle(inp, torch.float32)[0] if D > 128 else None, ref[0], D)
    print(f"{what}: max |logZ - oracle| {logz_err(got[0], ref[0]):.2e}, bound {atol:.2e}", flush=True)
    assert_close_stats(got, ref, what, logz_atol=atol)


def _into(inp, dev, **kw):
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, D, device=dev)]
    full_estep_into(*[inp[k].to(dev) for k in KEYS], *out, **kw)
    torch.cuda.synchronize()
    return out


# (N, K, D): every padded width above 128 (160, 192, 224, 256: two to four waves of
# sig_outer blocks), ragged D, partial row tiles, K = 1.
SHAPES = [(300, 5, 129), (2000, 16, 160), (700, 9, 181), (500, 7, 200), (1000, 12, 224), (400, 9, 256),
          (37, 1, 250)]


@pytest.mark.parametrize("N,K,D", SHAPES)
def test_wide_d_against_oracle(N, K, D, gpu_device):
    print(f"full wide N={N} K={K} D={D}", flush=True)
    inp = data.full_clustered(N, K, D, seed=N + K + D)
    got = _into(inp, gpu_device)
    check_wide(got, inp, f"full N={N} K={K} D={D}", D)


@pytest.mark.parametrize("D", [200, 256])
def test_wide_d_skip_agrees_with_dense(D, gpu_device):
    """Gathering only the needed rows against FGMM_FLAG_DENSE: logZ bitwise, statistics to
    1e-5 (other groupings of the same nonzero terms)."""
    inp = data.full_clustered(3000, 24, D, seed=6)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device, dense=True)
    assert_dense_agrees(a, b, bitwise=False)
    check_wide(b, inp, f"full dense D={D}", D)


def test_wide_d_phase_split_equals_one_call(gpu_device):
    """PHASE1 then PHASE2 on one workspace gives the single call's outputs bitwise."""
    N, K, D = 2000, 20, 200
    inp = data.full_clustered(N, K, D, seed=16)
    dev = gpu_device
    ref = _into(inp, dev)
    from flash_gmm import _lib
    L = _lib.lib()
    ws = torch.empty(L.fgmm_full_workspace_bytes(N, K, D), dtype=torch.uint8, device=dev)
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, D, device=dev)]
    args = [inp[k].to(dev) for k in KEYS]
    full_estep_into(*args, *out, workspace=ws, phase=1)
    full_estep_into(*args, None, *out[1:], workspace=ws, phase=2)
    torch.cuda.synchronize()
    for u, v in zip(out, ref):
        assert torch.equal(u, v)


def test_wide_d_stored_request_runs_the_default_plan(gpu_device):
    """The stored log-joint applies up to D = 128; above, store_log_joint=True takes the
    default plan (same workspace, same bits)."""
    N, K, D = 1500, 10, 192
    from flash_gmm import _lib
    L = _lib.lib()
    assert L.fgmm_full_workspace_bytes(N, K, D) == L.fgmm_full_workspace_bytes_ex(N, K, D, _lib.FLAG_STORE_LOGJOINT)
    inp = data.full_clustered(N, K, D, seed=8)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device, store_log_joint=True)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_wide_d_mid_size(gpu_device):
    """D = 200 at N=16,384, K=64 against the float64 oracle."""
    inp = data.full_clustered(16384, 64, 200, seed=4)
    got = _into(inp, gpu_device)
    ref = oracle(inp)
    err = (got[0].cpu().double() - ref[0]).abs().max().item()
    print(f"full N=16384 K=64 D=200: max |logZ - oracle| = {err:.3e}", flush=True)
    check_wide(got, inp, "full N=16384 K=64 D=200", 200, ref=ref)


# Above D = 256: one past the register-resident width, GloVe-300, a power of two,
# ragged widths over several coordinate groups and sig strips, K = 1 at D = 1000.
SHAPES_ABOVE_256 = [(257, 3, 257), (600, 5, 300), (400, 4, 512), (300, 2, 520), (65, 1, 1000)]


@pytest.mark.parametrize("N,K,D", SHAPES_ABOVE_256)
def test_above_256_against_oracle(N, K, D, gpu_device):
    print(f"full wide N={N} K={K} D={D}", flush=True)
    inp = data.full_clustered(N, K, D, seed=N + K + D)
    got = _into(inp, gpu_device)
    check_wide(got, inp, f"full N={N} K={K} D={D}", D)


def test_above_256_dense_and_phase_split_are_bitwise(gpu_device):
    """Above D = 256 pass 2 reads the stored log-joint: skipping the steps whose
    responsibilities are zero adds nothing, so FGMM_FLAG_DENSE gives the same bits;
    PHASE1 then PHASE2 on one workspace gives the single call's bits."""
    N, K, D = 1500, 6, 300
    inp = data.full_clustered(N, K, D, seed=21)
    dev = gpu_device
    ref = _into(inp, dev)
    dense = _into(inp, dev, dense=True)
    for u, v in zip(ref, dense):
        assert torch.equal(u, v)
    from flash_gmm import _lib
    L = _lib.lib()
    ws = torch.empty(L.fgmm_full_workspace_bytes(N, K, D), dtype=torch.uint8, device=dev)
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, D, device=dev)]
    args = [inp[k].to(dev) for k in KEYS]
    full_estep_into(*args, *out, workspace=ws, phase=1)
    full_estep_into(*args, None, *out[1:], workspace=ws, phase=2)
    torch.cuda.synchronize()
    for u, v in zip(out, ref):
        assert torch.equal(u, v)


def test_above_256_mid_size(gpu_device):
    """D = 300 at N=8,192, K=16 against the float64 oracle, with the sig_outer
    invariant sum_k sig_outer_k = X^T X."""
    N, K, D = 8192, 16, 300
    inp = data.full_clustered(N, K, D, seed=5)
    got = _into(inp, gpu_device)
    check_wide(got, inp, f"full N={N} K={K} D={D}", D)
    X = inp["X"].double()
    xtx = X.T @ X
    tot = got[3].double().cpu().sum(0)
    assert float((tot - xtx).abs().max()) <= 1e-4 * float(xtx.abs().max())

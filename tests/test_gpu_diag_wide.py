"""GPU parity of the diagonal-covariance E-step above D = 128, where pass 1 tiles the
contraction over components (diag_lse_ctile) and pass 2 splits r^T [X | X^2] over
ranges of dimensions (diag_accum_drange), against the float64 oracle.  The reference
takes any D (flash_gmm_diag_h100.py:317: BLOCK_D is the next power of two)."""

import os
import sys

import pytest
import torch

from flash_gmm import data, diag_estep_into
from oracle import gmm_oracle as O

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from parity import assert_close_stats, assert_dense_agrees, logz_atol_fp32, logz_err  # noqa: E402

pytestmark = pytest.mark.gpu


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


def _into(inp, dev, **kw):
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, device=dev)]
    diag_estep_into(*[inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi")], *out, **kw)
    torch.cuda.synchronize()
    return out


# (N, K, D): one past the register-resident width, ragged K and D, GloVe-300 and
# GIST-960 widths, two and three dimension ranges (1100, 2100), tiny K.
SHAPES = [(300, 5, 129), (2500, 260, 192), (3000, 200, 300), (4097, 257, 301), (2000, 130, 960),
          (1500, 70, 1100), (700, 40, 2100), (33, 1, 640)]


@pytest.mark.parametrize("N,K,D", SHAPES)
def test_wide_d_against_oracle(N, K, D, gpu_device):
    print(f"diag wide N={N} K={K} D={D}", flush=True)
    inp = data.diag_clustered(N, K, D, seed=N + K + D)
    got = _into(inp, gpu_device)
    check_wide(got, inp, f"diag N={N} K={K} D={D}", D)


@pytest.mark.parametrize("N,K,D", [(6000, 512, 256), (3000, 300, 960)])
def test_wide_d_skip_agrees_with_dense(N, K, D, gpu_device):
    """Gathering only the needed rows against FGMM_FLAG_DENSE: logZ bitwise, statistics to
    1e-5 (other groupings of the same nonzero terms)."""
    inp = data.diag_clustered(N, K, D, seed=6)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device, dense=True)
    assert_dense_agrees(a, b, bitwise=False)
    check_wide(b, inp, f"diag dense N={N} K={K} D={D}", D)


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("D", [200, 1100])
def test_wide_d_phase_split_equals_one_call(D, stored, gpu_device):
    """PHASE1 then PHASE2 on one workspace gives the single call's outputs bitwise (the
    stored plan applies up to D = 256)."""
    inp = data.diag_clustered(3000, 160, D, seed=16)
    dev = gpu_device
    ref = _into(inp, dev, store_log_joint=stored)
    N, K = 3000, 160
    from flash_gmm import _lib
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


def test_wide_d_need_masks_from_the_running_max(gpu_device):
    """More component blocks than pass 1 keeps half-block bounds for in LDS (K=6,000):
    the need masks come from the running-max bound; against the dense pass and the oracle."""
    inp = data.diag_clustered(1200, 6000, 160, seed=23)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device, dense=True)
    assert_dense_agrees(a, b, bitwise=False)
    check_wide(a, inp, "diag running-max masks D=160", 160)


def test_wide_d_randn_variances(gpu_device):
    """Overlapping components (X, mu ~ N(0, I), per-dimension log variances ~ U(-0.5, 0.5)):
    most (row, block) pairs are needed."""
    g = torch.Generator().manual_seed(5)
    N, K, D = 3000, 128, 400
    inp = dict(X=torch.randn(N, D, generator=g), mu=torch.randn(K, D, generator=g),
               log_sigma_sq=torch.rand(K, D, generator=g) - 0.5,
               log_pi=torch.log_softmax(torch.randn(K, generator=g, dtype=torch.float64), 0).float())
    got = _into(inp, gpu_device)
    check_wide(got, inp, "diag randn D=400", D)


def test_wide_d_mid_size(gpu_device):
    """GIST-960 width at N=16,384, K=512 against the float64 oracle."""
    inp = data.diag_clustered(16384, 512, 960, seed=4)
    got = _into(inp, gpu_device)
    ref = oracle(inp)
    err = (got[0].cpu().double() - ref[0]).abs().max().item()
    print(f"diag N=16384 K=512 D=960: max |logZ - oracle| = {err:.3e}", flush=True)
    check_wide(got, inp, "diag N=16384 K=512 D=960", 960, ref=ref)

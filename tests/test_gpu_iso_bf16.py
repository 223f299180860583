"""GPU parity of the isotropic E-step under the bf16 operand contract (precision="bf16",
FGMM_FLAG_BF16) against the oracle restatement of that contract."""

import math

import pytest
import torch

from flash_gmm import FlashGMMError, data, flash_gmm_estep, iso_estep_into
from oracle import gmm_oracle as O
from parity import (LOGZ_ATOL_BF16, REL_BF16_STATS_WIDE, assert_close_stats, assert_dense_agrees,
                    logz_atol_bf16, logz_err)

pytestmark = pytest.mark.gpu

KEYS = ("X", "mu", "log_sigma_sq", "log_pi")


def oracle(inp):
    return O.estep_iso_bf16(*[inp[k] for k in KEYS])


def _into(inp, dev, **kw):
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, device=dev)]
    iso_estep_into(*[inp[k].to(dev) for k in KEYS], *out, precision="bf16", **kw)
    torch.cuda.synchronize()
    return out


SHAPES = [(1, 1, 1), (33, 1, 1), (31, 3, 5), (200, 5, 7), (129, 33, 32), (1000, 64, 32),
          (2000, 130, 61), (3000, 100, 96), (5000, 300, 128), (700, 40, 129), (4000, 260, 192),
          (3000, 200, 256), (2048, 1, 64), (4097, 70, 100)]


@pytest.mark.parametrize("N,K,D", SHAPES)
def test_edge_shapes(N, K, D, gpu_device):
    inp = data.iso_clustered(N, K, D, seed=N + K + D)
    got = _into(inp, gpu_device)
    assert_close_stats(got, oracle(inp), f"bf16 N={N} K={K} D={D}", logz_atol=LOGZ_ATOL_BF16)


def test_plain_gaussian_data(gpu_device):
    """The reference's own smoke data (flash_gmm.py:224-236): X, mu ~ N(0, I)."""
    g = torch.Generator().manual_seed(0)
    N, K, D = 20000, 256, 128
    inp = {"X": torch.randn(N, D, generator=g), "mu": torch.randn(K, D, generator=g),
           "log_sigma_sq": torch.zeros(K), "log_pi": torch.full((K,), -math.log(K))}
    assert_close_stats(_into(inp, gpu_device), oracle(inp), "bf16 smoke data", logz_atol=LOGZ_ATOL_BF16)


def test_headline_shape_mid_size(gpu_device):
    inp = data.iso_clustered(32768, 1024, 128, seed=1)
    assert_close_stats(_into(inp, gpu_device), oracle(inp), "bf16 K1024 D128", logz_atol=LOGZ_ATOL_BF16)


@pytest.mark.parametrize("N,K,D", [(12000, 1024, 128), (7777, 300, 61), (5000, 64, 32), (3000, 200, 256)])
def test_need_masks_agree_with_dense(N, K, D, gpu_device):
    """Up to D = 128 pass 1 writes need masks and the gathering pass 2 adds the needed
    rows' terms; FGMM_FLAG_DENSE runs every row of every block: logZ bitwise, the
    statistics to 1e-5 (other groupings of the same nonzero terms).  Above D = 128
    (no masks) skipping zero steps is bitwise the dense run."""
    inp = data.iso_clustered(N, K, D, seed=4)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device, dense=True)
    assert_dense_agrees(a, b, bitwise=D > 128)
    assert_close_stats(a, oracle(inp), f"bf16 gather N={N} K={K} D={D}", logz_atol=LOGZ_ATOL_BF16)


def test_phase_split_and_accumulate(gpu_device):
    """PHASE1 then PHASE2 equals one call bitwise; ACCUMULATE over chunks equals one call."""
    from flash_gmm import _lib
    inp = data.iso_clustered(9000, 128, 64, seed=10)
    dev = gpu_device
    ref = _into(inp, dev)
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    L = _lib.lib()
    ws = torch.empty(L.fgmm_iso_workspace_bytes_ex(N, K, D, _lib.FLAG_BF16), dtype=torch.uint8, device=dev)
    args = [inp[k].to(dev) for k in KEYS]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, device=dev)]
    iso_estep_into(*args, *out, workspace=ws, phase=1, precision="bf16")
    iso_estep_into(*args, None, *out[1:], workspace=ws, phase=2, precision="bf16")
    torch.cuda.synchronize()
    for u, v in zip(out, ref):
        assert torch.equal(u, v)
    nk = torch.zeros(K, device=dev)
    ma = torch.zeros(K, D, device=dev)
    sg = torch.zeros(K, device=dev)
    for n0 in range(0, N, 2500):
        iso_estep_into(args[0][n0:n0 + 2500], *args[1:], None, nk, ma, sg, accumulate=True, precision="bf16")
    torch.cuda.synchronize()
    torch.testing.assert_close(nk, ref[1], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(ma, ref[2], rtol=1e-5, atol=1e-5 * float(ref[2].abs().max()))
    torch.testing.assert_close(sg, ref[3], rtol=1e-5, atol=1e-4 * float(ref[3].abs().max()))


def test_bad_precision_string(gpu_device):
    inp = data.iso_plain(10, 4, 8, seed=11)
    with pytest.raises(FlashGMMError):
        flash_gmm_estep(*[inp[k].to(gpu_device) for k in KEYS], precision="fp16")


# Above D = 256 the contract stores the log-joint: pass 1 tiles the contraction over
# components, pass 2 reads r from the stored rows per range of 256 dimensions.
# GloVe-300 and GIST-960 widths, one past the narrow kernels, several dimension
# ranges with a partial last one, partial component tiles and K = 1.
WIDE_SHAPES = [(1000, 40, 257), (3000, 100, 300), (2000, 130, 960), (700, 33, 1100), (65, 1, 640)]


@pytest.mark.parametrize("N,K,D", WIDE_SHAPES)
def test_above_256_against_oracle(N, K, D, gpu_device):
    print(f"iso bf16 wide N={N} K={K} D={D}", flush=True)
    inp = data.iso_clustered(N, K, D, seed=N + K + D)
    got, ref = _into(inp, gpu_device), oracle(inp)
    atol = logz_atol_bf16(O.estep_iso_bf16(*[inp[k] for k in KEYS], dtype=torch.float32)[0], ref[0], D)
    print(f"max |logZ - oracle| {logz_err(got[0], ref[0]):.2e}, bound {atol:.2e}", flush=True)
    # mu_acc sums bf16(r) x: with the log-joint within the float32 restatement's
    # error of the replay, bf16(r) can round one unit apart (parity.REL_BF16_STATS_WIDE).
    assert_close_stats(got, ref, f"bf16 N={N} K={K} D={D}", logz_atol=atol, bf16_stats=True,
                       bf16_rel=REL_BF16_STATS_WIDE)


def test_above_256_plain_gaussian_dense_and_phase_split(gpu_device):
    """The reference's smoke data at D = 960 (every r fractional) against the oracle;
    FGMM_FLAG_DENSE and PHASE1-then-PHASE2 give the single call's bits."""
    from flash_gmm import _lib
    g = torch.Generator().manual_seed(7)
    N, K, D = 4000, 64, 960
    inp = {"X": torch.randn(N, D, generator=g), "mu": torch.randn(K, D, generator=g),
           "log_sigma_sq": torch.zeros(K), "log_pi": torch.full((K,), -math.log(K))}
    dev = gpu_device
    ref = _into(inp, dev)
    r64 = oracle(inp)
    atol = logz_atol_bf16(O.estep_iso_bf16(*[inp[k] for k in KEYS], dtype=torch.float32)[0], r64[0], D)
    print(f"max |logZ - oracle| {logz_err(ref[0], r64[0]):.2e}, bound {atol:.2e}", flush=True)
    assert_close_stats(ref, r64, "bf16 smoke data D=960", logz_atol=atol, bf16_stats=True,
                       bf16_rel=REL_BF16_STATS_WIDE)
    for u, v in zip(_into(inp, dev, dense=True), ref):
        assert torch.equal(u, v)
    L = _lib.lib()
    ws = torch.empty(L.fgmm_iso_workspace_bytes_ex(N, K, D, _lib.FLAG_BF16), dtype=torch.uint8, device=dev)
    args = [inp[k].to(dev) for k in KEYS]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, device=dev)]
    iso_estep_into(*args, *out, workspace=ws, phase=1, precision="bf16")
    iso_estep_into(*args, None, *out[1:], workspace=ws, phase=2, precision="bf16")
    torch.cuda.synchronize()
    for u, v in zip(out, ref):
        assert torch.equal(u, v)

"""GPU parity of the diagonal-covariance E-step under the bf16 operand contract
(precision="bf16", FGMM_FLAG_BF16) against the oracle restatement of that contract,
gmm_oracle.estep_diag_bf16 (flash_gmm_diag_h100.py:63-130, :159-282, :317-343)."""

import pytest
import torch

from flash_gmm import FlashGMMError, data, diag_estep_into, flash_gmm_estep_diag
from oracle import gmm_oracle as O
from parity import (LOGZ_ATOL_BF16, REL_BF16_STATS_WIDE, assert_close_stats, assert_dense_agrees,
                    logz_atol_bf16, logz_err)

pytestmark = pytest.mark.gpu

KEYS = ("X", "mu", "log_sigma_sq", "log_pi")


def oracle(inp):
    return O.estep_diag_bf16(*[inp[k] for k in KEYS])


def _into(inp, dev, **kw):
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, device=dev)]
    diag_estep_into(*[inp[k].to(dev) for k in KEYS], *out, precision="bf16", **kw)
    torch.cuda.synchronize()
    return out


# Every padded width (32 .. 256), one / two / many component blocks per workgroup,
# partial row tiles and slabs, ragged K and D.
SHAPES = [(1, 1, 1), (33, 1, 1), (31, 3, 5), (200, 5, 7), (129, 33, 32), (1000, 64, 32),
          (2000, 130, 61), (3000, 100, 96), (1500, 40, 96), (5000, 300, 128), (700, 40, 129),
          (4000, 260, 192), (3000, 200, 256), (900, 20, 256), (2048, 1, 64), (4097, 70, 100)]


@pytest.mark.parametrize("N,K,D", SHAPES)
def test_edge_shapes(N, K, D, gpu_device):
    inp = data.diag_clustered(N, K, D, seed=N + K + D)
    print(f"diag bf16 N={N} K={K} D={D}", flush=True)
    got = _into(inp, gpu_device)
    assert_close_stats(got, oracle(inp), f"diag bf16 N={N} K={K} D={D}", logz_atol=LOGZ_ATOL_BF16, bf16_stats=True)


def test_entry_point(gpu_device):
    inp = data.diag_clustered(3000, 64, 48, seed=12)
    got = flash_gmm_estep_diag(*[inp[k].to(gpu_device) for k in KEYS], precision="bf16")
    torch.cuda.synchronize()
    assert_close_stats(got, oracle(inp), "diag bf16 entry", logz_atol=LOGZ_ATOL_BF16, bf16_stats=True)


def test_overlapping_components(gpu_device):
    """Fractional responsibilities: every product's bf16 rounding matters."""
    g = torch.Generator().manual_seed(13)
    N, K, D = 6000, 24, 40
    inp = {"X": torch.randn(N, D, generator=g) * 1.5, "mu": torch.randn(K, D, generator=g) * 0.5,
           "log_sigma_sq": torch.rand(K, D, generator=g) - 0.5,
           "log_pi": torch.log_softmax(torch.randn(K, generator=g), 0)}
    assert_close_stats(_into(inp, gpu_device), oracle(inp), "diag bf16 overlapping",
                       logz_atol=LOGZ_ATOL_BF16, bf16_stats=True)


def test_headline_shape_mid_size(gpu_device):
    inp = data.diag_clustered(32768, 1024, 96, seed=2)
    assert_close_stats(_into(inp, gpu_device), oracle(inp), "diag bf16 K1024 D96",
                       logz_atol=LOGZ_ATOL_BF16, bf16_stats=True)


@pytest.mark.parametrize("N,K,D", [(12000, 1024, 96), (7777, 300, 61), (5000, 64, 32), (3000, 100, 200)])
def test_need_masks_agree_with_dense(N, K, D, gpu_device):
    """Up to D = 128 pass 1 writes need masks and the gathering pass 2 adds the needed
    rows' terms; FGMM_FLAG_DENSE runs every row of every block: logZ bitwise, the
    statistics to 1e-5 (other groupings of the same nonzero terms).  Above D = 128
    (no masks) skipping zero steps is bitwise the dense run."""
    inp = data.diag_clustered(N, K, D, seed=4)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device, dense=True)
    assert_dense_agrees(a, b, bitwise=D > 128)
    assert_close_stats(a, oracle(inp), f"diag bf16 gather N={N} K={K} D={D}", logz_atol=LOGZ_ATOL_BF16,
                       bf16_stats=True)


def test_phase_split_and_accumulate(gpu_device):
    """PHASE1 then PHASE2 equals one call bitwise; ACCUMULATE over chunks equals one call."""
    from flash_gmm import _lib
    inp = data.diag_clustered(9000, 128, 64, seed=10)
    dev = gpu_device
    ref = _into(inp, dev)
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    L = _lib.lib()
    ws = torch.empty(L.fgmm_diag_workspace_bytes_ex(N, K, D, _lib.FLAG_BF16), dtype=torch.uint8, device=dev)
    args = [inp[k].to(dev) for k in KEYS]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, device=dev)]
    diag_estep_into(*args, *out, workspace=ws, phase=1, precision="bf16")
    diag_estep_into(*args, None, *out[1:], workspace=ws, phase=2, precision="bf16")
    torch.cuda.synchronize()
    for u, v in zip(out, ref):
        assert torch.equal(u, v)
    nk = torch.zeros(K, device=dev)
    ma = torch.zeros(K, D, device=dev)
    sg = torch.zeros(K, D, device=dev)
    for n0 in range(0, N, 2500):
        diag_estep_into(args[0][n0:n0 + 2500], *args[1:], None, nk, ma, sg, accumulate=True,
                        precision="bf16")
    torch.cuda.synchronize()
    torch.testing.assert_close(nk, ref[1], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(ma, ref[2], rtol=1e-5, atol=1e-5 * float(ref[2].abs().max()))
    torch.testing.assert_close(sg, ref[3], rtol=1e-5, atol=1e-4 * float(ref[3].abs().max()))


def test_deterministic(gpu_device):
    inp = data.diag_clustered(20000, 512, 96, seed=6)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_bad_precision_string(gpu_device):
    inp = data.diag_clustered(10, 4, 8, seed=11)
    with pytest.raises(FlashGMMError):
        flash_gmm_estep_diag(*[inp[k].to(gpu_device) for k in KEYS], precision="fp16")


# Above D = 256 the contract stores the log-joint (pass 1 tiled over components, pass 2
# from the stored rows per range of 128 dimensions): GloVe-300 and GIST-960 widths, one
# past the narrow kernels, a partial last range and component tile, K = 1.
WIDE_SHAPES = [(1000, 40, 257), (3000, 100, 300), (2000, 130, 960), (700, 33, 1100), (65, 1, 640)]


@pytest.mark.parametrize("N,K,D", WIDE_SHAPES)
def test_above_256_against_oracle(N, K, D, gpu_device):
    print(f"diag bf16 wide N={N} K={K} D={D}", flush=True)
    inp = data.diag_clustered(N, K, D, seed=N + K + D)
    got, ref = _into(inp, gpu_device), oracle(inp)
    atol = logz_atol_bf16(O.estep_diag_bf16(*[inp[k] for k in KEYS], dtype=torch.float32)[0], ref[0], D)
    print(f"max |logZ - oracle| {logz_err(got[0], ref[0]):.2e}, bound {atol:.2e}", flush=True)
    assert_close_stats(got, ref, f"diag bf16 N={N} K={K} D={D}", logz_atol=atol, bf16_stats=True,
                       bf16_rel=REL_BF16_STATS_WIDE)


def test_above_256_dense_and_phase_split(gpu_device):
    """FGMM_FLAG_DENSE and PHASE1-then-PHASE2 give the single call's bits at D = 300."""
    from flash_gmm import _lib, diag_estep_into
    N, K, D = 3000, 70, 300
    inp = data.diag_clustered(N, K, D, seed=31)
    dev = gpu_device
    ref = _into(inp, dev)
    for u, v in zip(_into(inp, dev, dense=True), ref):
        assert torch.equal(u, v)
    L = _lib.lib()
    ws = torch.empty(L.fgmm_diag_workspace_bytes_ex(N, K, D, _lib.FLAG_BF16), dtype=torch.uint8, device=dev)
    args = [inp[k].to(dev) for k in KEYS]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, device=dev)]
    diag_estep_into(*args, *out, workspace=ws, phase=1, precision="bf16")
    diag_estep_into(*args, None, *out[1:], workspace=ws, phase=2, precision="bf16")
    torch.cuda.synchronize()
    for u, v in zip(out, ref):
        assert torch.equal(u, v)

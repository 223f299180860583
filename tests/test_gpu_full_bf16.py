"""GPU parity of the full-covariance E-step under the bf16 operand contract
(precision="bf16", FGMM_FLAG_BF16) against the oracle restatement of that contract,
gmm_oracle.estep_full_bf16 (flash_gmm_full_h100.py:71-228, :289-298).  sig_outer is
checked element-wise like the fp32 path's (it is not symmetric under this contract)."""

import pytest
import torch

from flash_gmm import FlashGMMError, data, flash_gmm_estep_full, full_estep_into
from oracle import gmm_oracle as O
from parity import LOGZ_ATOL_BF16, assert_close_stats

pytestmark = pytest.mark.gpu

KEYS = ("X", "mu", "prec_chol", "log_pi")


def oracle(inp):
    return O.estep_full_bf16(*[inp[k] for k in KEYS])


def _into(inp, dev, **kw):
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, D, device=dev)]
    full_estep_into(*[inp[k].to(dev) for k in KEYS], *out, precision="bf16", **kw)
    torch.cuda.synchronize()
    return out


# Every padded width (32 .. 128), component counts that leave workgroup slots empty,
# partial row tiles and slabs, ragged D.
SHAPES = [(1, 1, 1), (33, 5, 3), (500, 12, 16), (300, 7, 64), (1000, 33, 40), (129, 4, 32),
          (2000, 9, 63), (400, 9, 65), (600, 11, 96), (300, 5, 100), (500, 7, 128), (3, 2, 127),
          (5000, 2, 48)]


@pytest.mark.parametrize("N,K,D", SHAPES)
def test_edge_shapes(N, K, D, gpu_device):
    inp = data.full_clustered(N, K, D, seed=N + K + D)
    print(f"full bf16 N={N} K={K} D={D}", flush=True)
    assert_close_stats(_into(inp, gpu_device), oracle(inp), f"full bf16 N={N} K={K} D={D}",
                       logz_atol=LOGZ_ATOL_BF16, bf16_stats=True)


def _overlapping(N, K, D, seed):
    """Heavily overlapping components, so that responsibilities are fractional."""
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(K, D, D, generator=g, dtype=torch.float64)
    sigma = A @ A.transpose(1, 2) / D + 0.5 * torch.eye(D, dtype=torch.float64)
    return {"X": torch.randn(N, D, generator=g) * 1.5, "mu": torch.randn(K, D, generator=g) * 0.5,
            "prec_chol": torch.linalg.cholesky(torch.linalg.inv(sigma)).float(),
            "log_pi": torch.log_softmax(torch.randn(K, generator=g), 0)}


def test_entry_point_and_asymmetry(gpu_device):
    inp = _overlapping(4000, 16, 32, seed=12)
    got = flash_gmm_estep_full(*[inp[k].to(gpu_device) for k in KEYS], precision="bf16")
    torch.cuda.synchronize()
    ref = oracle(inp)
    assert_close_stats(got, ref, "full bf16 entry", logz_atol=LOGZ_ATOL_BF16, bf16_stats=True)
    # The contract's sig_outer is not symmetric, and the kernel reproduces that.
    s = got[3].double().cpu()
    assert (s - s.transpose(1, 2)).abs().max() > 0
    torch.testing.assert_close(s - s.transpose(1, 2), ref[3] - ref[3].transpose(1, 2), rtol=0,
                               atol=1e-4 * float(ref[3].abs().max()))


def test_headline_shape_mid_size(gpu_device):
    inp = data.full_clustered(20000, 256, 64, seed=3)
    assert_close_stats(_into(inp, gpu_device), oracle(inp), "full bf16 K256 D64", logz_atol=LOGZ_ATOL_BF16, bf16_stats=True)


@pytest.mark.parametrize("N,K,D", [(12000, 256, 64), (3000, 30, 96), (5000, 8, 32), (2000, 6, 128)])
def test_zero_step_skip_is_bitwise_dense(N, K, D, gpu_device):
    inp = data.full_clustered(N, K, D, seed=4)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device, dense=True)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_phase_split_and_accumulate(gpu_device):
    """PHASE1 then PHASE2 equals one call bitwise; ACCUMULATE over chunks equals one call."""
    from flash_gmm import _lib
    inp = data.full_clustered(9000, 24, 48, seed=10)
    dev = gpu_device
    ref = _into(inp, dev)
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    L = _lib.lib()
    ws = torch.empty(L.fgmm_full_workspace_bytes_ex(N, K, D, _lib.FLAG_BF16), dtype=torch.uint8, device=dev)
    args = [inp[k].to(dev) for k in KEYS]
    out = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, D, device=dev)]
    full_estep_into(*args, *out, workspace=ws, phase=1, precision="bf16")
    full_estep_into(*args, None, *out[1:], workspace=ws, phase=2, precision="bf16")
    torch.cuda.synchronize()
    for u, v in zip(out, ref):
        assert torch.equal(u, v)
    nk = torch.zeros(K, device=dev)
    ma = torch.zeros(K, D, device=dev)
    sg = torch.zeros(K, D, D, device=dev)
    for n0 in range(0, N, 2500):
        full_estep_into(args[0][n0:n0 + 2500], *args[1:], None, nk, ma, sg, accumulate=True,
                        precision="bf16")
    torch.cuda.synchronize()
    torch.testing.assert_close(nk, ref[1], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(ma, ref[2], rtol=1e-5, atol=1e-5 * float(ref[2].abs().max()))
    torch.testing.assert_close(sg, ref[3], rtol=1e-5, atol=1e-5 * float(ref[3].abs().max()))


def test_deterministic(gpu_device):
    inp = data.full_clustered(20000, 64, 64, seed=6)
    a = _into(inp, gpu_device)
    b = _into(inp, gpu_device)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_bad_precision_string(gpu_device):
    inp = data.full_clustered(10, 4, 8, seed=11)
    with pytest.raises(FlashGMMError):
        flash_gmm_estep_full(*[inp[k].to(gpu_device) for k in KEYS], precision="fp16")


def test_log_joint_beyond_16gib_runs_in_row_chunks(gpu_device):
    """N x K x 4 bytes above 16 GiB: the library splits the call into row chunks of
    16 GiB / (4 K) rows on one workspace.  The result equals explicit calls on the same
    boundaries (the first overwriting, the second accumulating) bit for bit, logZ of
    sampled rows in both chunks matches the oracle, and a phase split is refused."""
    from flash_gmm import _lib
    dev = gpu_device
    K, D = 1024, 8
    chunk = (16 << 30) // (K * 32 * 4) // 8 * 8 * 32          # rows per 16 GiB of log-joint
    N = chunk + 3000
    assert N * K * 4 > 16 << 30
    print(f"full bf16 chunked N={N} K={K} D={D} chunk={chunk}", flush=True)
    inp = data.full_clustered(N, K, D, seed=21, device=dev)
    L = _lib.lib()
    assert L.fgmm_full_workspace_bytes_ex(N, K, D, _lib.FLAG_BF16) == \
        L.fgmm_full_workspace_bytes_ex(chunk, K, D, _lib.FLAG_BF16)
    args = [inp[k] for k in KEYS]
    got = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, D, device=dev)]
    full_estep_into(*args, *got, precision="bf16")
    ref = [torch.empty(N, device=dev), torch.empty(K, device=dev), torch.empty(K, D, device=dev),
           torch.empty(K, D, D, device=dev)]
    full_estep_into(args[0][:chunk], *args[1:], ref[0][:chunk], *ref[1:], precision="bf16")
    full_estep_into(args[0][chunk:], *args[1:], ref[0][chunk:], *ref[1:], accumulate=True, precision="bf16")
    torch.cuda.synchronize()
    for u, v in zip(got, ref):
        assert torch.equal(u, v)
    assert abs(got[1].double().sum().item() - N) <= 1e-4 * N
    rows = torch.cat([torch.arange(0, 512), torch.arange(chunk - 256, chunk + 256), torch.arange(N - 512, N)])
    sub = {k: v.cpu() for k, v in inp.items()}
    sub["X"] = sub["X"][rows]
    lz = O.estep_full_bf16(*[sub[k] for k in KEYS])[0]
    assert (got[0].cpu()[rows].double() - lz).abs().max().item() <= LOGZ_ATOL_BF16
    with pytest.raises(FlashGMMError):
        full_estep_into(*args, *got, phase=1, precision="bf16")

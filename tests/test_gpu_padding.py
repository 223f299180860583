"""Rows of X whose stride is wider than D, with NaN in the columns between D and the
stride, through the C ABI: no kernel may read a value past column D.  The row loads of
the passes select their addresses instead of branching, so a lane with nothing to read
loads a neighbouring in-bounds vector and must drop it; this pins that for widths that
end inside a 4-float vector (D % 4 != 0), inside a 16-dimension chunk, and past the
component-tiled width, on every plan."""

import os
import sys

import pytest
import torch

from flash_gmm import _lib, data
from oracle import gmm_oracle as O

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from parity import LOGZ_ATOL_BF16, assert_close_stats, logz_atol_fp32  # noqa: E402

pytestmark = pytest.mark.gpu


def _padded(X, dev, extra=12):
    """X on the device with a row stride of round_up(D, 4) + extra floats, NaN past D."""
    N, D = X.shape
    ld = (D + 3) // 4 * 4 + extra
    big = torch.full((N, ld), float("nan"), device=dev)
    big[:, :D] = X.to(dev)
    return big, ld


def _outs(N, K, D, dev, sig_shape):
    nan = float("nan")
    return [torch.full((N,), nan, device=dev), torch.full((K,), nan, device=dev),
            torch.full((K, D), nan, device=dev), torch.full(sig_shape, nan, device=dev)]


def _iso(inp, dev, flags):
    L = _lib.lib()
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    Xp, ld = _padded(inp["X"], dev)
    mu, lss, lpi = (inp[k].to(dev).contiguous() for k in ("mu", "log_sigma_sq", "log_pi"))
    o = _outs(N, K, D, dev, (K,))
    ws = torch.empty(max(1, L.fgmm_iso_workspace_bytes_ex(N, K, D, flags)), dtype=torch.uint8, device=dev)
    st = L.fgmm_iso_estep_f32(Xp.data_ptr(), ld, N, D, mu.data_ptr(), D, K, lss.data_ptr(), lpi.data_ptr(),
                              *[t.data_ptr() for t in o], ws.data_ptr(), ws.numel(), flags,
                              _lib.stream_handle(dev))
    _lib.check(st, "iso padded")
    torch.cuda.synchronize()
    return o


def _diag(inp, dev, flags):
    L = _lib.lib()
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    Xp, ld = _padded(inp["X"], dev)
    mu, lss, lpi = (inp[k].to(dev).contiguous() for k in ("mu", "log_sigma_sq", "log_pi"))
    o = _outs(N, K, D, dev, (K, D))
    ws = torch.empty(max(1, L.fgmm_diag_workspace_bytes_ex(N, K, D, flags)), dtype=torch.uint8, device=dev)
    st = L.fgmm_diag_estep_f32(Xp.data_ptr(), ld, N, D, mu.data_ptr(), D, K, lss.data_ptr(), D, lpi.data_ptr(),
                               *[t.data_ptr() for t in o], ws.data_ptr(), ws.numel(), flags,
                               _lib.stream_handle(dev))
    _lib.check(st, "diag padded")
    torch.cuda.synchronize()
    return o


def _full(inp, dev, flags):
    L = _lib.lib()
    N, D = inp["X"].shape
    K = inp["mu"].shape[0]
    Xp, ld = _padded(inp["X"], dev)
    mu, pc, lpi = (inp[k].to(dev).contiguous() for k in ("mu", "prec_chol", "log_pi"))
    o = _outs(N, K, D, dev, (K, D, D))
    ws = torch.empty(max(1, L.fgmm_full_workspace_bytes_ex(N, K, D, flags)), dtype=torch.uint8, device=dev)
    st = L.fgmm_full_estep_f32(Xp.data_ptr(), ld, N, D, mu.data_ptr(), D, K, pc.data_ptr(), lpi.data_ptr(),
                               *[t.data_ptr() for t in o], ws.data_ptr(), ws.numel(), flags,
                               _lib.stream_handle(dev))
    _lib.check(st, "full padded")
    torch.cuda.synchronize()
    return o


PLANS = {"default": 0, "dense": _lib.FLAG_DENSE, "stored": _lib.FLAG_STORE_LOGJOINT}


@pytest.mark.parametrize("plan", list(PLANS))
@pytest.mark.parametrize("N,K,D", [(6000, 200, 99), (6000, 200, 100), (3000, 96, 50), (2000, 64, 203)])
def test_iso_padding_is_never_read(N, K, D, plan, gpu_device):
    inp = data.iso_clustered(N, K, D, seed=D + 3)
    args = [inp[k] for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    ref = O.estep_iso(*args)
    got = _iso(inp, gpu_device, PLANS[plan])
    atol = logz_atol_fp32(O.estep_iso(*args, dtype=torch.float32)[0] if D > 128 else None, ref[0], D)
    assert_close_stats(got, ref, f"iso padded D={D} {plan}", logz_atol=atol)


@pytest.mark.parametrize("N,K,D", [(6000, 200, 99), (3000, 96, 50)])
def test_iso_bf16_padding_is_never_read(N, K, D, gpu_device):
    inp = data.iso_clustered(N, K, D, seed=D + 5)
    ref = O.estep_iso_bf16(*[inp[k] for k in ("X", "mu", "log_sigma_sq", "log_pi")])
    got = _iso(inp, gpu_device, _lib.FLAG_BF16)
    assert_close_stats(got, ref, f"iso bf16 padded D={D}", logz_atol=LOGZ_ATOL_BF16)


@pytest.mark.parametrize("plan", list(PLANS))
@pytest.mark.parametrize("N,K,D", [(5000, 128, 99), (3000, 64, 50), (2000, 64, 203)])
def test_diag_padding_is_never_read(N, K, D, plan, gpu_device):
    inp = data.diag_clustered(N, K, D, seed=D + 7)
    args = [inp[k] for k in ("X", "mu", "log_sigma_sq", "log_pi")]
    ref = O.estep_diag(*args)
    got = _diag(inp, gpu_device, PLANS[plan])
    atol = logz_atol_fp32(O.estep_diag(*args, dtype=torch.float32)[0] if D > 128 else None, ref[0], D)
    assert_close_stats(got, ref, f"diag padded D={D} {plan}", logz_atol=atol)


@pytest.mark.parametrize("plan", ["default", "stored"])
@pytest.mark.parametrize("N,K,D", [(3000, 32, 50), (2000, 16, 99), (1500, 8, 150)])
def test_full_padding_is_never_read(N, K, D, plan, gpu_device):
    """Above D = 128 the full model's stored plan is not offered: a call that asks for it
    (FGMM_FLAG_STORE_LOGJOINT) runs the default plan, and gives its bits exactly."""
    inp = data.full_clustered(N, K, D, seed=D + 9)
    args = [inp[k] for k in ("X", "mu", "prec_chol", "log_pi")]
    ref = O.estep_full(*args)
    got = _full(inp, gpu_device, PLANS[plan])
    atol = logz_atol_fp32(O.estep_full(*args, dtype=torch.float32)[0] if D > 128 else None, ref[0], D)
    assert_close_stats(got, ref, f"full padded D={D} {plan}", logz_atol=atol)
    if plan == "stored" and D > 128:
        default = _full(inp, gpu_device, PLANS["default"])
        for u, v in zip(got, default):
            assert torch.equal(u, v)

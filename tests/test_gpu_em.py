"""GPU M-step, in-memory EM and the streaming EM driver."""

import math
import os

import numpy as np
import pytest
import torch

from flash_gmm import (FlashGMMError, SynthIsoSource, data, em_diag, em_full, em_iso, flash_gmm_estep,
                       flash_gmm_estep_diag, flash_gmm_estep_full, mstep_diag, mstep_full, mstep_iso,
                       stream_em_iso)
from oracle import gmm_oracle as O

pytestmark = pytest.mark.gpu


def _params(K, D, seed, dev):
    g = torch.Generator().manual_seed(seed)
    centres = torch.randn(K, D, generator=g) * 2
    mu = (centres + 0.5 * torch.randn(K, D, generator=g)).to(dev)
    lss = torch.zeros(K, device=dev)
    lpi = torch.full((K,), -math.log(K), device=dev)
    return centres, mu, lss, lpi


@pytest.mark.parametrize("exact", [False, True])
def test_mstep_matches_readme_formulas(exact, gpu_device):
    inp = data.iso_clustered(4000, 40, 24, seed=21)
    dev = gpu_device
    X, mu, lss, lpi = (inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    _, Nk, mu_acc, sig = flash_gmm_estep(X, mu, lss, lpi)
    mu_old = mu.clone()
    mstep_iso(Nk, mu_acc, sig, 4000, mu, lss, lpi, exact_variance=exact)
    torch.cuda.synchronize()
    pi, m, s2 = O.mstep_iso(Nk.double().cpu(), mu_acc.double().cpu(), sig.double().cpu(), 4000, 24)
    if exact:
        s2 = s2 - ((m - mu_old.double().cpu()) ** 2).sum(1) / 24
    torch.testing.assert_close(mu.double().cpu(), m, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(lss.double().cpu(), torch.log(s2), rtol=0, atol=1e-6)
    torch.testing.assert_close(lpi.double().cpu(), torch.log(pi), rtol=0, atol=1e-6)


def test_mstep_empty_component_keeps_parameters(gpu_device):
    dev = gpu_device
    K, D = 4, 8
    Nk = torch.tensor([10.0, 0.0, 5.0, 0.0], device=dev)
    mu_acc = torch.randn(K, D, device=dev)
    sig = torch.rand(K, device=dev) * 100
    mu = torch.randn(K, D, device=dev)
    lss = torch.full((K,), 0.3, device=dev)
    lpi = torch.zeros(K, device=dev)
    mu0 = mu.clone()
    mstep_iso(Nk, mu_acc, sig, 15, mu, lss, lpi, var_floor=1e-3)
    torch.cuda.synchronize()
    assert torch.equal(mu[1], mu0[1]) and torch.equal(mu[3], mu0[3])
    assert float(lss[1]) == pytest.approx(0.3) and math.isinf(float(lpi[1]))
    assert float(lpi[0]) == pytest.approx(math.log(10 / 15), abs=1e-6)


def test_em_loglik_is_non_decreasing(gpu_device):
    inp = data.iso_clustered(20000, 32, 16, seed=22)
    dev = gpu_device
    X, mu, lss, lpi = (inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    ll = em_iso(X, mu, lss, lpi, 6, exact_variance=True)
    assert all(b >= a - 1e-6 * abs(a) for a, b in zip(ll, ll[1:])), ll


def _stream_vs_memory(dev, N, K, D, chunk, iters, source_kind):
    centres, mu, lss, lpi = _params(K, D, 23, dev)
    src = SynthIsoSource(centres.numpy(), seed=4)
    X = torch.from_numpy(src.rows(0, N)).to(dev)
    mu_m, lss_m, lpi_m = mu.clone(), lss.clone(), lpi.clone()
    ll_m = em_iso(X, mu_m, lss_m, lpi_m, iters)
    source = src if source_kind == "native" else (lambda r0, n: src.rows(r0, n))
    rep = stream_em_iso(source, N, mu, lss, lpi, iterations=iters, chunk_rows=chunk)
    torch.cuda.synchronize()
    torch.testing.assert_close(mu, mu_m, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(lss, lss_m, rtol=0, atol=1e-4)
    torch.testing.assert_close(lpi, lpi_m, rtol=0, atol=1e-4)
    np.testing.assert_allclose(rep["loglik"], ll_m, rtol=1e-6)
    assert rep["iterations"] == iters and rep["device_bytes"] > 0
    return rep


def test_stream_em_matches_in_memory_native_source(gpu_device):
    rep = _stream_vs_memory(gpu_device, 200_000, 64, 32, 48_000, 2, "native")
    assert rep["total_ms"] >= rep["source_ms"]


def test_stream_em_python_source_and_odd_dimension(gpu_device):
    _stream_vs_memory(gpu_device, 30_000, 20, 30, 7_000, 2, "python")


def test_stream_em_source_error_is_reported(gpu_device):
    dev = gpu_device
    centres, mu, lss, lpi = _params(8, 16, 24, dev)
    src = SynthIsoSource(centres.numpy(), seed=4)

    def failing(row0, n):
        if row0 >= 20_000:
            raise RuntimeError("disk went away")
        return src.rows(row0, n)

    with pytest.raises(FlashGMMError, match="row source"):
        stream_em_iso(failing, 50_000, mu, lss, lpi, iterations=1, chunk_rows=10_000)
    # the driver released its resources: a following call works
    rep = stream_em_iso(src, 50_000, mu, lss, lpi, iterations=1, chunk_rows=10_000)
    assert rep["iterations"] == 1


@pytest.mark.parametrize("exact", [False, True])
def test_diag_mstep_matches_oracle(exact, gpu_device):
    inp = data.diag_clustered(5000, 30, 20, seed=31)
    dev = gpu_device
    X, mu, lss, lpi = (inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    _, Nk, mu_acc, sig = flash_gmm_estep_diag(X, mu, lss, lpi)
    mu_old = mu.clone()
    mstep_diag(Nk, mu_acc, sig, 5000, mu, lss, lpi, exact_variance=exact)
    torch.cuda.synchronize()
    pi, m, var = O.mstep_diag(Nk.double().cpu(), mu_acc.double().cpu(), sig.double().cpu(), 5000)
    if exact:
        var = var - (m - mu_old.double().cpu()) ** 2
    torch.testing.assert_close(mu.double().cpu(), m, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(lss.double().cpu(), torch.log(var), rtol=0, atol=1e-6)
    torch.testing.assert_close(lpi.double().cpu(), torch.log(pi), rtol=0, atol=1e-6)


@pytest.mark.parametrize("D", [16, 64, 100, 128, 160, 256, 300])
def test_full_mstep_matches_oracle(D, gpu_device):
    """Up to D = 128 the fp64 matrices sit in LDS; above, in stream-ordered device scratch."""
    # every component holds well over D rows, so each Sigma_k is positive definite
    N = 24000 if D <= 128 else 60000
    inp = data.full_clustered(N, 12, D, seed=32)
    dev = gpu_device
    X, mu, L, lpi = (inp[k].to(dev) for k in ("X", "mu", "prec_chol", "log_pi"))
    _, Nk, mu_acc, so = flash_gmm_estep_full(X, mu, L, lpi)
    assert float(Nk.min()) > 2 * D
    info = torch.zeros(1, dtype=torch.int32, device=dev)
    mstep_full(Nk, mu_acc, so, N, mu, L, lpi, reg_covar=1e-6, info=info)
    torch.cuda.synchronize()
    assert int(info.item()) == 0
    pi, m, cov = O.mstep_full(Nk.double().cpu(), mu_acc.double().cpu(), so.double().cpu(), N)
    cov = 0.5 * (cov + cov.transpose(1, 2)) + 1e-6 * torch.eye(D, dtype=torch.float64)
    ref_L = O.prec_chol_from_cov(cov)
    torch.testing.assert_close(mu.double().cpu(), m, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(lpi.double().cpu(), torch.log(pi), rtol=0, atol=1e-6)
    got = L.double().cpu()
    assert torch.all(torch.triu(got, 1) == 0)
    torch.testing.assert_close(got, ref_L, rtol=1e-5, atol=1e-5 * float(ref_L.abs().max()))


def test_full_mstep_counts_indefinite_covariance(gpu_device):
    dev = gpu_device
    K, D = 2, 8
    Nk = torch.tensor([10.0, 10.0], device=dev)
    mu_acc = torch.zeros(K, D, device=dev)
    so = torch.zeros(K, D, D, device=dev)
    so[0] = 10 * torch.eye(D, device=dev)          # Sigma = I
    so[1, 0, 0] = -10.0                              # Sigma with a negative variance
    mu = torch.zeros(K, D, device=dev)
    L = torch.empty(K, D, D, device=dev)
    lpi = torch.zeros(K, device=dev)
    info = torch.zeros(1, dtype=torch.int32, device=dev)
    mstep_full(Nk, mu_acc, so, 20, mu, L, lpi, reg_covar=1e-3, info=info)
    torch.cuda.synchronize()
    assert int(info.item()) == 1          # one component, counted once
    torch.testing.assert_close(L[0], torch.eye(D, device=dev) / (1 + 1e-3) ** 0.5)


def test_em_diag_and_full_loglik_non_decreasing(gpu_device):
    dev = gpu_device
    inp = data.diag_clustered(20000, 24, 16, seed=33)
    X, mu, lss, lpi = (inp[k].to(dev) for k in ("X", "mu", "log_sigma_sq", "log_pi"))
    ll = em_diag(X, mu, lss, lpi, 6, exact_variance=True)
    assert all(b >= a - 1e-6 * abs(a) for a, b in zip(ll, ll[1:])), ll
    inp = data.full_clustered(20000, 10, 12, seed=34)
    X, mu, L, lpi = (inp[k].to(dev) for k in ("X", "mu", "prec_chol", "log_pi"))
    ll = em_full(X, mu, L, lpi, 6, reg_covar=1e-6)
    assert all(b >= a - 1e-6 * abs(a) for a, b in zip(ll, ll[1:])), ll


def test_stream_em_c5_shape_against_the_oracle(gpu_device):
    """The streaming driver at the shape of the 1e9-row workload (K=1024, D=128), on
    N=2M rows in four 512K-row chunks, two iterations: the parameters it applies and
    the log-likelihood it reports for each iteration against the float64 oracle's
    E-step over the same host rows followed by the README M-step (README.md:59-61),
    all to 1e-4 (mu norm-wise, log sigma^2 and log pi absolute)."""
    dev = gpu_device
    K, D, N, chunk = 1024, 128, 2_000_000, 1 << 19
    centres, mu, lss, lpi = _params(K, D, 25, dev)
    src = SynthIsoSource(centres.numpy(), seed=4)
    params = [t.cpu().double().clone() for t in (mu, lss, lpi)]
    rep = stream_em_iso(src, N, mu, lss, lpi, iterations=2, chunk_rows=chunk)
    torch.cuda.synchronize()
    assert rep["iterations"] == 2
    print("C5-shape oracle over 2M streamed rows, two iterations (float64, CPU)", flush=True)
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    X = torch.from_numpy(src.rows(0, N))
    for it in range(2):
        m0, l0, p0 = params
        logZ, Nk, mu_acc, sig = O.estep_iso(X, m0, l0, p0)
        assert float(Nk.min()) > 100      # every component is populated: no empty-component rule
        pi, m, s2 = O.mstep_iso(Nk, mu_acc, sig, N, D)
        params = [m, torch.log(s2), torch.log(pi)]
        ll = float(logZ.sum())
        print(f"iteration {it}: loglik {rep['loglik'][it]:.6e} (oracle {ll:.6e})", flush=True)
        assert abs(rep["loglik"][it] - ll) <= 1e-4 * N
    m, ls, lp = params
    scale = float(m.abs().max())
    assert float((mu.double().cpu() - m).abs().max()) <= 1e-4 * scale
    assert float((lss.double().cpu() - ls).abs().max()) <= 1e-4
    assert float((lpi.double().cpu() - lp).abs().max()) <= 1e-4


@pytest.mark.parametrize("iters", [1, 2])
def test_stream_em_c5_chunking_matches_in_memory(iters, gpu_device):
    """The streaming workload's own chunking: K=1024, D=128, chunk_rows = 2^24 (8 GiB
    pinned buffers), N = 20M rows (one full chunk and one partial), one and two
    iterations (the second overlaps the next iteration's first copies with the
    M-step).  Each iteration's parameters and log-likelihood against the in-memory
    E-step plus device M-step on the same rows, to 1e-5."""
    dev = gpu_device
    K, D, N, chunk = 1024, 128, 20_000_000, 1 << 24
    centres, mu, lss, lpi = _params(K, D, 26, dev)
    src = SynthIsoSource(centres.numpy(), seed=4)
    print(f"C5 chunking: {N} rows in chunks of {chunk}, {iters} iteration(s)", flush=True)
    X = torch.from_numpy(src.rows(0, N)).to(dev)
    mu_m, lss_m, lpi_m = mu.clone(), lss.clone(), lpi.clone()
    ll_m = em_iso(X, mu_m, lss_m, lpi_m, iters)
    del X
    torch.cuda.empty_cache()
    rep = stream_em_iso(src, N, mu, lss, lpi, iterations=iters, chunk_rows=chunk)
    torch.cuda.synchronize()
    assert rep["iterations"] == iters
    scale = float(mu_m.abs().max())
    err_mu = float((mu - mu_m).abs().max()) / scale
    err_ls = float((lss - lss_m).abs().max())
    err_lp = float((lpi - lpi_m).abs().max())
    print(f"streamed vs in-memory: mu {err_mu:.2e} (norm-wise), log sigma^2 {err_ls:.2e}, log pi {err_lp:.2e}",
          flush=True)
    assert err_mu <= 1e-5 and err_ls <= 1e-5 and err_lp <= 1e-5
    np.testing.assert_allclose(rep["loglik"], ll_m, rtol=1e-6)

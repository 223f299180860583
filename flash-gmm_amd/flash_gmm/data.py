"""Seeded synthetic GMM workloads.

The reference ships no datasets; its only workload is the smoke benchmark at
flash_gmm.py:224-234 (X ~ N(0, I), mu ~ N(0, I), lss = 0, uniform log pi).
The workloads below are the E-step shapes this package is measured on.  In
"N(0, s I)" the second argument is a variance (N(0, 4I) has std 2).

Every generator takes an explicit ``seed`` and ``device`` and draws from a
``torch.Generator`` on that device, so the same (seed, device) always yields
the same tensors.  CPU and GPU generators produce different streams: parity
tests generate on the CPU and copy to the GPU.  Values that pass through a
transcendental function (variances, log-softmax weights) are computed in
float64 and rounded to float32 once, because float32 vectorised exp/log differ
in the last bit between host CPUs and the golden fixtures identify inputs by
their bytes.
"""

from __future__ import annotations

import math
from typing import Dict

import numpy as np
import torch


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def _randn(g, *shape, device, std=1.0):
    return torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std


def _rand(g, *shape, device, lo=0.0, hi=1.0):
    return torch.rand(*shape, generator=g, device=device, dtype=torch.float32) * (hi - lo) + lo


def _log_softmax(v: torch.Tensor) -> torch.Tensor:
    return torch.log_softmax(v.double(), dim=0).float()


def iso_plain(N: int, K: int, D: int, seed: int = 0, device="cpu") -> Dict[str, torch.Tensor]:
    """X ~ N(0, I), mu ~ N(0, 4I), lss = 0, lpi = -log K (the N=10,000, K=64, D=32 golden case)."""
    g = _gen(device, seed)
    X = _randn(g, N, D, device=device)
    mu = _randn(g, K, D, device=device, std=2.0)
    lss = torch.zeros(K, device=device)
    lpi = torch.full((K,), -math.log(K), device=device)
    return dict(X=X, mu=mu, log_sigma_sq=lss, log_pi=lpi)


def _assign_rows(g, N, K, device, probs=None):
    if probs is None:
        return torch.randint(0, K, (N,), generator=g, device=device)
    return torch.multinomial(probs.to(device), N, replacement=True, generator=g)


def iso_clustered(N: int, K: int, D: int, seed: int = 1, device="cpu",
                  row_chunk: int = 1 << 20) -> Dict[str, torch.Tensor]:
    """Clustered isotropic workload (the N=1M, K=1024, D=128 headline shape).

    centres c ~ N(0, 4I); assignment uniform; X = c[a] + N(0, I);
    mu = c + N(0, 0.25 I); lss ~ U(-0.5, 0.5); lpi = log_softmax(N(0, 1)).
    """
    g = _gen(device, seed)
    c = _randn(g, K, D, device=device, std=2.0)
    mu = c + _randn(g, K, D, device=device, std=0.5)
    lss = _rand(g, K, device=device, lo=-0.5, hi=0.5)
    lpi = _log_softmax(_randn(g, K, device=device))
    X = torch.empty(N, D, device=device, dtype=torch.float32)
    for n0 in range(0, N, row_chunk):
        n1 = min(N, n0 + row_chunk)
        a = _assign_rows(g, n1 - n0, K, device)
        X[n0:n1] = c[a] + _randn(g, n1 - n0, D, device=device)
    return dict(X=X, mu=mu, log_sigma_sq=lss, log_pi=lpi)


def diag_clustered(N: int, K: int, D: int, seed: int = 2, device="cpu",
                   row_chunk: int = 1 << 20) -> Dict[str, torch.Tensor]:
    """Axis-aligned clusters (the N=1M, K=1024, D=96 diagonal shape).

    centres ~ N(0, 4I); per-(k, d) log variance ~ U(-1, 1);
    X = c[a] + exp(0.5 logvar[a]) * N(0, I); mu = c + N(0, 0.25 I);
    lss = logvar (K x D); lpi uniform.
    """
    g = _gen(device, seed)
    c = _randn(g, K, D, device=device, std=2.0)
    logvar = _rand(g, K, D, device=device, lo=-1.0, hi=1.0)
    mu = c + _randn(g, K, D, device=device, std=0.5)
    lpi = torch.full((K,), -math.log(K), device=device)
    X = torch.empty(N, D, device=device, dtype=torch.float32)
    sd = torch.exp(0.5 * logvar.double()).float()
    for n0 in range(0, N, row_chunk):
        n1 = min(N, n0 + row_chunk)
        a = _assign_rows(g, n1 - n0, K, device)
        X[n0:n1] = c[a] + sd[a] * _randn(g, n1 - n0, D, device=device)
    return dict(X=X, mu=mu, log_sigma_sq=logvar, log_pi=lpi)


def full_clustered(N: int, K: int, D: int, seed: int = 3, device="cpu") -> Dict[str, torch.Tensor]:
    """Full-covariance mixture (the N=250K, K=256, D=64 shape).

    A_k ~ N(0, 1) (D x D); Sigma_k = A_k A_k^T / D + 0.1 I;
    prec_chol_k = cholesky(inv(Sigma_k)) computed in float64 on the host and
    rounded to float32 (lower-triangular, L L^T = Sigma^-1, the
    parameterisation of flash_gmm_full_h100.py:238,247-248);
    centres ~ N(0, 4I), mu = centres; lpi = log_softmax(N(0, 0.5));
    X sampled from the mixture with assignment ~ pi.
    """
    g = _gen(device, seed)
    A = torch.randn(K, D, D, generator=g, device=device, dtype=torch.float32)
    # The host-side float64 algebra runs per component in numpy: batched float64
    # products and factorizations through torch's CPU backend have returned a
    # non-positive-definite inverse now and then on some hosts.
    A64 = A.double().cpu().numpy()
    prec = np.empty((K, D, D))
    chs = np.empty((K, D, D))
    for k in range(K):
        s = A64[k] @ A64[k].T / D + 0.1 * np.eye(D)
        chs[k] = np.linalg.cholesky(s)
        prec[k] = np.linalg.cholesky(np.linalg.inv(s))
    prec_chol = torch.from_numpy(prec)
    chol_sigma = torch.from_numpy(chs)
    mu = _randn(g, K, D, device=device, std=2.0)
    lpi = _log_softmax(_randn(g, K, device=device, std=math.sqrt(0.5)))
    a = _assign_rows(g, N, K, device, probs=torch.exp(lpi.double()).float())
    z = _randn(g, N, D, device=device)
    X = torch.empty(N, D, device=device, dtype=torch.float32)
    cs = chol_sigma.float().double().to(device)
    mu64 = mu.double()
    for k in range(K):
        idx = (a == k).nonzero(as_tuple=True)[0]
        if idx.numel():
            X[idx] = (mu64[k] + z[idx].double() @ cs[k].T).float()
    return dict(X=X, mu=mu, prec_chol=prec_chol.float().contiguous().to(device), log_pi=lpi)


def reference_smoke(N: int = 1_000_000, K: int = 1024, D: int = 128, seed: int = 0,
                    device="cpu") -> Dict[str, torch.Tensor]:
    """The reference's own smoke workload shape (flash_gmm.py:228-234)."""
    g = _gen(device, seed)
    X = _randn(g, N, D, device=device)
    mu = _randn(g, K, D, device=device)
    lss = torch.zeros(K, device=device)
    lpi = torch.full((K,), -math.log(K), device=device)
    return dict(X=X, mu=mu, log_sigma_sq=lss, log_pi=lpi)


def diag_reference_smoke(N: int = 1_000_000, K: int = 1024, D: int = 96, seed: int = 0,
                         device="cpu") -> Dict[str, torch.Tensor]:
    """The reference smoke workload's data (flash_gmm.py:228-234: X, mu ~ N(0, I),
    uniform weights) for the diagonal model, with per-dimension variances
    log sigma^2 ~ N(0, 0.2^2): every component is within reach of every row."""
    g = _gen(device, seed)
    X = _randn(g, N, D, device=device)
    mu = _randn(g, K, D, device=device)
    lss = 0.2 * _randn(g, K, D, device=device)
    lpi = torch.full((K,), -math.log(K), device=device)
    return dict(X=X, mu=mu, log_sigma_sq=lss, log_pi=lpi)


def full_reference_smoke(N: int = 250_000, K: int = 256, D: int = 64, seed: int = 0,
                         device="cpu") -> Dict[str, torch.Tensor]:
    """The reference smoke workload's data (flash_gmm.py:228-234: X, mu ~ N(0, I),
    uniform weights) for the full model: Sigma_k = I + 0.2 A_k A_k^T / D with
    A_k ~ N(0, 1), prec_chol_k = cholesky(inv(Sigma_k)) in float64 on the host.
    Every component is within reach of every row."""
    g = _gen(device, seed)
    X = _randn(g, N, D, device=device)
    mu = _randn(g, K, D, device=device)
    A64 = torch.randn(K, D, D, generator=g, device=device, dtype=torch.float32).double().cpu().numpy()
    prec = np.empty((K, D, D))
    for k in range(K):
        s = np.eye(D) + 0.2 * (A64[k] @ A64[k].T) / D
        prec[k] = np.linalg.cholesky(np.linalg.inv(s))
    prec_chol = torch.from_numpy(prec).float().contiguous().to(device)
    lpi = torch.full((K,), -math.log(K), device=device)
    return dict(X=X, mu=mu, prec_chol=prec_chol, log_pi=lpi)


WORKLOADS = {
    # name: (generator, default sizes, default seed)
    "iso_n10k_k64_d32": (iso_plain, dict(N=10_000, K=64, D=32), 0),
    "iso_n1m_k1024_d128": (iso_clustered, dict(N=1_000_000, K=1024, D=128), 1),
    "diag_n1m_k1024_d96": (diag_clustered, dict(N=1_000_000, K=1024, D=96), 2),
    "full_n250k_k256_d64": (full_clustered, dict(N=250_000, K=256, D=64), 3),
    # the reference's own smoke workload (flash_gmm.py:228-234): nearly every
    # responsibility is nonzero, so no accumulation work can be skipped
    "iso_ref_n1m_k1024_d128": (reference_smoke, dict(N=1_000_000, K=1024, D=128), 0),
    # the same dense regime for the diagonal model at its benchmark shape
    "diag_ref_n1m_k1024_d96": (diag_reference_smoke, dict(N=1_000_000, K=1024, D=96), 0),
    "full_ref_n250k_k256_d64": (full_reference_smoke, dict(N=250_000, K=256, D=64), 0),
    # wider shapes (split-dimension accumulation paths)
    "diag_n1m_k256_d256": (diag_clustered, dict(N=1_000_000, K=256, D=256), 5),
    "full_n100k_k64_d128": (full_clustered, dict(N=100_000, K=64, D=128), 6),
    # widths above 128 (GIST-960 and the full model's widest)
    "iso_n1m_k1024_d256": (iso_clustered, dict(N=1_000_000, K=1024, D=256), 1),
    "iso_n1m_k1024_d960": (iso_clustered, dict(N=1_000_000, K=1024, D=960), 1),
    "diag_n1m_k1024_d960": (diag_clustered, dict(N=1_000_000, K=1024, D=960), 2),
    "full_n100k_k64_d256": (full_clustered, dict(N=100_000, K=64, D=256), 6),
}


def make(name: str, device="cpu", seed=None, **sizes) -> Dict[str, torch.Tensor]:
    fn, defaults, dseed = WORKLOADS[name]
    kw = dict(defaults)
    kw.update(sizes)
    return fn(seed=dseed if seed is None else seed, device=device, **kw)

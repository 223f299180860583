"""CPU oracle for the Flash-GMM E-step — TEST INFRASTRUCTURE ONLY.

This module restates the reference's E-step mathematics on the CPU with
PyTorch so that the HIP kernels can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the checker: the product path in ``flash_gmm`` never calls it
and fails loudly when its native library is missing.

Every function is chunked over rows so that the N x K responsibility matrix is
never held whole, and runs in either float64 (the golden) or float32 (the
reference's own arithmetic, used as the CPU baseline).

Parity pinning (what checks each function, see tests/test_oracle.py):

* ``estep_iso`` -- logZ against scipy.stats.multivariate_normal.logpdf +
  scipy.special.logsumexp; all four outputs against sklearn's spherical
  GaussianMixture internals; the expansion form against the direct form;
  invariants (sum Nk = N, sum_k mu_acc = sum_n x_n, the sig_acc identity);
  special cases (K = 1, identical components, far-apart clusters); brute force
  with Python loops on tiny inputs; committed golden vectors.
* ``estep_diag`` -- scipy logpdf with a diagonal covariance, sklearn 'diag'
  internals, brute force, invariants, reduction to ``estep_iso`` when every
  per-dimension variance of a component is equal.
* ``estep_iso_bf16`` -- the bf16 operand contract of the reference's H100 kernels:
  equal to ``estep_iso`` (logZ, Nk, sig_acc) on inputs that are exact in bfloat16
  and within the bf16 rounding of r for mu_acc; an independent scalar-loop
  version with bit-level rounding on tiny inputs.
* ``estep_diag_bf16`` -- the bf16 operand contract of the reference's diagonal
  H100 kernels: equal to ``estep_diag`` (logZ, Nk) when every rounded operand is
  already exact in bfloat16 (weights that are powers of two, x with few
  significant bits) and within the bf16 rounding of r for mu_acc and sig_acc; an
  independent scalar-loop version with bit-level rounding on tiny inputs.
* ``estep_full_bf16`` -- the bf16 operand contract of the reference's full H100
  kernels: equal to ``estep_full`` (logZ, Nk) when x and L are already exact in
  bfloat16, within the bf16 rounding of r (and of r x for sig_outer) for the
  statistics; an independent scalar-loop version on tiny inputs.
* ``estep_full`` -- scipy logpdf with the full covariance recovered from the
  precision Cholesky factor, sklearn 'full' internals, brute force, reduction
  to ``estep_diag`` for diagonal factors.
* ``mstep_*`` -- closed forms against the README formulas, checked by the
  fixed point of an exactly-fitted single component (sample mean, variance and
  covariance); ``prec_chol_from_cov`` by L L^T cov = I, lower-triangularity with a
  positive diagonal, and L = diag(sigma^-1/2) for a diagonal cov.
"""

from __future__ import annotations

import math
from typing import Tuple

import torch

LOG_2PI = 1.8378770664093453  # flash_gmm.py:91
Tensor = torch.Tensor

_DEFAULT_CHUNK = 16384


def _as(t: Tensor, dtype: torch.dtype) -> Tensor:
    return t.detach().to(device="cpu", dtype=dtype)


def iso_log_prob(X: Tensor, mu: Tensor, lss: Tensor, lpi: Tensor,
                 form: str = "expansion") -> Tuple[Tensor, Tensor]:
    """Per-(n, k) log joint ll_nk and squared distance sq_nk for spherical components.

    Follows flash_gmm.py:84-93:
        sq = ||x||^2 - 2 x.mu + ||mu||^2             (form="expansion")
        ll = lpi - 0.5 * sq * exp(-lss) - 0.5 * D * (log2pi + lss)
    ``form="direct"`` evaluates sq as sum_d (x_d - mu_d)^2 instead (no
    cancellation; used for the float64 golden on small inputs).
    """
    D = X.shape[1]
    if form == "expansion":
        x_sq = (X * X).sum(dim=1)                       # flash_gmm.py:85
        mu_sq = (mu * mu).sum(dim=1)                    # flash_gmm.py:86
        xmu = X @ mu.T                                  # flash_gmm.py:87
        sq = x_sq[:, None] - 2.0 * xmu + mu_sq[None, :]  # flash_gmm.py:88
    elif form == "direct":
        sq = ((X[:, None, :] - mu[None, :, :]) ** 2).sum(dim=2)
    else:
        raise ValueError(form)
    inv_s = torch.exp(-lss)                             # flash_gmm.py:90
    ll = lpi[None, :] - 0.5 * sq * inv_s[None, :] - 0.5 * D * (LOG_2PI + lss[None, :])  # :92
    return ll, sq


def estep_iso(X: Tensor, mu: Tensor, log_sigma_sq: Tensor, log_pi: Tensor, *,
              dtype: torch.dtype = torch.float64, form: str = "expansion",
              chunk: int = _DEFAULT_CHUNK) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Isotropic E-step: (logZ, Nk, mu_acc, sig_acc).

    Pass 1 (logZ = logsumexp_k ll) follows flash_gmm.py:84-103; pass 2 follows
    flash_gmm.py:141-166: r = exp(ll - logZ), Nk = sum_n r,
    sig_acc = sum_n r * sq (sq by the same expansion), mu_acc = r^T X.
    Shapes and dtypes follow flash_gmm.py:187-195.
    """
    X, mu = _as(X, dtype), _as(mu, dtype)
    lss, lpi = _as(log_sigma_sq, dtype), _as(log_pi, dtype)
    N, D = X.shape
    K = mu.shape[0]
    logZ = torch.empty(N, dtype=dtype)
    Nk = torch.zeros(K, dtype=dtype)
    mu_acc = torch.zeros(K, D, dtype=dtype)
    sig_acc = torch.zeros(K, dtype=dtype)
    for n0 in range(0, N, chunk):
        x = X[n0:n0 + chunk]
        ll, sq = iso_log_prob(x, mu, lss, lpi, form)
        lz = torch.logsumexp(ll, dim=1)                 # flash_gmm.py:95-102
        logZ[n0:n0 + chunk] = lz
        r = torch.exp(ll - lz[:, None])                 # flash_gmm.py:151
        Nk += r.sum(dim=0)                              # flash_gmm.py:155
        sig_acc += (r * sq).sum(dim=0)                  # flash_gmm.py:156
        mu_acc += r.T @ x                               # flash_gmm.py:161
    return logZ, Nk, mu_acc, sig_acc


LOG2_E = 1.4426950408889634  # flash_gmm_h100.py:247


def bf16_round(t: Tensor) -> Tensor:
    """Round float32 values to bfloat16 (nearest, ties to even), returned as float64."""
    return t.to(torch.float32).to(torch.bfloat16).to(torch.float64)


def estep_iso_bf16(X: Tensor, mu: Tensor, log_sigma_sq: Tensor, log_pi: Tensor, *,
                   chunk: int = _DEFAULT_CHUNK,
                   dtype: torch.dtype = torch.float64) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Isotropic E-step with the bf16 operand contract of flash_gmm_h100.py:247-328.

    X and mu are rounded to bfloat16 for both contractions (:277-284); x_sq is the
    sum of squares of the rounded x (:105-107); mu_sq, ish and c0 come from the
    float32 mu (:286-292); ll2 = c0 - ish x_sq + 2 ish x.mu in log2 units
    (:137-138); r = 2^(ll2 - logZ2); Nk = sum r, sig_acc = sum r (x_sq - 2 x.mu +
    mu_sq) (:210-224); mu_acc = bf16(r)^T x (:230-231); logZ = logZ2 ln 2 (:326).
    Everything except those roundings is float64 here (the reference accumulates
    in float32); ``dtype=torch.float32`` evaluates the same steps in float32 (the
    constants formed in float64 and rounded once), the reference's own arithmetic,
    whose distance from the float64 result bounds what a float32 kernel can reach.
    """
    X32, mu32 = _as(X, torch.float32), _as(mu, torch.float32)
    Xb, mub = bf16_round(X32).to(dtype), bf16_round(mu32).to(dtype)
    lss, lpi = _as(log_sigma_sq, torch.float64), _as(log_pi, torch.float64)
    N, D = X32.shape
    K = mu32.shape[0]
    mu_sq = (mu32.double() ** 2).sum(dim=1)
    ish = 0.5 * torch.exp(-lss) * LOG2_E
    c0 = (lpi - 0.5 * D * (LOG_2PI + lss)) * LOG2_E - ish * mu_sq
    mu_sq, ish, c0 = mu_sq.to(dtype), ish.to(dtype), c0.to(dtype)
    logZ = torch.empty(N, dtype=dtype)
    Nk = torch.zeros(K, dtype=dtype)
    mu_acc = torch.zeros(K, D, dtype=dtype)
    sig_acc = torch.zeros(K, dtype=dtype)
    ln2 = math.log(2.0)
    for n0 in range(0, N, chunk):
        xb = Xb[n0:n0 + chunk]
        x_sq = (xb * xb).sum(dim=1)
        xmu = xb @ mub.T
        ll2 = c0[None, :] - ish[None, :] * x_sq[:, None] + (2.0 * ish[None, :]) * xmu
        lz2 = torch.logsumexp(ll2 * ln2, dim=1) / ln2
        logZ[n0:n0 + chunk] = lz2 * ln2
        r = torch.exp2(ll2 - lz2[:, None])
        Nk += r.sum(dim=0)
        sig_acc += (r * (x_sq[:, None] - 2.0 * xmu + mu_sq[None, :])).sum(dim=0)
        mu_acc += bf16_round(r).to(dtype).T @ xb
    return logZ, Nk, mu_acc, sig_acc


def diag_log_prob(X: Tensor, mu: Tensor, lss: Tensor, lpi: Tensor,
                  form: str = "expansion") -> Tensor:
    """Per-(n, k) log joint for diagonal components (natural-log units).

    The reference works in log2 units with
        inv_sigma_sq = exp(-lss) * 0.5*log2e,  mu_w = mu * inv_sigma_sq
        c0 = (lpi - 0.5*(D*log2pi + sum_d lss)) * log2e - sum_d mu^2 e^{-lss} * 0.5*log2e
        ll2 = c0 - (x^2) . inv_sigma_sq^T + 2 x . mu_w^T
    (flash_gmm_diag_h100.py:332-340, :116-119).  Dividing by log2e gives the
    natural-log form evaluated here.
    """
    D = X.shape[1]
    w = torch.exp(-lss)                                  # (K, D)
    if form == "expansion":
        quad = (X * X) @ w.T - 2.0 * X @ (mu * w).T + (mu * mu * w).sum(dim=1)[None, :]
    elif form == "direct":
        quad = (((X[:, None, :] - mu[None, :, :]) ** 2) * w[None, :, :]).sum(dim=2)
    else:
        raise ValueError(form)
    ll = lpi[None, :] - 0.5 * (D * LOG_2PI + lss.sum(dim=1))[None, :] - 0.5 * quad
    return ll


def estep_diag(X: Tensor, mu: Tensor, log_sigma_sq: Tensor, log_pi: Tensor, *,
               dtype: torch.dtype = torch.float64, form: str = "expansion",
               chunk: int = _DEFAULT_CHUNK) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Diagonal-covariance E-step: (logZ, Nk, mu_acc, sig_acc[K, D]).

    sig_acc[k, d] = sum_n r_nk (x_nd - mu_kd)^2, which the reference finalises
    as rxsq - 2 mu * mu_local + mu^2 * nk (flash_gmm_diag_h100.py:254-260) and
    returns sliced to (K, D) (:380-384).
    """
    X, mu = _as(X, dtype), _as(mu, dtype)
    lss, lpi = _as(log_sigma_sq, dtype), _as(log_pi, dtype)
    N, D = X.shape
    K = mu.shape[0]
    if lss.shape != (K, D):
        raise ValueError(f"log_sigma_sq must be (K, D)=({K}, {D}), got {tuple(lss.shape)}")
    logZ = torch.empty(N, dtype=dtype)
    Nk = torch.zeros(K, dtype=dtype)
    mu_acc = torch.zeros(K, D, dtype=dtype)
    rxsq = torch.zeros(K, D, dtype=dtype)
    for n0 in range(0, N, chunk):
        x = X[n0:n0 + chunk]
        ll = diag_log_prob(x, mu, lss, lpi, form)
        lz = torch.logsumexp(ll, dim=1)
        logZ[n0:n0 + chunk] = lz
        r = torch.exp(ll - lz[:, None])
        Nk += r.sum(dim=0)
        mu_acc += r.T @ x
        rxsq += r.T @ (x * x)
    sig_acc = rxsq - 2.0 * mu * mu_acc + mu * mu * Nk[:, None]
    return logZ, Nk, mu_acc, sig_acc


def diag_bf16_weights(mu: Tensor, log_sigma_sq: Tensor) -> Tuple[Tensor, Tensor]:
    """float32 W1 = exp(-lss) * 0.5 log2e and W2 = mu * W1 of flash_gmm_diag_h100.py:332-333.

    exp is rounded once from float64 (the reference's float32 exp may differ from
    that by an ulp, which moves a bfloat16 rounding only at a tie).
    """
    lss32 = _as(log_sigma_sq, torch.float32)
    e32 = torch.exp(-lss32.double()).float()
    w1 = e32 * torch.tensor(0.5 * LOG2_E, dtype=torch.float32)
    w2 = _as(mu, torch.float32) * w1
    return w1, w2


def estep_diag_bf16(X: Tensor, mu: Tensor, log_sigma_sq: Tensor, log_pi: Tensor, *,
                    chunk: int = _DEFAULT_CHUNK,
                    dtype: torch.dtype = torch.float64) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Diagonal E-step with the bf16 operand contract of flash_gmm_diag_h100.py.

    x and x^2 (squared in float32) are rounded to bfloat16 (:86-88, :238-239), and so
    are W1 and W2 (:332-333, :342-343); c0 comes from the float32 parameters
    (:335-339); ll2 = c0 - bf16(x^2) . bf16(W1) + 2 bf16(x) . bf16(W2) (:116-119,
    :242-244); r = 2^(ll2 - logZ2) (:250); Nk = sum r (:254); mu_acc = bf16(r)^T
    bf16(x) and rxsq = bf16(r)^T bf16(x^2) (:251, :255-256); sig_acc = rxsq -
    2 mu mu_acc + mu^2 Nk (:260); logZ = logZ2 ln 2 (:382).  Rows are partitioned (no slab
    overlap, unlike :220-231).  Everything except the roundings is float64 here
    (the reference accumulates in float32); ``dtype=torch.float32`` evaluates the
    same steps in float32, as estep_iso_bf16 does.
    """
    X32 = _as(X, torch.float32)
    mu64 = _as(mu, torch.float64)
    lss, lpi = _as(log_sigma_sq, torch.float64), _as(log_pi, torch.float64)
    N, D = X32.shape
    K = mu64.shape[0]
    if lss.shape != (K, D):
        raise ValueError(f"log_sigma_sq must be (K, D)=({K}, {D}), got {tuple(lss.shape)}")
    w1, w2 = diag_bf16_weights(mu, log_sigma_sq)
    w1b, w2b = bf16_round(w1).to(dtype), bf16_round(w2).to(dtype)
    c0 = ((lpi - 0.5 * (D * LOG_2PI + lss.sum(dim=1))) * LOG2_E
          - 0.5 * LOG2_E * (mu64 * mu64 * torch.exp(-lss)).sum(dim=1)).to(dtype)
    logZ = torch.empty(N, dtype=dtype)
    Nk = torch.zeros(K, dtype=dtype)
    mu_acc = torch.zeros(K, D, dtype=dtype)
    rxsq = torch.zeros(K, D, dtype=dtype)
    ln2 = math.log(2.0)
    for n0 in range(0, N, chunk):
        x = X32[n0:n0 + chunk]
        xb, xsqb = bf16_round(x).to(dtype), bf16_round(x * x).to(dtype)
        ll2 = c0[None, :] - xsqb @ w1b.T + 2.0 * (xb @ w2b.T)
        lz2 = torch.logsumexp(ll2 * ln2, dim=1) / ln2
        logZ[n0:n0 + chunk] = lz2 * ln2
        r = torch.exp2(ll2 - lz2[:, None])
        rb = bf16_round(r).to(dtype)
        Nk += r.sum(dim=0)
        mu_acc += rb.T @ xb
        rxsq += rb.T @ xsqb
    m = mu64.to(dtype)
    sig_acc = rxsq - 2.0 * m * mu_acc + m * m * Nk[:, None]
    return logZ, Nk, mu_acc, sig_acc


def full_log_prob(X: Tensor, mu: Tensor, prec_chol: Tensor, lpi: Tensor) -> Tensor:
    """Per-(n, k) log joint for full covariance given L_k with L_k L_k^T = Sigma_k^-1.

    Follows flash_gmm_full_h100.py:289-296 and :124-130:
        v = L^T x - L^T mu,  maha = ||v||^2,
        ll = lpi + sum_d log(|L_dd| + 1e-30) - 0.5*D*log2pi - 0.5*maha
    """
    D = X.shape[1]
    LT = prec_chol.transpose(-1, -2)                               # :289
    LT_mu = torch.einsum("kij,kj->ki", LT, mu)                      # :290
    log_diag_sum = torch.log(prec_chol.diagonal(dim1=-2, dim2=-1).abs() + 1e-30).sum(dim=-1)  # :294
    v = torch.einsum("kij,nj->nki", LT, X) - LT_mu[None, :, :]      # :124-126
    maha = (v * v).sum(dim=2)                                       # :127
    return lpi[None, :] + log_diag_sum[None, :] - 0.5 * D * LOG_2PI - 0.5 * maha


def estep_full(X: Tensor, mu: Tensor, prec_chol: Tensor, log_pi: Tensor, *,
               dtype: torch.dtype = torch.float64,
               chunk: int = 4096) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Full-covariance E-step: (logZ, Nk, mu_acc, sig_outer[K, D, D]).

    sig_outer[k] = sum_n r_nk x_n x_n^T, uncentred (flash_gmm_full_h100.py:213-228,
    docstring :251-255).
    """
    X, mu = _as(X, dtype), _as(mu, dtype)
    L, lpi = _as(prec_chol, dtype), _as(log_pi, dtype)
    N, D = X.shape
    K = mu.shape[0]
    if L.shape != (K, D, D):
        raise ValueError(f"prec_chol must be (K, D, D)=({K}, {D}, {D}), got {tuple(L.shape)}")
    logZ = torch.empty(N, dtype=dtype)
    Nk = torch.zeros(K, dtype=dtype)
    mu_acc = torch.zeros(K, D, dtype=dtype)
    sig_outer = torch.zeros(K, D, D, dtype=dtype)
    for n0 in range(0, N, chunk):
        x = X[n0:n0 + chunk]
        ll = full_log_prob(x, mu, L, lpi)
        lz = torch.logsumexp(ll, dim=1)
        logZ[n0:n0 + chunk] = lz
        r = torch.exp(ll - lz[:, None])
        Nk += r.sum(dim=0)
        mu_acc += r.T @ x
        sig_outer += torch.einsum("nk,ni,nj->kij", r, x, x)
    return logZ, Nk, mu_acc, sig_outer


def estep_full_bf16(X: Tensor, mu: Tensor, prec_chol: Tensor, log_pi: Tensor, *,
                    chunk: int = 1024) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Full-covariance E-step with the bf16 operand contract of flash_gmm_full_h100.py.

    x and L^T are rounded to bfloat16 (:98, :176, :298); b = L^T mu stays float32
    (:290); v = bf16(x) . bf16(L^T)^T - b and maha = sum v^2 (:125-127, :192-194);
    ll2 = c0 - 0.5 log2e maha with c0 = (lpi + sum_d log(|L_dd| + 1e-30) - 0.5 D
    log 2pi) log2e (:294-296, :196); r = 2^(ll2 - logZ2) (:198); Nk = sum r (:203);
    mu_acc = bf16(r)^T bf16(x) (:200, :207); sig_outer[k, d2, :] = sum_n
    bf16(r_nk x_nd2) bf16(x_n) with x_nd2 the float32 value (:216-222), which is not
    symmetric; logZ = logZ2 ln 2 (:335).  Everything except the roundings is float64
    here (the reference accumulates in float32).
    """
    X32, mu32 = _as(X, torch.float32), _as(mu, torch.float32)
    L32, lpi = _as(prec_chol, torch.float32), _as(log_pi, torch.float64)
    N, D = X32.shape
    K = mu32.shape[0]
    if L32.shape != (K, D, D):
        raise ValueError(f"prec_chol must be (K, D, D)=({K}, {D}, {D}), got {tuple(L32.shape)}")
    Lb = bf16_round(L32)                                            # L_bf[k, d1, d2]
    b = torch.einsum("kij,ki->kj", L32.double(), mu32.double())     # (L^T mu)[k, d2]
    log_diag_sum = torch.log(L32.double().diagonal(dim1=-2, dim2=-1).abs() + 1e-30).sum(dim=-1)
    c0 = (lpi + log_diag_sum - 0.5 * D * LOG_2PI) * LOG2_E
    logZ = torch.empty(N, dtype=torch.float64)
    Nk = torch.zeros(K, dtype=torch.float64)
    mu_acc = torch.zeros(K, D, dtype=torch.float64)
    sig_outer = torch.zeros(K, D, D, dtype=torch.float64)
    ln2 = math.log(2.0)
    for n0 in range(0, N, chunk):
        x32 = X32[n0:n0 + chunk]
        xb = bf16_round(x32)
        v = torch.einsum("kij,ni->nkj", Lb, xb) - b[None, :, :]
        ll2 = c0[None, :] - 0.5 * LOG2_E * (v * v).sum(dim=2)
        lz2 = torch.logsumexp(ll2 * ln2, dim=1) / ln2
        logZ[n0:n0 + chunk] = lz2 * ln2
        r = torch.exp2(ll2 - lz2[:, None])
        Nk += r.sum(dim=0)
        mu_acc += bf16_round(r).T @ xb
        rx = bf16_round(r[:, :, None] * x32.double()[:, None, :])   # (n, k, d2)
        sig_outer += torch.einsum("nki,nj->kij", rx, xb)
    return logZ, Nk, mu_acc, sig_outer


# ---------------------------------------------------------------------------
# M-steps (README.md:59-61, :99-100; flash_gmm_full_h100.py:257-260)
# ---------------------------------------------------------------------------

def mstep_iso(Nk: Tensor, mu_acc: Tensor, sig_acc: Tensor, N: int, D: int):
    """pi = Nk/N, mu = mu_acc/Nk, sigma^2 = sig_acc/(D*Nk)  (README.md:59-61)."""
    pi = Nk / N
    mu = mu_acc / Nk[:, None]
    sigma_sq = sig_acc / (D * Nk)
    return pi, mu, sigma_sq


def mstep_diag(Nk: Tensor, mu_acc: Tensor, sig_acc: Tensor, N: int):
    """pi = Nk/N, mu = mu_acc/Nk, sigma^2_kd = sig_acc_kd/Nk (the diagonal analogue of
    README.md:59-61; sig_acc is accumulated about the previous means)."""
    pi = Nk / N
    mu = mu_acc / Nk[:, None]
    var = sig_acc / Nk[:, None]
    return pi, mu, var


def prec_chol_from_cov(cov: Tensor) -> Tensor:
    """Lower-triangular L with L L^T = cov^-1 (the prec_chol parameterisation of
    flash_gmm_full_h100.py:238,247-248), in float64.  Per component in numpy: batched
    float64 inverses through torch's CPU backend have come back not positive definite
    on some hosts (see flash_gmm.data.full_clustered)."""
    import numpy as np
    c = cov.double().cpu().numpy()
    batch = c.reshape(-1, c.shape[-2], c.shape[-1])
    out = np.empty_like(batch)
    for k in range(batch.shape[0]):
        p = np.linalg.inv(batch[k])
        out[k] = np.linalg.cholesky(0.5 * (p + p.T))
    return torch.from_numpy(out.reshape(c.shape))


def mstep_full(Nk: Tensor, mu_acc: Tensor, sig_outer: Tensor, N: int):
    """Sigma_k = sig_outer/Nk - mu mu^T  (flash_gmm_full_h100.py:257-260)."""
    pi = Nk / N
    mu = mu_acc / Nk[:, None]
    cov = sig_outer / Nk[:, None, None] - mu[:, :, None] * mu[:, None, :]
    return pi, mu, cov


# ---------------------------------------------------------------------------
# Brute force (pure Python loops, tiny inputs only)
# ---------------------------------------------------------------------------

def _bf16_scalar(v: float) -> float:
    """Round one float to bfloat16 by bit manipulation: nearest, ties to even."""
    import struct
    b = struct.unpack("<I", struct.pack("<f", v))[0]
    lsb = (b >> 16) & 1
    b = (b + 0x7FFF + lsb) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", b))[0]


def brute_estep_iso_bf16(X, mu, lss, lpi):
    """Scalar-loop version of estep_iso_bf16 for tiny inputs (bit-level bf16 rounding)."""
    X = [[float(v) for v in row] for row in X.tolist()]
    mu = [[float(v) for v in row] for row in mu.tolist()]
    lss = [float(v) for v in lss.tolist()]
    lpi = [float(v) for v in lpi.tolist()]
    N, D, K = len(X), len(X[0]) if X else 0, len(mu)
    xb = [[_bf16_scalar(v) for v in row] for row in X]
    mb = [[_bf16_scalar(v) for v in row] for row in mu]
    logZ, Nk = [], [0.0] * K
    mu_acc = [[0.0] * D for _ in range(K)]
    sig_acc = [0.0] * K
    for n in range(N):
        x_sq = sum(v * v for v in xb[n])
        ll2, sq = [], []
        for k in range(K):
            ish = 0.5 * math.exp(-lss[k]) / math.log(2.0)
            mu_sq = sum(v * v for v in mu[k])
            xmu = sum(xb[n][d] * mb[k][d] for d in range(D))
            c0 = (lpi[k] - 0.5 * D * (LOG_2PI + lss[k])) / math.log(2.0) - ish * mu_sq
            ll2.append(c0 - ish * x_sq + 2.0 * ish * xmu)
            sq.append(x_sq - 2.0 * xmu + mu_sq)
        m = max(ll2)
        lz2 = m + math.log2(sum(2.0 ** (v - m) for v in ll2))
        logZ.append(lz2 * math.log(2.0))
        for k in range(K):
            r = 2.0 ** (ll2[k] - lz2)
            Nk[k] += r
            sig_acc[k] += r * sq[k]
            rb = _bf16_scalar(r)
            for d in range(D):
                mu_acc[k][d] += rb * xb[n][d]
    return logZ, Nk, mu_acc, sig_acc


def brute_estep_diag_bf16(X, mu, lss, lpi):
    """Scalar-loop version of estep_diag_bf16 for tiny inputs (bit-level bf16 rounding)."""
    import struct

    def f32(v):
        return struct.unpack("<f", struct.pack("<f", v))[0]

    X = [[float(v) for v in row] for row in X.tolist()]
    mu = [[float(v) for v in row] for row in mu.tolist()]
    lss = [[float(v) for v in row] for row in lss.tolist()]
    lpi = [float(v) for v in lpi.tolist()]
    N, D, K = len(X), len(X[0]) if X else 0, len(mu)
    half_log2e = f32(0.5 / math.log(2.0))
    w1 = [[f32(f32(math.exp(-lss[k][d])) * half_log2e) for d in range(D)] for k in range(K)]
    w2 = [[f32(mu[k][d] * w1[k][d]) for d in range(D)] for k in range(K)]
    w1b = [[_bf16_scalar(v) for v in row] for row in w1]
    w2b = [[_bf16_scalar(v) for v in row] for row in w2]
    c0 = []
    for k in range(K):
        quad = sum(mu[k][d] ** 2 * math.exp(-lss[k][d]) for d in range(D))
        c0.append((lpi[k] - 0.5 * (D * LOG_2PI + sum(lss[k]))) / math.log(2.0)
                  - 0.5 / math.log(2.0) * quad)
    logZ, Nk = [], [0.0] * K
    mu_acc = [[0.0] * D for _ in range(K)]
    rxsq = [[0.0] * D for _ in range(K)]
    for n in range(N):
        xb = [_bf16_scalar(v) for v in X[n]]
        x2b = [_bf16_scalar(f32(v * v)) for v in X[n]]
        ll2 = [c0[k] - sum(x2b[d] * w1b[k][d] for d in range(D))
               + 2.0 * sum(xb[d] * w2b[k][d] for d in range(D)) for k in range(K)]
        m = max(ll2)
        lz2 = m + math.log2(sum(2.0 ** (v - m) for v in ll2))
        logZ.append(lz2 * math.log(2.0))
        for k in range(K):
            r = 2.0 ** (ll2[k] - lz2)
            Nk[k] += r
            rb = _bf16_scalar(r)
            for d in range(D):
                mu_acc[k][d] += rb * xb[d]
                rxsq[k][d] += rb * x2b[d]
    sig_acc = [[rxsq[k][d] - 2.0 * mu[k][d] * mu_acc[k][d] + mu[k][d] ** 2 * Nk[k] for d in range(D)]
               for k in range(K)]
    return logZ, Nk, mu_acc, sig_acc


def brute_estep_full_bf16(X, mu, L, lpi):
    """Scalar-loop version of estep_full_bf16 for tiny inputs (bit-level bf16 rounding)."""
    import struct

    def f32(v):
        return struct.unpack("<f", struct.pack("<f", v))[0]

    X = [[float(v) for v in row] for row in X.tolist()]
    mu = [[float(v) for v in row] for row in mu.tolist()]
    L = [[[float(v) for v in row] for row in Lk] for Lk in L.tolist()]
    lpi = [float(v) for v in lpi.tolist()]
    N, D, K = len(X), len(X[0]) if X else 0, len(mu)
    ln2 = math.log(2.0)
    c0, bvec = [], []
    for k in range(K):
        ld = sum(math.log(abs(L[k][d][d]) + 1e-30) for d in range(D))
        c0.append((lpi[k] + ld - 0.5 * D * LOG_2PI) / ln2)
        bvec.append([sum(L[k][i][j] * mu[k][i] for i in range(D)) for j in range(D)])
    logZ, Nk = [], [0.0] * K
    mu_acc = [[0.0] * D for _ in range(K)]
    sig = [[[0.0] * D for _ in range(D)] for _ in range(K)]
    for n in range(N):
        xb = [_bf16_scalar(v) for v in X[n]]
        ll2 = []
        for k in range(K):
            maha = 0.0
            for j in range(D):
                vj = sum(xb[i] * _bf16_scalar(L[k][i][j]) for i in range(D)) - bvec[k][j]
                maha += vj * vj
            ll2.append(c0[k] - 0.5 / ln2 * maha)
        m = max(ll2)
        lz2 = m + math.log2(sum(2.0 ** (v - m) for v in ll2))
        logZ.append(lz2 * ln2)
        for k in range(K):
            r = 2.0 ** (ll2[k] - lz2)
            Nk[k] += r
            rb = _bf16_scalar(r)
            for d in range(D):
                mu_acc[k][d] += rb * xb[d]
            for d2 in range(D):
                a = _bf16_scalar(f32(r * X[n][d2]))
                for d1 in range(D):
                    sig[k][d2][d1] += a * xb[d1]
    return logZ, Nk, mu_acc, sig


def brute_estep_iso(X, mu, lss, lpi):
    """Scalar-loop float64 E-step, for N, K, D <= ~16 (direct distances)."""
    X = [[float(v) for v in row] for row in X.tolist()]
    mu = [[float(v) for v in row] for row in mu.tolist()]
    lss = [float(v) for v in lss.tolist()]
    lpi = [float(v) for v in lpi.tolist()]
    N, D, K = len(X), len(X[0]) if X else 0, len(mu)
    logZ, Nk = [], [0.0] * K
    mu_acc = [[0.0] * D for _ in range(K)]
    sig_acc = [0.0] * K
    for n in range(N):
        sq = [sum((X[n][d] - mu[k][d]) ** 2 for d in range(D)) for k in range(K)]
        ll = [lpi[k] - 0.5 * sq[k] * math.exp(-lss[k]) - 0.5 * D * (LOG_2PI + lss[k])
              for k in range(K)]
        m = max(ll)
        lz = m + math.log(sum(math.exp(v - m) for v in ll))
        logZ.append(lz)
        for k in range(K):
            r = math.exp(ll[k] - lz)
            Nk[k] += r
            sig_acc[k] += r * sq[k]
            for d in range(D):
                mu_acc[k][d] += r * X[n][d]
    return logZ, Nk, mu_acc, sig_acc

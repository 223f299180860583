"""Pins the CPU oracle (oracle/gmm_oracle.py) before anything is checked against it.

Each check is independent of the oracle's own formula: scipy's Gaussian log
densities, sklearn's GaussianMixture estimators, a scalar-loop brute force,
closed-form special cases and exact invariants.  A plausible mistake (a dropped
normaliser term, a wrong sign, a transposed operand, the wrong mu in sig_acc)
fails at least one of them.
"""

import math

import numpy as np
import pytest
import torch
from scipy.special import logsumexp
from scipy.stats import multivariate_normal

from oracle import gmm_oracle as O

sk_mix = pytest.importorskip("sklearn.mixture._gaussian_mixture")


def _iso_inputs(N=200, K=5, D=6, seed=0, spread=2.0):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(N, D, generator=g, dtype=torch.float64)
    mu = torch.randn(K, D, generator=g, dtype=torch.float64) * spread
    lss = torch.rand(K, generator=g, dtype=torch.float64) - 0.5
    lpi = torch.log_softmax(torch.randn(K, generator=g, dtype=torch.float64), 0)
    return X, mu, lss, lpi


def _diag_inputs(N=200, K=5, D=6, seed=1):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(N, D, generator=g, dtype=torch.float64) * 1.5
    mu = torch.randn(K, D, generator=g, dtype=torch.float64) * 2
    lss = torch.rand(K, D, generator=g, dtype=torch.float64) * 2 - 1
    lpi = torch.log_softmax(torch.randn(K, generator=g, dtype=torch.float64), 0)
    return X, mu, lss, lpi


def _full_inputs(N=150, K=4, D=5, seed=2):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(N, D, generator=g, dtype=torch.float64) * 1.5
    mu = torch.randn(K, D, generator=g, dtype=torch.float64)
    A = torch.randn(K, D, D, generator=g, dtype=torch.float64)
    sigma = A @ A.transpose(1, 2) / D + 0.1 * torch.eye(D, dtype=torch.float64)
    L = torch.linalg.cholesky(torch.linalg.inv(sigma))
    lpi = torch.log_softmax(torch.randn(K, generator=g, dtype=torch.float64), 0)
    return X, mu, L, lpi, sigma


# --------------------------------------------------------------------------- iso

def test_iso_logz_matches_scipy():
    X, mu, lss, lpi = _iso_inputs()
    K, D = mu.shape
    logZ, *_ = O.estep_iso(X, mu, lss, lpi)
    comp = np.stack([multivariate_normal.logpdf(X.numpy(), mean=mu[k].numpy(),
                                                cov=math.exp(lss[k]) * np.eye(D)) + float(lpi[k])
                     for k in range(K)], axis=1)
    np.testing.assert_allclose(logZ.numpy(), logsumexp(comp, axis=1), rtol=0, atol=1e-10)


def test_iso_all_outputs_match_sklearn_spherical():
    X, mu, lss, lpi = _iso_inputs(N=300, K=4, D=5, seed=3)
    K, D = mu.shape
    Xn = X.numpy()
    prec_chol = np.exp(-0.5 * lss.numpy())
    ll = sk_mix._estimate_log_gaussian_prob(Xn, mu.numpy(), prec_chol, "spherical") + lpi.numpy()
    lz_sk = logsumexp(ll, axis=1)
    resp = np.exp(ll - lz_sk[:, None])
    nk, means, cov = sk_mix._estimate_gaussian_parameters(Xn, resp, 0.0, "spherical")
    nk = nk - 10 * np.finfo(resp.dtype).eps  # sklearn adds 10*eps to nk
    logZ, Nk, mu_acc, sig_acc = O.estep_iso(X, mu, lss, lpi)
    np.testing.assert_allclose(logZ.numpy(), lz_sk, atol=1e-10)
    np.testing.assert_allclose(Nk.numpy(), nk, rtol=1e-10)
    np.testing.assert_allclose(mu_acc.numpy(), means * nk[:, None], rtol=1e-9, atol=1e-10)
    # sum_n r ||x - mu_old||^2 = nk * (D * spherical_cov + ||new_mean - mu_old||^2)
    expect = nk * (D * cov + ((means - mu.numpy()) ** 2).sum(1))
    np.testing.assert_allclose(sig_acc.numpy(), expect, rtol=1e-9)


def test_iso_brute_force_tiny():
    X, mu, lss, lpi = _iso_inputs(N=7, K=3, D=4, seed=5)
    lz_b, nk_b, mu_b, sig_b = O.brute_estep_iso(X, mu, lss, lpi)
    logZ, Nk, mu_acc, sig_acc = O.estep_iso(X, mu, lss, lpi)
    np.testing.assert_allclose(logZ.numpy(), lz_b, atol=1e-12)
    np.testing.assert_allclose(Nk.numpy(), nk_b, rtol=1e-12)
    np.testing.assert_allclose(mu_acc.numpy(), np.array(mu_b), rtol=1e-11, atol=1e-13)
    np.testing.assert_allclose(sig_acc.numpy(), sig_b, rtol=1e-11)


def test_iso_expansion_equals_direct_in_fp64():
    X, mu, lss, lpi = _iso_inputs(N=500, K=8, D=16, seed=7)
    a = O.estep_iso(X, mu, lss, lpi, form="expansion")
    b = O.estep_iso(X, mu, lss, lpi, form="direct")
    for u, v in zip(a, b):
        np.testing.assert_allclose(u.numpy(), v.numpy(), rtol=1e-10, atol=1e-9)


def test_iso_chunking_does_not_change_results():
    X, mu, lss, lpi = _iso_inputs(N=1000, K=6, D=8, seed=11)
    a = O.estep_iso(X, mu, lss, lpi, chunk=1000)
    b = O.estep_iso(X, mu, lss, lpi, chunk=97)
    for u, v in zip(a, b):
        np.testing.assert_allclose(u.numpy(), v.numpy(), rtol=1e-12, atol=1e-12)


def test_iso_invariants():
    X, mu, lss, lpi = _iso_inputs(N=400, K=7, D=9, seed=13)
    logZ, Nk, mu_acc, sig_acc = O.estep_iso(X, mu, lss, lpi)
    assert abs(Nk.sum().item() - 400) < 1e-9
    np.testing.assert_allclose(mu_acc.sum(0).numpy(), X.sum(0).numpy(), atol=1e-9)
    # sig_acc = sum r ||x||^2 - 2 mu . mu_acc + ||mu||^2 Nk
    ll, _ = O.iso_log_prob(X, mu, lss, lpi)
    r = torch.exp(ll - logZ[:, None])
    ident = (r * (X * X).sum(1, keepdim=True)).sum(0) - 2 * (mu * mu_acc).sum(1) + (mu * mu).sum(1) * Nk
    np.testing.assert_allclose(sig_acc.numpy(), ident.numpy(), rtol=1e-9)


def test_iso_single_component_closed_form():
    X, mu, lss, lpi = _iso_inputs(N=100, K=1, D=5, seed=17)
    lpi = torch.zeros(1, dtype=torch.float64)
    logZ, Nk, mu_acc, sig_acc = O.estep_iso(X, mu, lss, lpi)
    ref = multivariate_normal.logpdf(X.numpy(), mean=mu[0].numpy(), cov=math.exp(lss[0]) * np.eye(5))
    np.testing.assert_allclose(logZ.numpy(), ref, atol=1e-11)
    assert abs(Nk.item() - 100) < 1e-10
    np.testing.assert_allclose(mu_acc[0].numpy(), X.sum(0).numpy(), atol=1e-10)
    np.testing.assert_allclose(sig_acc.item(), ((X - mu[0]) ** 2).sum().item(), rtol=1e-12)


def test_iso_identical_components_share_uniformly():
    X, mu, lss, lpi = _iso_inputs(N=120, K=1, D=4, seed=19)
    K = 5
    mu = mu.repeat(K, 1)
    lss = lss.repeat(K)
    lpi = torch.full((K,), -math.log(K), dtype=torch.float64)
    _, Nk, mu_acc, _ = O.estep_iso(X, mu, lss, lpi)
    np.testing.assert_allclose(Nk.numpy(), np.full(K, 120 / K), rtol=1e-12)
    np.testing.assert_allclose(mu_acc.numpy(), np.tile(X.sum(0).numpy() / K, (K, 1)), atol=1e-10)


def test_iso_far_clusters_give_kmeans_assignment():
    g = torch.Generator().manual_seed(23)
    K, D, N = 6, 3, 300
    centres = torch.randn(K, D, generator=g, dtype=torch.float64) * 100
    a = torch.randint(0, K, (N,), generator=g)
    X = centres[a] + torch.randn(N, D, generator=g, dtype=torch.float64)
    lss = torch.zeros(K, dtype=torch.float64)
    lpi = torch.full((K,), -math.log(K), dtype=torch.float64)
    _, Nk, mu_acc, _ = O.estep_iso(X, centres, lss, lpi)
    counts = torch.bincount(a, minlength=K).double()
    np.testing.assert_allclose(Nk.numpy(), counts.numpy(), atol=1e-9)
    sums = torch.zeros(K, D, dtype=torch.float64).index_add_(0, a, X)
    np.testing.assert_allclose(mu_acc.numpy(), sums.numpy(), atol=1e-7)


def test_iso_fp32_restatement_close_to_fp64():
    X, mu, lss, lpi = _iso_inputs(N=300, K=8, D=32, seed=29)
    a = O.estep_iso(X, mu, lss, lpi, dtype=torch.float64)
    b = O.estep_iso(X.float(), mu.float(), lss.float(), lpi.float(), dtype=torch.float32)
    assert (a[0] - b[0].double()).abs().max() < 1e-4
    np.testing.assert_allclose(b[1].double().numpy(), a[1].numpy(), rtol=1e-4)


# --------------------------------------------------------------------------- iso, bf16 contract

def test_iso_bf16_equals_fp64_on_bf16_exact_inputs():
    """With X and mu already exact in bfloat16, the bf16 contract changes only mu_acc
    (r is rounded to bf16 for r^T x): logZ, Nk and sig_acc equal the float64 E-step."""
    X, mu, lss, lpi = _iso_inputs(N=300, K=6, D=10, seed=21)
    X = O.bf16_round(X.float())
    mu = O.bf16_round(mu.float())
    ref = O.estep_iso(X, mu, lss, lpi)
    got = O.estep_iso_bf16(X, mu, lss, lpi)
    np.testing.assert_allclose(got[0].numpy(), ref[0].numpy(), atol=1e-11)
    np.testing.assert_allclose(got[1].numpy(), ref[1].numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(got[3].numpy(), ref[3].numpy(), rtol=1e-9, atol=1e-10)
    err = (got[2] - ref[2]).abs().max() / ref[2].abs().max()
    assert 1e-6 < err < 2.0 ** -8          # bf16(r) rounding is visible, and bounded


def test_iso_bf16_brute_force_tiny():
    """Against a scalar loop that rounds to bfloat16 by bit manipulation."""
    X, mu, lss, lpi = _iso_inputs(N=9, K=3, D=5, seed=22)
    X, mu = X.float(), mu.float()
    lz_b, nk_b, mu_b, sig_b = O.brute_estep_iso_bf16(X, mu, lss, lpi)
    logZ, Nk, mu_acc, sig_acc = O.estep_iso_bf16(X, mu, lss, lpi)
    np.testing.assert_allclose(logZ.numpy(), lz_b, atol=1e-11)
    np.testing.assert_allclose(Nk.numpy(), nk_b, rtol=1e-11)
    np.testing.assert_allclose(mu_acc.numpy(), np.array(mu_b), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(sig_acc.numpy(), sig_b, rtol=1e-10)


def test_bf16_float32_mode_is_the_same_contract_in_float32():
    """dtype=float32 evaluates the bf16 contracts' steps in float32: at small D it
    stays within float32 rounding of the float64 evaluation (logZ 1e-4, statistics
    1e-4), and it is not the float64 evaluation itself (the rounding is visible)."""
    X, mu, lss, lpi = _iso_inputs(N=400, K=7, D=24, seed=23)
    a = O.estep_iso_bf16(X, mu, lss, lpi)
    b = O.estep_iso_bf16(X, mu, lss, lpi, dtype=torch.float32)
    assert b[0].dtype == torch.float32
    assert 0 < (a[0] - b[0].double()).abs().max() < 1e-4
    for u, v in zip(a[1:], b[1:]):
        np.testing.assert_allclose(v.double().numpy(), u.numpy(), rtol=1e-4, atol=1e-4 * float(u.abs().max()))
    g = torch.Generator().manual_seed(24)
    lssd = torch.rand(7, 24, generator=g, dtype=torch.float64) - 0.5
    a = O.estep_diag_bf16(X, mu, lssd, lpi)
    b = O.estep_diag_bf16(X, mu, lssd, lpi, dtype=torch.float32)
    assert 0 < (a[0] - b[0].double()).abs().max() < 1e-4
    for u, v in zip(a[1:], b[1:]):
        np.testing.assert_allclose(v.double().numpy(), u.numpy(), rtol=1e-4, atol=1e-4 * float(u.abs().max()))


def test_bf16_scalar_rounding_ties_to_even():
    """The brute-force rounding itself: ties go to the even bfloat16 neighbour."""
    one_ulp = 2.0 ** -7                      # bf16 spacing at 1.0
    assert O._bf16_scalar(1.0 + one_ulp / 2) == 1.0                    # tie, even below
    assert O._bf16_scalar(1.0 + 1.5 * one_ulp) == 1.0 + 2 * one_ulp   # tie, even above
    assert O._bf16_scalar(1.0 + 0.6 * one_ulp) == 1.0 + one_ulp
    assert O._bf16_scalar(-3.0) == -3.0


# --------------------------------------------------------------------------- diag

def test_diag_logz_matches_scipy_and_sklearn():
    X, mu, lss, lpi = _diag_inputs()
    K, D = mu.shape
    logZ, Nk, mu_acc, sig_acc = O.estep_diag(X, mu, lss, lpi)
    comp = np.stack([multivariate_normal.logpdf(X.numpy(), mean=mu[k].numpy(),
                                                cov=np.diag(np.exp(lss[k].numpy()))) + float(lpi[k])
                     for k in range(K)], axis=1)
    np.testing.assert_allclose(logZ.numpy(), logsumexp(comp, axis=1), atol=1e-10)
    Xn = X.numpy()
    ll = sk_mix._estimate_log_gaussian_prob(Xn, mu.numpy(), np.exp(-0.5 * lss.numpy()), "diag") + lpi.numpy()
    resp = np.exp(ll - logsumexp(ll, axis=1)[:, None])
    nk, means, cov = sk_mix._estimate_gaussian_parameters(Xn, resp, 0.0, "diag")
    nk = nk - 10 * np.finfo(resp.dtype).eps
    np.testing.assert_allclose(Nk.numpy(), nk, rtol=1e-10)
    np.testing.assert_allclose(mu_acc.numpy(), means * nk[:, None], rtol=1e-9, atol=1e-10)
    expect = nk[:, None] * (cov + (means - mu.numpy()) ** 2)
    np.testing.assert_allclose(sig_acc.numpy(), expect, rtol=1e-8, atol=1e-9)


def test_diag_equals_iso_for_equal_variances():
    X, mu, lss, lpi = _iso_inputs(N=200, K=5, D=7, seed=31)
    iso = O.estep_iso(X, mu, lss, lpi)
    dg = O.estep_diag(X, mu, lss[:, None].repeat(1, 7), lpi)
    for i in range(3):
        np.testing.assert_allclose(dg[i].numpy(), iso[i].numpy(), rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(dg[3].sum(1).numpy(), iso[3].numpy(), rtol=1e-10)


def test_diag_direct_form():
    X, mu, lss, lpi = _diag_inputs(N=100, K=4, D=5, seed=37)
    a = O.estep_diag(X, mu, lss, lpi, form="expansion")
    b = O.estep_diag(X, mu, lss, lpi, form="direct")
    for u, v in zip(a, b):
        np.testing.assert_allclose(u.numpy(), v.numpy(), rtol=1e-10, atol=1e-9)


# --------------------------------------------------------------------------- diag, bf16 contract

def _pow2_weight_lss(j: int) -> float:
    """A float32 log-variance for which the contract's weight W1 = fp32(exp(-lss)) *
    fp32(0.5 log2 e) is exactly 2**j (so rounding W1 to bfloat16 changes nothing)."""
    start = np.float32(-math.log(2.0 ** j / (0.5 * O.LOG2_E)))
    bits = start.view(np.int32)
    for m in range(4096):
        for s in (m, -m):
            cand = np.array(bits + s, dtype=np.int32).view(np.float32)
            w1, _ = O.diag_bf16_weights(torch.zeros(1, 1), torch.tensor([[float(cand)]]))
            if float(w1) == 2.0 ** j:
                return float(cand)
    raise AssertionError(f"no float32 lss gives W1 = 2^{j}")


def test_diag_bf16_equals_fp64_on_bf16_exact_operands():
    """When x, x^2, W1 and W2 are all exact in bfloat16 (x = k/4 with |k| <= 15, W1 a
    power of two, mu exact in bfloat16), the contract only rounds r for mu_acc and
    rxsq: logZ and Nk equal the float64 E-step up to the float32 rounding of W1 that
    the reference's own c0 (exact exp) does not share (~1e-7 relative)."""
    g = torch.Generator().manual_seed(31)
    N, K, D = 400, 5, 7
    X = torch.randint(-15, 16, (N, D), generator=g).double() / 4
    mu = O.bf16_round((torch.randn(K, D, generator=g) * 1.5).float())
    js = torch.randint(-3, 2, (K, D), generator=g)
    lss = torch.tensor([[_pow2_weight_lss(int(j)) for j in row] for row in js], dtype=torch.float64)
    lpi = torch.log_softmax(torch.randn(K, generator=g, dtype=torch.float64), 0)
    w1, w2 = O.diag_bf16_weights(mu, lss)
    assert torch.equal(O.bf16_round(w1), w1.double()) and torch.equal(O.bf16_round(w2), w2.double())
    assert torch.equal(O.bf16_round((X * X).float()), X * X)
    ref = O.estep_diag(X, mu, lss, lpi)
    got = O.estep_diag_bf16(X, mu, lss, lpi)
    np.testing.assert_allclose(got[0].numpy(), ref[0].numpy(), atol=2e-5)
    np.testing.assert_allclose(got[1].numpy(), ref[1].numpy(), rtol=2e-5, atol=1e-9)
    # r is rounded to bfloat16 for mu_acc and rxsq: visible, and bounded by 2^-8.
    err_mu = ((got[2] - ref[2]).abs().max() / ref[2].abs().max()).item()
    err_sig = ((got[3] - ref[3]).abs().max() / ref[3].abs().max()).item()
    assert 1e-7 < err_mu < 2.0 ** -8 and err_sig < 2.0 ** -7


def test_diag_bf16_brute_force_tiny():
    """Against a scalar loop that rounds to bfloat16 by bit manipulation."""
    X, mu, lss, lpi = _diag_inputs(N=9, K=3, D=5, seed=23)
    X, mu, lss = X.float(), mu.float(), lss.float()
    lz_b, nk_b, mu_b, sig_b = O.brute_estep_diag_bf16(X, mu, lss, lpi)
    logZ, Nk, mu_acc, sig_acc = O.estep_diag_bf16(X, mu, lss, lpi)
    np.testing.assert_allclose(logZ.numpy(), lz_b, atol=1e-10)
    np.testing.assert_allclose(Nk.numpy(), nk_b, rtol=1e-10)
    np.testing.assert_allclose(mu_acc.numpy(), np.array(mu_b), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(sig_acc.numpy(), np.array(sig_b), rtol=1e-9, atol=1e-10)


def test_diag_bf16_invariants():
    """Responsibilities sum to one per row; mu_acc sums to the rows' bf16 values up to
    the bf16 rounding of r."""
    X, mu, lss, lpi = _diag_inputs(N=500, K=8, D=6, seed=24)
    logZ, Nk, mu_acc, sig_acc = O.estep_diag_bf16(X.float(), mu.float(), lss.float(), lpi)
    assert abs(Nk.sum().item() - 500) < 1e-9
    xb = O.bf16_round(X.float())
    err = (mu_acc.sum(dim=0) - xb.sum(dim=0)).abs().max() / xb.abs().sum(dim=0).max()
    assert err < 2.0 ** -8
    assert (sig_acc > -1e-9).all()


# --------------------------------------------------------------------------- full

def test_full_matches_scipy_and_sklearn():
    X, mu, L, lpi, sigma = _full_inputs()
    K, D = mu.shape
    logZ, Nk, mu_acc, sig_outer = O.estep_full(X, mu, L, lpi)
    comp = np.stack([multivariate_normal.logpdf(X.numpy(), mean=mu[k].numpy(), cov=sigma[k].numpy())
                     + float(lpi[k]) for k in range(K)], axis=1)
    np.testing.assert_allclose(logZ.numpy(), logsumexp(comp, axis=1), atol=1e-9)
    Xn = X.numpy()
    ll = sk_mix._estimate_log_gaussian_prob(Xn, mu.numpy(), L.numpy(), "full") + lpi.numpy()
    resp = np.exp(ll - logsumexp(ll, axis=1)[:, None])
    nk, means, cov = sk_mix._estimate_gaussian_parameters(Xn, resp, 0.0, "full")
    nk = nk - 10 * np.finfo(resp.dtype).eps
    np.testing.assert_allclose(Nk.numpy(), nk, rtol=1e-10)
    np.testing.assert_allclose(mu_acc.numpy(), means * nk[:, None], rtol=1e-9, atol=1e-10)
    expect = nk[:, None, None] * (cov + means[:, :, None] * means[:, None, :])
    np.testing.assert_allclose(sig_outer.numpy(), expect, rtol=1e-8, atol=1e-9)


def test_full_equals_diag_for_diagonal_factor():
    X, mu, lss, lpi = _diag_inputs(N=120, K=3, D=4, seed=41)
    L = torch.diag_embed(torch.exp(-0.5 * lss))
    f = O.estep_full(X, mu, L, lpi)
    d = O.estep_diag(X, mu, lss, lpi)
    for i in range(3):
        np.testing.assert_allclose(f[i].numpy(), d[i].numpy(), rtol=1e-11, atol=1e-11)
    # diagonal of the centred second moment about the old mean = diag sig_acc
    c = f[3].diagonal(dim1=1, dim2=2) - 2 * mu * f[2] + mu * mu * f[1][:, None]
    np.testing.assert_allclose(c.numpy(), d[3].numpy(), rtol=1e-9, atol=1e-9)


# --------------------------------------------------------------------------- full, bf16 contract

def test_full_bf16_equals_fp64_on_bf16_exact_operands():
    """With x and L already exact in bfloat16, the contract rounds only r (mu_acc) and
    r x_d2 (sig_outer): logZ and Nk equal the float64 E-step, the statistics stay
    within the bf16 rounding, and sig_outer loses its symmetry by about that much."""
    X, mu, L, lpi, _ = _full_inputs(N=300, K=4, D=6, seed=51)
    X = O.bf16_round(X.float())
    L = O.bf16_round(L.float())
    mu = mu.float().double()
    ref = O.estep_full(X, mu, L, lpi)
    got = O.estep_full_bf16(X, mu, L, lpi)
    np.testing.assert_allclose(got[0].numpy(), ref[0].numpy(), atol=1e-9)
    np.testing.assert_allclose(got[1].numpy(), ref[1].numpy(), rtol=1e-9, atol=1e-12)
    for i in (2, 3):
        err = ((got[i] - ref[i]).abs().max() / ref[i].abs().max()).item()
        assert 1e-7 < err < 2.0 ** -8, (i, err)
    asym = ((got[3] - got[3].transpose(1, 2)).abs().max() / got[3].abs().max()).item()
    assert 0 < asym < 2.0 ** -7


def test_full_bf16_brute_force_tiny():
    """Against a scalar loop that rounds to bfloat16 by bit manipulation."""
    X, mu, L, lpi, _ = _full_inputs(N=8, K=3, D=4, seed=52)
    X, mu, L = X.float(), mu.float(), L.float()
    lz_b, nk_b, mu_b, sig_b = O.brute_estep_full_bf16(X, mu, L, lpi)
    logZ, Nk, mu_acc, sig = O.estep_full_bf16(X, mu, L, lpi)
    np.testing.assert_allclose(logZ.numpy(), lz_b, atol=1e-10)
    np.testing.assert_allclose(Nk.numpy(), nk_b, rtol=1e-10)
    np.testing.assert_allclose(mu_acc.numpy(), np.array(mu_b), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(sig.numpy(), np.array(sig_b), rtol=1e-9, atol=1e-11)


def test_full_bf16_invariants():
    X, mu, L, lpi, _ = _full_inputs(N=400, K=5, D=5, seed=53)
    logZ, Nk, mu_acc, sig = O.estep_full_bf16(X.float(), mu.float(), L.float(), lpi)
    assert abs(Nk.sum().item() - 400) < 1e-9
    xb = O.bf16_round(X.float())
    err = (mu_acc.sum(dim=0) - xb.sum(dim=0)).abs().max() / xb.abs().sum(dim=0).max()
    assert err < 2.0 ** -8
    # the trace of sum_k sig_outer_k is sum_n ||x_n||^2 up to the roundings
    tr = sig.diagonal(dim1=1, dim2=2).sum().item()
    assert abs(tr - (X.float().double() ** 2).sum().item()) / tr < 2.0 ** -7


# --------------------------------------------------------------------------- M-step

def test_mstep_iso_single_component():
    g = torch.Generator().manual_seed(43)
    X = torch.randn(500, 3, generator=g, dtype=torch.float64) * 2 + 1
    mu0 = X.mean(0, keepdim=True)
    _, Nk, mu_acc, sig_acc = O.estep_iso(X, mu0, torch.zeros(1, dtype=torch.float64),
                                         torch.zeros(1, dtype=torch.float64))
    pi, mu, s2 = O.mstep_iso(Nk, mu_acc, sig_acc, 500, 3)
    assert abs(pi.item() - 1) < 1e-12
    np.testing.assert_allclose(mu.numpy(), mu0.numpy(), atol=1e-12)
    np.testing.assert_allclose(s2.item(), ((X - mu0) ** 2).mean().item(), rtol=1e-12)


def test_mstep_full_recovers_sample_covariance():
    X, mu, L, lpi, _ = _full_inputs(N=200, K=1, D=4, seed=47)
    _, Nk, mu_acc, so = O.estep_full(X, mu, L, torch.zeros(1, dtype=torch.float64))
    _, m, cov = O.mstep_full(Nk, mu_acc, so, 200)
    np.testing.assert_allclose(m[0].numpy(), X.mean(0).numpy(), atol=1e-12)
    np.testing.assert_allclose(cov[0].numpy(), np.cov(X.numpy().T, bias=True), atol=1e-10)


def test_mstep_diag_single_component():
    g = torch.Generator().manual_seed(48)
    X = torch.randn(400, 5, generator=g, dtype=torch.float64) * torch.tensor([1.0, 2, 3, 0.5, 1.5]) - 2
    mu0 = X.mean(0, keepdim=True)
    _, Nk, mu_acc, sig = O.estep_diag(X, mu0, torch.zeros(1, 5, dtype=torch.float64),
                                      torch.zeros(1, dtype=torch.float64))
    pi, mu, var = O.mstep_diag(Nk, mu_acc, sig, 400)
    assert abs(pi.item() - 1) < 1e-12
    np.testing.assert_allclose(mu.numpy(), mu0.numpy(), atol=1e-12)
    np.testing.assert_allclose(var[0].numpy(), X.var(0, unbiased=False).numpy(), rtol=1e-10)


def test_prec_chol_from_cov():
    g = torch.Generator().manual_seed(49)
    A = torch.randn(3, 6, 6, generator=g, dtype=torch.float64)
    cov = A @ A.transpose(1, 2) / 6 + 0.1 * torch.eye(6, dtype=torch.float64)
    L = O.prec_chol_from_cov(cov)
    eye = torch.eye(6, dtype=torch.float64).expand(3, 6, 6)
    torch.testing.assert_close(L @ L.transpose(1, 2) @ cov, eye, rtol=0, atol=1e-10)
    assert torch.all(torch.triu(L, 1) == 0) and torch.all(torch.diagonal(L, dim1=1, dim2=2) > 0)
    d = torch.tensor([0.5, 2.0, 4.0], dtype=torch.float64)
    torch.testing.assert_close(O.prec_chol_from_cov(torch.diag(d)), torch.diag(d.rsqrt()),
                               rtol=0, atol=1e-14)

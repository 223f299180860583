"""The native synthetic row source (host code, no GPU): counter-based
reproducibility and the distribution of its rows."""

import os

import numpy as np
import pytest
from scipy import stats

from flash_gmm import FlashGMMError, SynthIsoSource


def test_rows_do_not_depend_on_chunking_or_threads():
    c = np.random.default_rng(0).normal(size=(7, 33)).astype(np.float32)
    one = SynthIsoSource(c, seed=11, threads=1).rows(0, 1000)
    parts = SynthIsoSource(c, seed=11, threads=4)
    two = np.concatenate([parts.rows(0, 377), parts.rows(377, 623)])
    assert np.array_equal(one, two)
    assert np.array_equal(one[500:520], SynthIsoSource(c, seed=11).rows(500, 20))


def test_seeds_differ():
    c = np.zeros((3, 8), np.float32)
    a = SynthIsoSource(c, seed=1).rows(0, 100)
    b = SynthIsoSource(c, seed=2).rows(0, 100)
    assert not np.allclose(a, b)


@pytest.mark.parametrize("D", [128, 30, 1])
def test_noise_is_standard_normal(D):
    x = SynthIsoSource(np.zeros((1, D), np.float32), seed=5).rows(0, max(20000, 400000 // D))
    v = x.reshape(-1).astype(np.float64)
    n = v.size
    assert abs(v.mean()) < 5 / np.sqrt(n)
    assert abs(v.var() - 1) < 5 * np.sqrt(2 / n)
    assert abs(stats.kurtosis(v, fisher=False) - 3) < 0.05
    assert stats.kstest(v, "norm").pvalue > 1e-3
    # coordinates are uncorrelated
    if D > 1:
        r = np.corrcoef(x[:, 0], x[:, D - 1])[0, 1]
        assert abs(r) < 5 / np.sqrt(x.shape[0])


def test_assignment_is_uniform():
    K = 8
    c = np.zeros((K, 4), np.float32)
    c[:, 0] = np.arange(K) * 100.0
    x = SynthIsoSource(c, seed=9).rows(0, 80000)
    a = np.rint(x[:, 0] / 100.0).astype(int)
    counts = np.bincount(a, minlength=K)
    assert counts.sum() == 80000
    assert stats.chisquare(counts).pvalue > 1e-3
    np.testing.assert_allclose(x[:, 1:].mean(0), 0.0, atol=0.05)


def test_bad_arguments():
    s = SynthIsoSource(np.zeros((2, 4), np.float32))
    with pytest.raises(FlashGMMError):
        s.rows(-1, 10)


def test_simd_philox_matches_scalar(tmp_path):
    """AVX2 and AVX-512 Philox sweeps equal the scalar generator word for word."""
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    exe = str(tmp_path / "rng_simd_check")
    subprocess.run(["g++", "-O2", "-march=x86-64-v3", "-std=c++17",
                    "-I" + os.path.join(root, "include"),
                    "-I" + os.path.join(root, "flash-gmm_amd", "csrc"),
                    os.path.join(here, "rng_simd_check.cpp"), "-o", exe, "-pthread", "-lmvec", "-lm"],
                   check=True)
    out = subprocess.run([exe], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr

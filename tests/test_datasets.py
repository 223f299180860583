"""Local embedding files (the formats of SIFT1M, GIST, Deep10M and GloVe) as row
sources: CPU checks of the native memory-mapped reader and the text reader, on
small files written here; a GPU check streams a file through the EM driver."""

import os

import numpy as np
import pytest
import torch

from flash_gmm import FlashGMMError, datasets


@pytest.fixture
def rows():
    rng = np.random.default_rng(7)
    return rng.normal(size=(1037, 24)).astype(np.float32) * 3


@pytest.mark.parametrize("ext", [".fvecs", ".fbin"])
def test_float_files_round_trip(tmp_path, rows, ext):
    path = str(tmp_path / ("x" + ext))
    datasets.write_vecs(path, rows)
    with datasets.VecsFile(path, threads=3) as f:
        assert (f.N, f.D) == rows.shape
        np.testing.assert_array_equal(f.rows(0, f.N), rows)
        np.testing.assert_array_equal(f.rows(500, 37), rows[500:537])
        np.testing.assert_array_equal(f(1036, 1), rows[1036:])
    np.testing.assert_array_equal(datasets.load_rows(path, 10, 5).numpy(), rows[10:15])


@pytest.mark.parametrize("ext", [".bvecs", ".u8bin"])
def test_byte_files_become_floats(tmp_path, ext):
    b = np.random.default_rng(8).integers(0, 256, size=(3000, 128), dtype=np.uint8)   # SIFT-like
    path = str(tmp_path / ("x" + ext))
    datasets.write_vecs(path, b)
    with datasets.VecsFile(path) as f:
        assert (f.N, f.D) == (3000, 128)
        got = f.rows(0, 3000)                 # several host threads
        assert got.dtype == np.float32
        np.testing.assert_array_equal(got, b.astype(np.float32))


def test_fvecs_layout_is_the_published_one(tmp_path):
    """Per vector an int32 dimension then the float32 values (the SIFT1M base file)."""
    path = str(tmp_path / "two.fvecs")
    with open(path, "wb") as fh:
        for v in ([1.0, 2.0, 3.0], [4.0, 5.0, 6.0]):
            fh.write(np.int32(3).tobytes() + np.array(v, dtype=np.float32).tobytes())
    with datasets.VecsFile(path) as f:
        np.testing.assert_array_equal(f.rows(0, 2), [[1, 2, 3], [4, 5, 6]])


def test_malformed_and_missing_files_are_rejected(tmp_path):
    bad = str(tmp_path / "bad.fvecs")
    with open(bad, "wb") as fh:   # second vector claims another dimension
        fh.write(np.int32(2).tobytes() + np.zeros(2, np.float32).tobytes())
        fh.write(np.int32(3).tobytes() + np.zeros(1, np.float32).tobytes())
    with pytest.raises(FlashGMMError):
        datasets.VecsFile(bad)
    short = str(tmp_path / "short.fbin")
    with open(short, "wb") as fh:  # header promises more than the file holds
        fh.write(np.array([10, 4], np.uint32).tobytes() + np.zeros(8, np.float32).tobytes())
    with pytest.raises(FlashGMMError):
        datasets.VecsFile(short)
    # Headers whose n * d * 4 passes 2^64 (and would wrap to a small size in a
    # product test): n = d = 2^31 and n = d = 2^32 - 1; and one far too large for bytes.
    for ext, n, d in ((".fbin", 1 << 31, 1 << 31), (".fbin", 2**32 - 1, 2**32 - 1), (".u8bin", 1 << 31, 1 << 31)):
        wrap = str(tmp_path / ("wrap" + ext))
        with open(wrap, "wb") as fh:
            fh.write(np.array([n, d], np.uint32).tobytes() + np.zeros(16, np.float32).tobytes())
        with pytest.raises(FlashGMMError):
            datasets.VecsFile(wrap)
    with pytest.raises(FlashGMMError):
        datasets.VecsFile(str(tmp_path / "absent.fvecs"))
    with pytest.raises(FlashGMMError):
        datasets.vecs_format("x.npy")
    path = str(tmp_path / "ok.fvecs")
    datasets.write_vecs(path, np.ones((4, 2), np.float32))
    with datasets.VecsFile(path) as f:
        with pytest.raises(FlashGMMError):
            f.rows(3, 2)          # past the end


def test_text_embeddings(tmp_path, rows):
    """GloVe text (token then values per line), with and without a word2vec header."""
    lines = [f"w{i} " + " ".join(f"{v:.6f}" for v in r) for i, r in enumerate(rows[:50])]
    for header in ("", "50 24\n"):
        path = str(tmp_path / f"glove{len(header)}.txt")
        with open(path, "w") as fh:
            fh.write(header + "\n".join(lines) + "\n")
        f = datasets.TextEmbeddingFile(path)
        assert (f.N, f.D) == (50, 24)
        np.testing.assert_allclose(f.rows(0, 50), np.round(rows[:50], 6), atol=1e-6)
        np.testing.assert_allclose(f(7, 3), np.round(rows[7:10], 6), atol=1e-6)
        assert f.tokens(3, 2) == ["w3", "w4"]
        assert datasets.load_rows(path).shape == (50, 24)


@pytest.mark.gpu
def test_stream_em_from_an_fvecs_file(tmp_path, gpu_device):
    """Streaming EM over an .fvecs file (native source) equals in-memory EM on its rows."""
    from flash_gmm import em_iso, stream_em_iso
    g = torch.Generator().manual_seed(9)
    K, D, N = 48, 32, 60000
    centres = torch.randn(K, D, generator=g) * 2
    X = centres[torch.randint(0, K, (N,), generator=g)] + torch.randn(N, D, generator=g)
    path = str(tmp_path / "data.fvecs")
    datasets.write_vecs(path, X.numpy())
    dev = gpu_device
    mu = (centres + 0.5 * torch.randn(K, D, generator=g)).to(dev)
    lss = torch.zeros(K, device=dev)
    lpi = torch.full((K,), -float(np.log(K)), device=dev)
    mu_m, lss_m, lpi_m = mu.clone(), lss.clone(), lpi.clone()
    ll_m = em_iso(datasets.load_rows(path, device=dev), mu_m, lss_m, lpi_m, 2)
    with datasets.VecsFile(path) as f:
        rep = stream_em_iso(f, N, mu, lss, lpi, iterations=2, chunk_rows=16000)
    torch.cuda.synchronize()
    torch.testing.assert_close(mu, mu_m, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(lss, lss_m, rtol=0, atol=1e-4)
    np.testing.assert_allclose(rep["loglik"], ll_m, rtol=1e-6)


@pytest.mark.gpu
def test_stream_em_gist_width_file_against_the_oracle(tmp_path, gpu_device):
    """A GIST-width .fvecs file (D = 960, where pass 1 tiles over components) streamed
    through the EM driver in three chunks, one iteration: the parameters it applies and
    the log-likelihood it reports against the float64 oracle's E-step over the file's
    rows followed by the README M-step (README.md:59-61)."""
    import sys
    from flash_gmm import stream_em_iso
    from oracle import gmm_oracle as O
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from parity import logz_atol_fp32
    g = torch.Generator().manual_seed(11)
    K, D, N = 64, 960, 30000
    centres = torch.randn(K, D, generator=g) * 0.5
    X = centres[torch.randint(0, K, (N,), generator=g)] + torch.randn(N, D, generator=g)
    path = str(tmp_path / "gist_like.fvecs")
    datasets.write_vecs(path, X.numpy())
    mu0 = centres + 0.1 * torch.randn(K, D, generator=g)
    lss0 = torch.zeros(K)
    lpi0 = torch.full((K,), -float(np.log(K)))
    dev = gpu_device
    mu, lss, lpi = mu0.to(dev), lss0.to(dev), lpi0.to(dev)
    with datasets.VecsFile(path) as f:
        rep = stream_em_iso(f, N, mu, lss, lpi, iterations=1, chunk_rows=12000)
    torch.cuda.synchronize()
    logZ, Nk, mu_acc, sig = O.estep_iso(X, mu0, lss0, lpi0)
    assert float(Nk.min()) > 100          # every component is populated
    pi, m, s2 = O.mstep_iso(Nk, mu_acc, sig, N, D)
    scale = float(m.abs().max())
    assert float((mu.double().cpu() - m).abs().max()) <= 2e-4 * scale
    assert float((lss.double().cpu() - torch.log(s2)).abs().max()) <= 3e-4
    assert float((lpi.double().cpu() - torch.log(pi)).abs().max()) <= 2e-4
    # The log-likelihood is a sum of N logZ values: N times the logZ bound at this
    # width (the float32 restatement's error on these rows, above D = 128).
    lz32 = O.estep_iso(X, mu0, lss0, lpi0, dtype=torch.float32)[0]
    assert abs(rep["loglik"][0] - float(logZ.sum())) <= logz_atol_fp32(lz32, logZ, D) * N

"""EM on the device: M-steps for the three covariance models, in-memory EM loops
and the streaming isotropic EM driver for data sets larger than device memory.

The reference has no EM code; its README gives the M-step formulas
(README.md:59-61) and a chunked streaming recipe (README.md:81-103).  Here the
M-step is a HIP kernel and streaming is the native driver fgmm_stream_em_iso
(pinned double buffers, a copy stream and a compute stream), fed by a host row
source: the built-in counter-based generator (SynthIsoSource) or any Python
callable returning rows.
"""

from __future__ import annotations

import ctypes
from typing import Callable, Union

import numpy as np
import torch

from . import _lib
from ._lib import FlashGMMError
from .estep import diag_estep_into, full_estep_into, iso_estep_into

MSTEP_EXACT_VARIANCE = 1 << 8
MAX_REPORTED_ITERS = 16

ROW_SOURCE = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                              ctypes.c_int64, ctypes.POINTER(ctypes.c_float))


class _SynthIso(ctypes.Structure):
    _fields_ = [("centres", ctypes.c_void_p), ("K", ctypes.c_int64), ("D", ctypes.c_int64),
                ("seed", ctypes.c_uint64), ("threads", ctypes.c_int)]


class _EmConfig(ctypes.Structure):
    _fields_ = [("N", ctypes.c_int64), ("K", ctypes.c_int64), ("D", ctypes.c_int64),
                ("chunk_rows", ctypes.c_int64), ("iterations", ctypes.c_int),
                ("var_floor", ctypes.c_double), ("mstep_flags", ctypes.c_uint)]


class _EmReport(ctypes.Structure):
    _fields_ = [("iterations", ctypes.c_int), ("total_ms", ctypes.c_double),
                ("source_ms", ctypes.c_double), ("h2d_ms", ctypes.c_double),
                ("estep_ms", ctypes.c_double), ("mstep_ms", ctypes.c_double),
                ("device_bytes", ctypes.c_size_t), ("pinned_bytes", ctypes.c_size_t),
                ("loglik", ctypes.c_double * MAX_REPORTED_ITERS), ("setup_ms", ctypes.c_double)]


def _declare(L):
    if getattr(L, "_em_declared", False):
        return L
    L.fgmm_synth_iso_source.restype = ctypes.c_int
    L.fgmm_synth_iso_source.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_int64, ctypes.c_void_p]
    L.fgmm_iso_mstep_f32.restype = ctypes.c_int
    L.fgmm_iso_mstep_f32.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [
        ctypes.c_double, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_uint, ctypes.c_void_p]
    L.fgmm_diag_mstep_f32.restype = ctypes.c_int
    L.fgmm_diag_mstep_f32.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [
        ctypes.c_double, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
        ctypes.c_void_p, ctypes.c_uint, ctypes.c_void_p]
    L.fgmm_full_mstep_f32.restype = ctypes.c_int
    L.fgmm_full_mstep_f32.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [
        ctypes.c_double, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_void_p]
    L.fgmm_stream_em_iso.restype = ctypes.c_int
    L.fgmm_stream_em_iso.argtypes = [ctypes.POINTER(_EmConfig), ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.POINTER(_EmReport)]
    L._em_declared = True
    return L


class SynthIsoSource:
    """Clustered rows x_n = centres[a_n] + N(0, I), a_n uniform (native generator).

    Row n depends only on (seed, n): Philox4x32-10 keyed by the seed with the row
    index in the counter, so chunking and threading do not change the data.
    """

    def __init__(self, centres, seed: int = 4, threads: int = 0):
        c = np.ascontiguousarray(np.asarray(centres, dtype=np.float32))
        if c.ndim != 2:
            raise FlashGMMError("centres must be (K, D)")
        self.centres = c
        self.K, self.D = c.shape
        self._s = _SynthIso(c.ctypes.data, self.K, self.D, int(seed) & (2**64 - 1), int(threads))

    @property
    def fn(self):
        L = _declare(_lib.lib())
        return ctypes.cast(L.fgmm_synth_iso_source, ctypes.c_void_p).value

    @property
    def user(self):
        return ctypes.addressof(self._s)

    def rows(self, row0: int, nrows: int) -> np.ndarray:
        L = _declare(_lib.lib())
        out = np.empty((nrows, self.D), dtype=np.float32)
        st = L.fgmm_synth_iso_source(ctypes.addressof(self._s), row0, nrows, self.D, out.ctypes.data)
        _lib.check(st, "fgmm_synth_iso_source")
        return out


def mstep_iso(Nk, mu_acc, sig_acc, N: int, mu, log_sigma_sq, log_pi, *, var_floor: float = 0.0,
              exact_variance: bool = False) -> None:
    """Device M-step: updates mu, log_sigma_sq, log_pi in place (README.md:59-61)."""
    K, D = mu.shape
    for t in (Nk, mu_acc, sig_acc, mu, log_sigma_sq, log_pi):
        if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
            raise FlashGMMError("M-step tensors must be contiguous float32 on the GPU")
    L = _declare(_lib.lib())
    with torch.cuda.device(mu.device):
        st = L.fgmm_iso_mstep_f32(Nk.data_ptr(), mu_acc.data_ptr(), sig_acc.data_ptr(), int(N), K, D,
                                  float(var_floor), mu.data_ptr(), D, log_sigma_sq.data_ptr(),
                                  log_pi.data_ptr(), MSTEP_EXACT_VARIANCE if exact_variance else 0,
                                  _lib.stream_handle(mu.device))
    _lib.check(st, "fgmm_iso_mstep_f32")


def _check_dev_f32(*ts):
    for t in ts:
        if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
            raise FlashGMMError("M-step tensors must be contiguous float32 on the GPU")


def mstep_diag(Nk, mu_acc, sig_acc, N: int, mu, log_sigma_sq, log_pi, *, var_floor: float = 0.0,
               exact_variance: bool = False) -> None:
    """Device diagonal M-step: mu, log_sigma_sq (K x D) and log_pi updated in place."""
    K, D = mu.shape
    _check_dev_f32(Nk, mu_acc, sig_acc, mu, log_sigma_sq, log_pi)
    L = _declare(_lib.lib())
    with torch.cuda.device(mu.device):
        st = L.fgmm_diag_mstep_f32(Nk.data_ptr(), mu_acc.data_ptr(), sig_acc.data_ptr(), int(N), K, D,
                                   float(var_floor), mu.data_ptr(), D, log_sigma_sq.data_ptr(), D,
                                   log_pi.data_ptr(), MSTEP_EXACT_VARIANCE if exact_variance else 0,
                                   _lib.stream_handle(mu.device))
    _lib.check(st, "fgmm_diag_mstep_f32")


def mstep_full(Nk, mu_acc, sig_outer, N: int, mu, prec_chol, log_pi, *, reg_covar: float = 1e-6,
               info=None) -> None:
    """Device full-covariance M-step: mu, prec_chol (K x D x D, lower-triangular with
    L L^T = Sigma^-1) and log_pi updated in place.  ``info`` (an int32 device tensor of
    one element, zeroed by the caller) counts components whose covariance was not
    positive definite."""
    K, D = mu.shape
    _check_dev_f32(Nk, mu_acc, sig_outer, mu, prec_chol, log_pi)
    if info is not None and not (info.is_cuda and info.dtype == torch.int32 and info.numel() >= 1):
        raise FlashGMMError("info must be an int32 tensor on the GPU")
    L = _declare(_lib.lib())
    with torch.cuda.device(mu.device):
        st = L.fgmm_full_mstep_f32(Nk.data_ptr(), mu_acc.data_ptr(), sig_outer.data_ptr(), int(N), K, D,
                                   float(reg_covar), mu.data_ptr(), D, prec_chol.data_ptr(),
                                   log_pi.data_ptr(), info.data_ptr() if info is not None else None,
                                   _lib.stream_handle(mu.device))
    _lib.check(st, "fgmm_full_mstep_f32")


def em_diag(X, mu, log_sigma_sq, log_pi, iterations: int, *, var_floor: float = 0.0,
            exact_variance: bool = False):
    """In-memory diagonal-covariance EM; returns per-iteration log-likelihoods."""
    N, D = X.shape
    K = mu.shape[0]
    dev = X.device
    logZ, Nk = torch.empty(N, device=dev), torch.empty(K, device=dev)
    mu_acc, sig = torch.empty(K, D, device=dev), torch.empty(K, D, device=dev)
    out = []
    for _ in range(iterations):
        diag_estep_into(X, mu, log_sigma_sq, log_pi, logZ, Nk, mu_acc, sig)
        out.append(float(logZ.double().sum()))
        mstep_diag(Nk, mu_acc, sig, N, mu, log_sigma_sq, log_pi, var_floor=var_floor,
                   exact_variance=exact_variance)
    return out


def em_full(X, mu, prec_chol, log_pi, iterations: int, *, reg_covar: float = 1e-6):
    """In-memory full-covariance EM; returns per-iteration log-likelihoods."""
    N, D = X.shape
    K = mu.shape[0]
    dev = X.device
    logZ, Nk = torch.empty(N, device=dev), torch.empty(K, device=dev)
    mu_acc, so = torch.empty(K, D, device=dev), torch.empty(K, D, D, device=dev)
    out = []
    for _ in range(iterations):
        full_estep_into(X, mu, prec_chol, log_pi, logZ, Nk, mu_acc, so)
        out.append(float(logZ.double().sum()))
        mstep_full(Nk, mu_acc, so, N, mu, prec_chol, log_pi, reg_covar=reg_covar)
    return out


def em_iso(X, mu, log_sigma_sq, log_pi, iterations: int, *, var_floor: float = 0.0,
           exact_variance: bool = False):
    """In-memory EM: ``iterations`` rounds of E-step + device M-step.

    Updates mu / log_sigma_sq / log_pi in place and returns the per-iteration
    log-likelihoods sum_n logZ_n (each evaluated before that iteration's M-step).
    """
    N, D = X.shape
    K = mu.shape[0]
    dev = X.device
    logZ = torch.empty(N, device=dev)
    Nk = torch.empty(K, device=dev)
    mu_acc = torch.empty(K, D, device=dev)
    sig = torch.empty(K, device=dev)
    out = []
    for _ in range(iterations):
        iso_estep_into(X, mu, log_sigma_sq, log_pi, logZ, Nk, mu_acc, sig)
        out.append(float(logZ.double().sum()))
        mstep_iso(Nk, mu_acc, sig, N, mu, log_sigma_sq, log_pi, var_floor=var_floor,
                  exact_variance=exact_variance)
    return out


def stream_em_iso(source: Union[SynthIsoSource, Callable[[int, int], np.ndarray]], N: int, mu,
                  log_sigma_sq, log_pi, *, iterations: int = 3, chunk_rows: int = 16 << 20,
                  var_floor: float = 0.0, exact_variance: bool = False) -> dict:
    """Streaming EM over N host rows; updates mu / log_sigma_sq / log_pi in place.

    ``source`` is a native source (SynthIsoSource, datasets.VecsFile over a local
    .fvecs / .bvecs / .fbin / .u8bin file) or a callable ``f(row0, nrows) ->
    (nrows, D)`` float32 array (datasets.TextEmbeddingFile is one).  Returns the
    driver's timing / memory report.
    """
    K, D = mu.shape
    for t in (mu, log_sigma_sq, log_pi):
        if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
            raise FlashGMMError("parameters must be contiguous float32 on the GPU")
    L = _declare(_lib.lib())
    cfg = _EmConfig(int(N), K, D, int(chunk_rows), int(iterations), float(var_floor),
                    MSTEP_EXACT_VARIANCE if exact_variance else 0)
    rep = _EmReport()
    keep = None
    if hasattr(source, "fn") and hasattr(source, "user"):
        # A native source (SynthIsoSource, datasets.VecsFile): the C callback runs
        # on the driver's thread with no Python in between.
        if source.D != D:
            raise FlashGMMError("source dimension does not match mu")
        if getattr(source, "N", N) < N:
            raise FlashGMMError(f"the source holds {source.N} rows, fewer than N={N}")
        fn, user = source.fn, source.user
    else:
        def _cb(user, row0, nrows, d, dst):
            try:
                rows = np.ascontiguousarray(source(int(row0), int(nrows)), dtype=np.float32).reshape(-1)
                if rows.size != nrows * d:
                    return 1
                ctypes.memmove(dst, rows.ctypes.data, rows.nbytes)
                return 0
            except Exception:  # any failure aborts the stream with FGMM_ERR_SOURCE
                return 1
        keep = ROW_SOURCE(_cb)
        fn, user = ctypes.cast(keep, ctypes.c_void_p).value, None
    torch.cuda.synchronize(mu.device)
    with torch.cuda.device(mu.device):
        st = L.fgmm_stream_em_iso(ctypes.byref(cfg), fn, user, mu.data_ptr(), log_sigma_sq.data_ptr(),
                                  log_pi.data_ptr(), ctypes.byref(rep))
    del keep
    _lib.check(st, "fgmm_stream_em_iso")
    return {
        "iterations": rep.iterations, "total_ms": rep.total_ms, "setup_ms": rep.setup_ms,
        "source_ms": rep.source_ms,
        "h2d_ms": rep.h2d_ms, "estep_ms": rep.estep_ms, "mstep_ms": rep.mstep_ms,
        "device_bytes": rep.device_bytes, "pinned_bytes": rep.pinned_bytes,
        "loglik": [rep.loglik[i] for i in range(min(rep.iterations, MAX_REPORTED_ITERS))],
    }

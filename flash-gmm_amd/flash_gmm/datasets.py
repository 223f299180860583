"""Local embedding files as row sources.

The reference tunes its kernels on SIFT1M, GloVe and Deep10M
(flash_gmm_diag_h100.py:17, :299-301; flash_gmm_h100.py:273) but ships no reader.
These readers take the layouts those sets are distributed in, from local files
(nothing is downloaded):

* ``VecsFile`` -- .fvecs / .bvecs (SIFT, GIST: per vector an int32 dimension, then
  the values) and .fbin / .u8bin (Deep: a uint32 count and dimension, then the
  values), memory-mapped by the native library (fgmm_vecs_open); it serves as the
  row source of ``stream_em_iso`` through the C callback, with no Python on the
  streaming path, and ``rows()`` returns any range as float32.
* ``TextEmbeddingFile`` -- GloVe / word2vec text: one vector per line, a token then
  D numbers (an optional "count dimension" first line is skipped); a line-offset
  index makes any row range readable.  It is a Python source (a callable).
* ``load_rows`` -- a whole file (or a range) as a float32 tensor, on the device
  when asked, for the in-memory E-step.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import FlashGMMError

FVECS, BVECS, FBIN, U8BIN = 0, 1, 2, 3
_EXT = {".fvecs": FVECS, ".bvecs": BVECS, ".fbin": FBIN, ".u8bin": U8BIN}


class _VecsFile(ctypes.Structure):
    _fields_ = [("base", ctypes.c_void_p), ("bytes", ctypes.c_size_t), ("N", ctypes.c_int64),
                ("D", ctypes.c_int64), ("format", ctypes.c_int), ("threads", ctypes.c_int)]


def _declare(L):
    if getattr(L, "_vecs_declared", False):
        return L
    L.fgmm_vecs_open.restype = ctypes.c_int
    L.fgmm_vecs_open.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_VecsFile)]
    L.fgmm_vecs_source.restype = ctypes.c_int
    L.fgmm_vecs_source.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                   ctypes.c_void_p]
    L.fgmm_vecs_close.restype = None
    L.fgmm_vecs_close.argtypes = [ctypes.POINTER(_VecsFile)]
    L._vecs_declared = True
    return L


def vecs_format(path: str) -> int:
    ext = os.path.splitext(path)[1].lower()
    if ext not in _EXT:
        raise FlashGMMError(f"unknown vector file extension {ext!r} (expected one of {sorted(_EXT)})")
    return _EXT[ext]


class VecsFile:
    """A memory-mapped .fvecs / .bvecs / .fbin / .u8bin file (native reader).

    ``N`` and ``D`` come from the file; byte-valued formats are returned as floats.
    Usable as ``stream_em_iso(VecsFile(path), N, ...)`` (its ``fn`` / ``user`` are the
    native callback and its state) and as ``f(row0, nrows)``.
    """

    def __init__(self, path: str, fmt: Optional[int] = None, threads: int = 0):
        self.path = path
        L = _declare(_lib.lib())
        self._f = _VecsFile()
        st = L.fgmm_vecs_open(os.fsencode(path), vecs_format(path) if fmt is None else int(fmt),
                              int(threads), ctypes.byref(self._f))
        _lib.check(st, f"fgmm_vecs_open({path!r})")
        self.N, self.D = int(self._f.N), int(self._f.D)

    @property
    def fn(self):
        return ctypes.cast(_declare(_lib.lib()).fgmm_vecs_source, ctypes.c_void_p).value

    @property
    def user(self):
        return ctypes.addressof(self._f)

    def rows(self, row0: int, nrows: int) -> np.ndarray:
        if self._f.base is None:
            raise FlashGMMError("file is closed")
        out = np.empty((nrows, self.D), dtype=np.float32)
        st = _declare(_lib.lib()).fgmm_vecs_source(self.user, int(row0), int(nrows), self.D, out.ctypes.data)
        _lib.check(st, "fgmm_vecs_source")
        return out

    __call__ = rows

    def close(self):
        if self._f.base:
            _declare(_lib.lib()).fgmm_vecs_close(ctypes.byref(self._f))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class TextEmbeddingFile:
    """GloVe / word2vec text embeddings: ``token v1 ... vD`` per line.

    A first line of exactly two integers (word2vec's "count dimension" header) is
    skipped.  Opening builds an index of line offsets (8 bytes per row); ``rows``
    parses any range.  ``tokens(row0, nrows)`` returns the tokens.
    """

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as fh:
            data = fh.read()
        starts = np.concatenate(([0], np.flatnonzero(np.frombuffer(data, dtype=np.uint8) == 10) + 1))
        starts = starts[starts < len(data)]
        first = data[starts[0]:starts[1] if len(starts) > 1 else len(data)].split()
        if len(first) == 2 and all(t.isdigit() for t in first):
            starts = starts[1:]
        if len(starts) == 0:
            raise FlashGMMError(f"{path}: no vectors")
        self._data = data
        self._starts = starts
        self.N = len(starts)
        self.D = len(data[starts[0]:self._end(0)].split()) - 1
        if self.D < 1:
            raise FlashGMMError(f"{path}: first line has no values")

    def _end(self, i):
        return self._starts[i + 1] if i + 1 < self.N else len(self._data)

    def rows(self, row0: int, nrows: int) -> np.ndarray:
        if row0 < 0 or nrows < 0 or row0 + nrows > self.N:
            raise FlashGMMError(f"rows [{row0}, {row0 + nrows}) outside [0, {self.N})")
        out = np.empty((nrows, self.D), dtype=np.float32)
        for i in range(nrows):
            parts = self._data[self._starts[row0 + i]:self._end(row0 + i)].split()
            if len(parts) != self.D + 1:
                raise FlashGMMError(f"{self.path}: line {row0 + i} has {len(parts) - 1} values, expected {self.D}")
            out[i] = np.array(parts[1:], dtype=np.float32)
        return out

    __call__ = rows

    def tokens(self, row0: int, nrows: int):
        return [self._data[self._starts[i]:self._end(i)].split(maxsplit=1)[0].decode("utf-8", "replace")
                for i in range(row0, row0 + nrows)]


def open_rows(path: str, threads: int = 0):
    """A row source for ``path``: VecsFile for the binary layouts, TextEmbeddingFile
    for .txt / .vec text."""
    ext = os.path.splitext(path)[1].lower()
    if ext in _EXT:
        return VecsFile(path, threads=threads)
    if ext in (".txt", ".vec"):
        return TextEmbeddingFile(path)
    raise FlashGMMError(f"unknown embedding file extension {ext!r}")


def load_rows(path: str, row0: int = 0, nrows: Optional[int] = None, device=None) -> torch.Tensor:
    """Rows [row0, row0 + nrows) of an embedding file (all of it by default) as a
    float32 (nrows, D) tensor, moved to ``device`` when given."""
    src = open_rows(path)
    n = src.N - row0 if nrows is None else nrows
    t = torch.from_numpy(src.rows(row0, n))
    if isinstance(src, VecsFile):
        src.close()
    return t.to(device) if device is not None else t


def write_vecs(path: str, X) -> None:
    """Write rows as .fvecs / .bvecs / .fbin / .u8bin (by extension)."""
    fmt = vecs_format(path)
    X = np.asarray(X)
    n, d = X.shape
    vals = X.astype(np.float32 if fmt in (FVECS, FBIN) else np.uint8)
    with open(path, "wb") as fh:
        if fmt in (FBIN, U8BIN):
            fh.write(np.array([n, d], dtype=np.uint32).tobytes())
            fh.write(np.ascontiguousarray(vals).tobytes())
        else:
            rec = np.empty((n, 4 + d * vals.itemsize), dtype=np.uint8)
            rec[:, :4] = np.frombuffer(np.int32(d).tobytes(), dtype=np.uint8)
            rec[:, 4:] = np.ascontiguousarray(vals).view(np.uint8).reshape(n, -1)
            fh.write(rec.tobytes())

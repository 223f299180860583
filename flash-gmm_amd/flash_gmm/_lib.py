"""ctypes binding of libflashgmm.so (the C ABI declared in include/flashgmm.h).

``torch`` is imported first on purpose: it loads its HIP runtime
(libamdhip64.so.7), and the dynamic loader then resolves this library's
dependency on the same soname to that already-loaded runtime, so torch's
streams and device pointers are valid here.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libflashgmm.so")

FGMM_OK = 0
FGMM_ERR_INVALID_ARG = -1
FGMM_ERR_UNSUPPORTED = -2
FGMM_ERR_WORKSPACE = -3
FGMM_ERR_HIP = -4
FGMM_ERR_SOURCE = -5
FGMM_ERR_SCRATCH = -6

FLAG_ACCUMULATE = 1 << 0
FLAG_NO_LOGZ = 1 << 1
FLAG_ATOMIC_REDUCE = 1 << 2
FLAG_PHASE1 = 1 << 3
FLAG_PHASE2 = 1 << 4
FLAG_DENSE = 1 << 5
FLAG_RECOMPUTE = 1 << 6
FLAG_BF16 = 1 << 7
FLAG_STORE_LOGJOINT = 1 << 9
FLAG_STORE_LOGJOINT_AUTO = 1 << 10


class FlashGMMError(AssertionError, ValueError):
    """Raised for invalid arguments or a failed native call.

    Derives from AssertionError because the reference reports its argument
    checks with ``assert`` (flash_gmm.py:189-190, flash_gmm_diag_h100.py:313,
    flash_gmm_full_h100.py:264), and from ValueError for ordinary callers.
    """


_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_u32 = ctypes.c_uint


def _declare(lib):
    lib.fgmm_version.restype = ctypes.c_int
    lib.fgmm_version.argtypes = []
    lib.fgmm_strerror.restype = ctypes.c_char_p
    lib.fgmm_strerror.argtypes = [ctypes.c_int]

    lib.fgmm_iso_workspace_bytes.restype = _sz
    lib.fgmm_iso_workspace_bytes.argtypes = [_i64, _i64, _i64]
    lib.fgmm_iso_workspace_bytes_ex.restype = _sz
    lib.fgmm_iso_workspace_bytes_ex.argtypes = [_i64, _i64, _i64, _u32]
    lib.fgmm_iso_estep_f32.restype = ctypes.c_int
    lib.fgmm_iso_estep_f32.argtypes = [
        _p, _i64, _i64, _i64,          # X, ldx, N, D
        _p, _i64, _i64,                # mu, ldmu, K
        _p, _p,                        # log_sigma_sq, log_pi
        _p, _p, _p, _p,                # logZ, Nk, mu_acc, sig_acc
        _p, _sz, _u32, _p,             # workspace, bytes, flags, stream
    ]
    decls = {
        "fgmm_diag_workspace_bytes": (_sz, [_i64, _i64, _i64]),
        "fgmm_diag_workspace_bytes_ex": (_sz, [_i64, _i64, _i64, _u32]),
        "fgmm_diag_estep_f32": (ctypes.c_int, [
            _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _p,
            _p, _p, _p, _p, _p, _sz, _u32, _p]),
        "fgmm_full_workspace_bytes": (_sz, [_i64, _i64, _i64]),
        "fgmm_full_workspace_bytes_ex": (_sz, [_i64, _i64, _i64, _u32]),
        "fgmm_full_estep_f32": (ctypes.c_int, [
            _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _p,
            _p, _p, _p, _p, _p, _sz, _u32, _p]),
        "fgmm_iso_estep_f32_noalloc": (ctypes.c_int, [
            _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _p,
            _p, _p, _p, _p, _u32, _p]),
        # The EM entry points (fgmm_iso_mstep_f32, fgmm_stream_em_iso,
        # fgmm_synth_iso_source) are declared in em.py next to their structs.
    }
    for name, (res, args) in decls.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def lib():
    """Load (once) and return the native library; raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FlashGMMError(
                f"native library not found at {LIB_PATH}; build it with "
                "`make -C flash-gmm_amd` (or __graft_entry__.build())")
        _lib = _declare(ctypes.CDLL(LIB_PATH))
    return _lib


def check(status: int, what: str) -> None:
    if status != FGMM_OK:
        msg = lib().fgmm_strerror(int(status)).decode()
        raise FlashGMMError(f"{what} failed: {msg} (status {status})")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream

"""Drop-in E-step entry points backed by the HIP kernels in libflashgmm.so.

Names, positional order, return tuples and argument checks follow the
reference:

* ``flash_gmm_estep(X, mu, log_sigma_sq, log_pi, BLOCK_N=64, BLOCK_K=16,
  BLOCK_D=128)`` -- flash_gmm.py:173-217 (and the 4-argument form of
  flash_gmm_h100.py:254-328).  The BLOCK_* keywords are accepted for
  compatibility and ignored: tiles are chosen by the library, and D is not
  limited by BLOCK_D (the same-named H100 entry sizes BLOCK_D from D,
  flash_gmm_h100.py:268-270).
* ``flash_gmm_estep_diag(X, mu, log_sigma_sq, log_pi)`` with log_sigma_sq of
  shape (K, D) -- flash_gmm_diag_h100.py:305-384; sig_acc is (K, D).
* ``flash_gmm_estep_full(X, mu, prec_chol, log_pi)`` with prec_chol (K, D, D)
  lower-triangular, L L^T = Sigma^-1 -- flash_gmm_full_h100.py:235-336; the
  fourth output is sig_outer (K, D, D) = sum_n r_nk x_n x_n^T.

Outputs are fresh float32 tensors on X.device (flash_gmm.py:192-195), written
asynchronously on torch's current stream; nothing synchronises.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import FlashGMMError

__all__ = ["flash_gmm_estep", "iso_estep_into", "flash_gmm_estep_diag", "diag_estep_into",
           "flash_gmm_estep_full", "full_estep_into"]


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise FlashGMMError(msg)


def _f32(t: torch.Tensor) -> torch.Tensor:
    """float32 view of a floating tensor (a converted copy for other dtypes): the
    kernels compute in float32, as the reference does (its wrappers assume float32
    inputs, flash_gmm.py:187-195)."""
    return t if t.dtype == torch.float32 else t.float()


def _prep_rows(X: torch.Tensor):
    """Return (X, ldx) when the kernels can read X in place, else a padded copy.

    The kernels read 16-byte row chunks: they need a unit column stride, a row
    stride that is a multiple of 4 elements and at least round_up(D, 4), and a
    16-byte aligned base.  In place is used only when D % 4 == 0, so a chunk
    never reaches past the last element of the tensor.  The reference accepts
    any strides (flash_gmm.py:202); other layouts are copied.
    """
    N, D = X.shape
    D4 = (D + 3) // 4 * 4
    if N == 0:
        return X, D4
    if D % 4 == 0 and X.data_ptr() % 16 == 0 and X.stride(1) == 1:
        if N == 1:
            return X, D4
        if X.stride(0) % 4 == 0 and X.stride(0) >= D4:
            return X, X.stride(0)
    Xp = torch.empty(N, D4, device=X.device, dtype=torch.float32)
    Xp[:, :D] = X
    return Xp, D4


def _check_common(X, mu, log_pi):
    _require(X.dim() == 2 and mu.dim() == 2, "X must be (N, D) and mu (K, D)")
    _require(X.is_cuda and mu.is_cuda, "Inputs must be on GPU.")  # flash_gmm.py:190
    _require(X.is_floating_point() and mu.is_floating_point(),
             "X and mu must be floating point (they are computed on in float32)")
    _require(mu.shape[1] == X.shape[1], f"mu must be (K, D) with D={X.shape[1]}, got {tuple(mu.shape)}")
    _require(mu.device == X.device, "X and mu must be on the same device")
    K = mu.shape[0]
    _require(log_pi.shape == (K,), f"log_pi must be ({K},), got {tuple(log_pi.shape)}")


def _vec(t: torch.Tensor, device, shape, name) -> torch.Tensor:
    _require(tuple(t.shape) == tuple(shape), f"{name} must be {tuple(shape)}, got {tuple(t.shape)}")
    return t.to(device=device, dtype=torch.float32).contiguous()


def _flags(accumulate, logZ, atomic_reduce, phase):
    flags = 0
    if accumulate:
        flags |= _lib.FLAG_ACCUMULATE
    if logZ is None:
        flags |= _lib.FLAG_NO_LOGZ
    if atomic_reduce:
        flags |= _lib.FLAG_ATOMIC_REDUCE
    if phase == 1:
        flags |= _lib.FLAG_PHASE1
    elif phase == 2:
        flags |= _lib.FLAG_PHASE2
    elif phase != 0:
        raise FlashGMMError(f"phase must be 0, 1 or 2, got {phase}")
    return flags


def _check_out(name, t, shape, dev):
    _require(t is not None and tuple(t.shape) == tuple(shape) and t.dtype == torch.float32
             and t.is_contiguous() and t.device == dev,
             f"{name} must be a contiguous float32 {tuple(shape)} tensor on {dev}")


def _empty_workspace(nbytes, dev):
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)


def _workspace(ws_fn, N, K, D, flags, dev, workspace):
    """Return (workspace, flags).

    The size depends on the device's compute-unit count, so it is queried with dev
    current.  A phase-2 call must reuse the workspace its phase-1 call filled.  When
    the stored log-joint's O(N*K) workspace cannot be allocated, the call falls back
    to the default O(N + K*D) plan (same results to the float32 bounds)."""
    with torch.cuda.device(dev):
        ws_bytes = int(ws_fn(N, K, D, flags))
    if flags & _lib.FLAG_PHASE2 and not flags & _lib.FLAG_PHASE1:
        _require(workspace is not None and workspace.numel() >= ws_bytes,
                 "phase=2 needs the workspace filled by the phase-1 call on the same inputs "
                 f"({ws_bytes} bytes)")
        return workspace, flags
    if workspace is not None and workspace.numel() >= ws_bytes:
        return workspace, flags
    try:
        return _empty_workspace(ws_bytes, dev), flags
    except torch.cuda.OutOfMemoryError:
        stored = _lib.FLAG_STORE_LOGJOINT | _lib.FLAG_STORE_LOGJOINT_AUTO
        if not flags & stored or flags & (_lib.FLAG_PHASE1 | _lib.FLAG_PHASE2):
            raise
        lean = flags & ~stored
        with torch.cuda.device(dev):
            lean_bytes = int(ws_fn(N, K, D, lean))
        if workspace is not None and workspace.numel() >= lean_bytes:
            return workspace, lean
        return _empty_workspace(lean_bytes, dev), lean


def _plan_flags(flags, dense, recompute, store_log_joint, precision):
    _require(store_log_joint in (True, False, "auto"),
             f"store_log_joint must be True, False or 'auto', got {store_log_joint!r}")
    if dense:
        flags |= _lib.FLAG_DENSE
    if recompute:
        flags |= _lib.FLAG_RECOMPUTE
    elif store_log_joint == "auto":
        flags |= _lib.FLAG_STORE_LOGJOINT_AUTO
    elif store_log_joint:
        flags |= _lib.FLAG_STORE_LOGJOINT
    if precision == "bf16":
        flags |= _lib.FLAG_BF16
    return flags


def _ptr(t, cond=True):
    return t.data_ptr() if (t is not None and cond) else None


def _rowmajor(t: torch.Tensor) -> torch.Tensor:
    """Unit stride along the last dimension (any row stride)."""
    return t if (t.dim() == 0 or t.stride(-1) == 1 or t.shape[-1] == 1) else t.contiguous()


def iso_estep_into(X, mu, log_sigma_sq, log_pi, logZ, Nk, mu_acc, sig_acc, *,
                   accumulate: bool = False, atomic_reduce: bool = False,
                   workspace: torch.Tensor | None = None, phase: int = 0,
                   dense: bool = False, recompute: bool = False,
                   store_log_joint: bool | str = False, precision: str = "fp32") -> None:
    """Isotropic E-step writing into caller-provided outputs.

    ``logZ`` may be None (it is then not written).  With ``accumulate`` the
    statistics are added to the current contents of Nk / mu_acc / sig_acc
    (streaming over row chunks, README.md:86-96).  ``phase`` 1 runs only the
    log-normaliser pass, 2 only the accumulation (reusing ``workspace`` from a
    phase-1 call on the same inputs), 0 both.  ``dense`` runs the accumulation
    steps whose responsibilities are all exactly zero instead of skipping them
    (same results; for timing).  By default the workspace is O(N + K*D) and the
    accumulation pass recomputes the log-joint where pass 1 found a possibly
    nonzero responsibility (``recompute=True`` asks for this explicitly).
    ``store_log_joint`` makes pass 1 store the fp32 N x K log-joint in the
    workspace for pass 2 to read (O(N*K) workspace, 4.3 GB at N=1M, K=1024;
    phase-split calls must agree).  ``store_log_joint="auto"`` (up to D = 128)
    reserves that workspace and lets a row-sample probe on the device choose per
    call: the stored branch where most (row, component block) pairs are needed
    (dense data), the default plan otherwise.
    ``precision="bf16"`` selects the bf16 operand contract of the reference's H100
    kernels (flash_gmm_h100.py:247-328): X and mu rounded to bfloat16 for the
    contractions, fp32 accumulation and log-sum-exp.
    """
    _check_common(X, mu, log_pi)
    _require(precision in ("fp32", "bf16"), f"precision must be 'fp32' or 'bf16', got {precision!r}")
    N, D = X.shape
    K = mu.shape[0]
    dev = X.device
    lss = _vec(log_sigma_sq, dev, (K,), "log_sigma_sq")
    lpi = _vec(log_pi, dev, (K,), "log_pi")
    Xk, ldx = _prep_rows(_f32(X))
    muk = _rowmajor(_f32(mu))
    ldmu = muk.stride(0) if K > 1 else D
    L = _lib.lib()
    flags = _plan_flags(_flags(accumulate, logZ, atomic_reduce, phase), dense, recompute,
                        store_log_joint, precision)
    workspace, flags = _workspace(L.fgmm_iso_workspace_bytes_ex, N, K, D, flags, dev, workspace)
    _check_out("Nk", Nk, (K,), dev)
    _check_out("mu_acc", mu_acc, (K, D), dev)
    _check_out("sig_acc", sig_acc, (K,), dev)
    if logZ is not None:
        _check_out("logZ", logZ, (N,), dev)
    with torch.cuda.device(dev):
        st = L.fgmm_iso_estep_f32(
            _ptr(Xk, N > 0), ldx, N, D, _ptr(muk, K > 0), ldmu, K,
            _ptr(lss, K > 0), _ptr(lpi, K > 0), _ptr(logZ, N > 0),
            _ptr(Nk, K > 0), _ptr(mu_acc, K > 0), _ptr(sig_acc, K > 0),
            workspace.data_ptr(), workspace.numel(), flags, _lib.stream_handle(dev))
    _lib.check(st, "fgmm_iso_estep_f32")


# The drop-in call reserves the stored log-joint's workspace (store_log_joint="auto")
# while it takes at most this fraction of the device's memory.
AUTO_STORE_MEMORY_FRACTION = 1.0 / 8


def _auto_store(N, K, D, dev, precision, model="iso"):
    """store_log_joint for the drop-in call: "auto" where its workspace is modest."""
    if precision != "fp32" or N == 0 or K == 0:
        return False
    L = _lib.lib()
    ws_ex = getattr(L, f"fgmm_{model}_workspace_bytes_ex")
    ws = getattr(L, f"fgmm_{model}_workspace_bytes")
    with torch.cuda.device(dev):
        extra = int(ws_ex(N, K, D, _lib.FLAG_STORE_LOGJOINT_AUTO)) - int(ws(N, K, D))
        total = torch.cuda.get_device_properties(dev).total_memory
    return "auto" if 0 < extra <= total * AUTO_STORE_MEMORY_FRACTION else False


def flash_gmm_estep(X: torch.Tensor, mu: torch.Tensor, log_sigma_sq: torch.Tensor,
                    log_pi: torch.Tensor, BLOCK_N: int = 64, BLOCK_K: int = 16,
                    BLOCK_D: int = 128, *, precision: str = "fp32"):
    """Flash-GMM isotropic E-step: returns (logZ, Nk, mu_acc, sig_acc).

    logZ (N,) per-sample log-normaliser, Nk (K,) = sum_n r_nk,
    mu_acc (K, D) = sum_n r_nk x_n, sig_acc (K,) = sum_n r_nk ||x_n - mu_k||^2
    (flash_gmm.py:22-37).  BLOCK_N / BLOCK_K / BLOCK_D are ignored.
    ``precision="bf16"`` follows the bf16 operand contract of the H100 variant
    (flash_gmm_h100.py:247-328) instead of fp32 arithmetic.  Up to D = 128 the
    call runs with store_log_joint="auto" (see iso_estep_into) while that
    workspace takes at most AUTO_STORE_MEMORY_FRACTION of the device's memory.
    """
    _check_common(X, mu, log_pi)
    N, D = X.shape
    K = mu.shape[0]
    dev = X.device
    logZ = torch.empty(N, device=dev, dtype=torch.float32)
    Nk = torch.empty(K, device=dev, dtype=torch.float32)
    mu_acc = torch.empty(K, D, device=dev, dtype=torch.float32)
    sig_acc = torch.empty(K, device=dev, dtype=torch.float32)
    iso_estep_into(X, mu, log_sigma_sq, log_pi, logZ, Nk, mu_acc, sig_acc, precision=precision,
                   store_log_joint=_auto_store(N, K, D, dev, precision))
    return logZ, Nk, mu_acc, sig_acc


def diag_estep_into(X, mu, log_sigma_sq, log_pi, logZ, Nk, mu_acc, sig_acc, *,
                    accumulate: bool = False, atomic_reduce: bool = False,
                    workspace: torch.Tensor | None = None, phase: int = 0, dense: bool = False,
                    recompute: bool = False, store_log_joint: bool | str = False,
                    precision: str = "fp32") -> None:
    """Diagonal-covariance E-step into caller-provided outputs (sig_acc is (K, D)).

    The plan arguments are iso_estep_into's; ``store_log_joint="auto"`` applies up
    to D = 96 (above, the call runs the default plan).

    ``precision="bf16"`` selects the bf16 operand contract of the reference's
    diagonal H100 kernels (flash_gmm_diag_h100.py:63-130, :159-282): x, x^2 and the
    weights exp(-lss)/2 log2 e and mu exp(-lss)/2 log2 e rounded to bfloat16, r
    rounded to bfloat16 for r^T x and r^T x^2, fp32 accumulation and log-sum-exp.
    The accumulation then always recomputes the contraction (``recompute`` has no
    effect).
    """
    _check_common(X, mu, log_pi)
    _require(precision in ("fp32", "bf16"), f"precision must be 'fp32' or 'bf16', got {precision!r}")
    N, D = X.shape
    K = mu.shape[0]
    dev = X.device
    _require(tuple(log_sigma_sq.shape) == (K, D),
             f"log_sigma_sq must be (K, D)=({K}, {D}), got {tuple(log_sigma_sq.shape)}")
    lss = _rowmajor(log_sigma_sq.to(device=dev, dtype=torch.float32))
    ldlss = lss.stride(0) if K > 1 else D
    lpi = _vec(log_pi, dev, (K,), "log_pi")
    Xk, ldx = _prep_rows(_f32(X))
    muk = _rowmajor(_f32(mu))
    ldmu = muk.stride(0) if K > 1 else D
    L = _lib.lib()
    _require(hasattr(L, "fgmm_diag_estep_f32"), "library built without the diagonal E-step")
    flags = _plan_flags(_flags(accumulate, logZ, atomic_reduce, phase), dense, recompute, store_log_joint,
                        precision)
    workspace, flags = _workspace(L.fgmm_diag_workspace_bytes_ex, N, K, D, flags, dev, workspace)
    _check_out("Nk", Nk, (K,), dev)
    _check_out("mu_acc", mu_acc, (K, D), dev)
    _check_out("sig_acc", sig_acc, (K, D), dev)
    if logZ is not None:
        _check_out("logZ", logZ, (N,), dev)
    with torch.cuda.device(dev):
        st = L.fgmm_diag_estep_f32(
            _ptr(Xk, N > 0), ldx, N, D, _ptr(muk, K > 0), ldmu, K, _ptr(lss, K > 0), ldlss,
            _ptr(lpi, K > 0), _ptr(logZ, N > 0), _ptr(Nk, K > 0), _ptr(mu_acc, K > 0),
            _ptr(sig_acc, K > 0), workspace.data_ptr(), workspace.numel(), flags,
            _lib.stream_handle(dev))
    _lib.check(st, "fgmm_diag_estep_f32")


def flash_gmm_estep_diag(X: torch.Tensor, mu: torch.Tensor, log_sigma_sq: torch.Tensor,
                         log_pi: torch.Tensor, *, precision: str = "fp32"):
    """Diagonal-covariance E-step: returns (logZ, Nk, mu_acc, sig_acc[K, D]).

    sig_acc[k, d] = sum_n r_nk (x_nd - mu_kd)^2 (flash_gmm_diag_h100.py:258-260).
    ``precision="bf16"`` follows the reference kernels' bf16 operand contract
    instead of fp32 arithmetic.  Up to D = 96 the call runs with
    store_log_joint="auto" (see diag_estep_into) while that workspace takes at most
    AUTO_STORE_MEMORY_FRACTION of the device's memory.
    """
    _check_common(X, mu, log_pi)
    N, D = X.shape
    K = mu.shape[0]
    _require(tuple(log_sigma_sq.shape) == (K, D),
             f"log_sigma_sq must be (K, D)=({K}, {D}), got {tuple(log_sigma_sq.shape)}")
    dev = X.device
    logZ = torch.empty(N, device=dev, dtype=torch.float32)
    Nk = torch.empty(K, device=dev, dtype=torch.float32)
    mu_acc = torch.empty(K, D, device=dev, dtype=torch.float32)
    sig_acc = torch.empty(K, D, device=dev, dtype=torch.float32)
    diag_estep_into(X, mu, log_sigma_sq, log_pi, logZ, Nk, mu_acc, sig_acc, precision=precision,
                    store_log_joint=_auto_store(N, K, D, dev, precision, "diag"))
    return logZ, Nk, mu_acc, sig_acc


def full_estep_into(X, mu, prec_chol, log_pi, logZ, Nk, mu_acc, sig_outer, *,
                    accumulate: bool = False, atomic_reduce: bool = False,
                    workspace: torch.Tensor | None = None, phase: int = 0, dense: bool = False,
                    recompute: bool = False, store_log_joint: bool | str = False,
                    precision: str = "fp32") -> None:
    """Full-covariance E-step into caller-provided outputs (sig_outer is (K, D, D)).

    The plan arguments are iso_estep_into's; ``store_log_joint="auto"`` applies up
    to D = 64 and K = 512 (elsewhere the call runs the default plan).

    ``precision="bf16"`` selects the bf16 operand contract of the reference's full
    H100 kernels (flash_gmm_full_h100.py:71-228): x and L rounded to bfloat16 for the
    whitening, L^T mu in float32, r rounded to bfloat16 for mu_acc and r x_d2 for
    sig_outer[k, d2, :] (which is then not exactly symmetric), fp32 accumulation and
    log-sum-exp.  That path always stores the log-joint (``recompute`` has no
    effect), at most 16 GiB of it at a time: the library runs larger N as row chunks
    of 16 GiB / (4 K) rows on one workspace, each chunk adding its statistics to the
    outputs, so the sums round once per chunk (a ``phase`` split of such a call is
    refused).
    """
    _check_common(X, mu, log_pi)
    _require(precision in ("fp32", "bf16"), f"precision must be 'fp32' or 'bf16', got {precision!r}")
    N, D = X.shape
    K = mu.shape[0]
    dev = X.device
    _require(tuple(prec_chol.shape) == (K, D, D),
             f"prec_chol must be (K, D, D)=({K}, {D}, {D}), got {tuple(prec_chol.shape)}")
    Lc = prec_chol.to(device=dev, dtype=torch.float32).contiguous()
    lpi = _vec(log_pi, dev, (K,), "log_pi")
    Xk, ldx = _prep_rows(_f32(X))
    muk = _rowmajor(_f32(mu))
    ldmu = muk.stride(0) if K > 1 else D
    L = _lib.lib()
    _require(hasattr(L, "fgmm_full_estep_f32"), "library built without the full-covariance E-step")
    flags = _plan_flags(_flags(accumulate, logZ, atomic_reduce, phase), dense, recompute, store_log_joint,
                        precision)
    workspace, flags = _workspace(L.fgmm_full_workspace_bytes_ex, N, K, D, flags, dev, workspace)
    _check_out("Nk", Nk, (K,), dev)
    _check_out("mu_acc", mu_acc, (K, D), dev)
    _check_out("sig_outer", sig_outer, (K, D, D), dev)
    if logZ is not None:
        _check_out("logZ", logZ, (N,), dev)
    with torch.cuda.device(dev):
        st = L.fgmm_full_estep_f32(
            _ptr(Xk, N > 0), ldx, N, D, _ptr(muk, K > 0), ldmu, K, _ptr(Lc, K > 0),
            _ptr(lpi, K > 0), _ptr(logZ, N > 0), _ptr(Nk, K > 0), _ptr(mu_acc, K > 0),
            _ptr(sig_outer, K > 0), workspace.data_ptr(), workspace.numel(), flags,
            _lib.stream_handle(dev))
    _lib.check(st, "fgmm_full_estep_f32")


def flash_gmm_estep_full(X: torch.Tensor, mu: torch.Tensor, prec_chol: torch.Tensor,
                         log_pi: torch.Tensor, *, precision: str = "fp32"):
    """Full-covariance E-step: returns (logZ, Nk, mu_acc, sig_outer[K, D, D]).

    prec_chol[k] is lower-triangular with prec_chol[k] @ prec_chol[k].T = Sigma_k^-1;
    sig_outer[k] = sum_n r_nk x_n x_n^T (flash_gmm_full_h100.py:245-260).
    ``precision="bf16"`` follows the reference kernels' bf16 operand contract
    instead of fp32 arithmetic.  Up to D = 64 the call runs with
    store_log_joint="auto" (see full_estep_into) while that workspace takes at most
    AUTO_STORE_MEMORY_FRACTION of the device's memory.
    """
    _check_common(X, mu, log_pi)
    N, D = X.shape
    K = mu.shape[0]
    _require(tuple(prec_chol.shape) == (K, D, D),
             f"prec_chol must be (K, D, D)=({K}, {D}, {D}), got {tuple(prec_chol.shape)}")
    dev = X.device
    logZ = torch.empty(N, device=dev, dtype=torch.float32)
    Nk = torch.empty(K, device=dev, dtype=torch.float32)
    mu_acc = torch.empty(K, D, device=dev, dtype=torch.float32)
    sig_outer = torch.empty(K, D, D, device=dev, dtype=torch.float32)
    full_estep_into(X, mu, prec_chol, log_pi, logZ, Nk, mu_acc, sig_outer, precision=precision,
                    store_log_joint=_auto_store(N, K, D, dev, precision, "full"))
    return logZ, Nk, mu_acc, sig_outer

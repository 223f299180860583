"""C ABI checks that need no GPU: the library loads, exports every function
declared in include/flashgmm.h, and rejects bad arguments before any HIP call."""

import ctypes
import os
import re

import pytest
import torch

from flash_gmm import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "flashgmm.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fgmm_\w+)\s*\(", text)))


def test_library_built_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"
    L = _lib.lib()
    assert L.fgmm_version() >= 10000


def test_exports_every_declared_symbol():
    names = declared_functions()
    assert "fgmm_iso_estep_f32" in names
    raw = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in names if not hasattr(raw, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_strerror_names_every_status():
    L = _lib.lib()
    for st in (0, -1, -2, -3, -4):
        assert L.fgmm_strerror(st).decode() != "unknown status"
    assert L.fgmm_strerror(-99).decode() == "unknown status"


def test_iso_workspace_bytes_grows_with_size():
    L = _lib.lib()
    R = _lib.FLAG_RECOMPUTE
    a = L.fgmm_iso_workspace_bytes(1000, 64, 32)
    b = L.fgmm_iso_workspace_bytes(1_000_000, 1024, 128)
    assert 0 < a < b
    assert L.fgmm_iso_workspace_bytes_ex(1_000_000, 1024, 128, R) == b
    assert L.fgmm_iso_workspace_bytes_ex(1_000_000, 1024, 128, 0) == b
    assert L.fgmm_iso_workspace_bytes(-1, 4, 4) == 0
    assert L.fgmm_iso_workspace_bytes(10, 4, 0) == 0
    assert L.fgmm_iso_workspace_bytes_ex(10, 4, 0, 0) == 0


def test_default_workspace_is_lean():
    """The default plan is O(N + K*D): per-row state (16 B/row), the slab partials and
    one need bit per (row, 32-component block), never the N x K log-joint
    (flash_gmm.py:14-15: the reference's working memory is O(K*D))."""
    L = _lib.lib()
    N, K, D = 1_000_000, 1024, 128
    lean = L.fgmm_iso_workspace_bytes(N, K, D)
    masks = (-(-N // 128) * 4) * (K // 32) * 4
    assert lean < 16 * N + masks + (40 << 20) < 64 << 20
    # diag: two need words per (tile, block) and partials of both moments
    assert L.fgmm_diag_workspace_bytes(N, K, 96) < 80 << 20
    # full: one need bit per (row, component), per-wave bounds of pass 1's persistent grid
    # (independent of N) and D x D partials per (slab, component)
    assert L.fgmm_full_workspace_bytes(250_000, 256, 64) < 96 << 20
    # all far below the N x K float32 log-joint (4 N K bytes)
    assert L.fgmm_diag_workspace_bytes(N, K, 96) < 0.02 * 4 * N * K


def test_iso_workspace_holds_stored_log_joint():
    """FGMM_FLAG_STORE_LOGJOINT adds, up to D = 128, the fp32 log-joint tiles (N/32 x
    K/32 x 4 KiB) and per 32-row tile the rows' bf16 X parts (2 x 32 x (D + 16) x 2
    bytes) and logZ pairs (256 bytes), tiles rounded to 8 per pass-1 workgroup as in
    the default plan (whose need masks both plans hold).  STORE_LOGJOINT_AUTO adds the
    same plus the probe's counts; RECOMPUTE overrides both."""
    L = _lib.lib()
    R, S, A = _lib.FLAG_RECOMPUTE, _lib.FLAG_STORE_LOGJOINT, _lib.FLAG_STORE_LOGJOINT_AUTO
    N, K, D = 1_000_000, 1024, 128
    stored = L.fgmm_iso_workspace_bytes_ex(N, K, D, S)
    auto = L.fgmm_iso_workspace_bytes_ex(N, K, D, A)
    lean = L.fgmm_iso_workspace_bytes(N, K, D)
    assert L.fgmm_iso_workspace_bytes_ex(N, K, D, S | R) == lean
    assert L.fgmm_iso_workspace_bytes_ex(N, K, D, A | R) == lean
    assert L.fgmm_iso_workspace_bytes_ex(N, K, D, A | S) == stored
    ptiles = -(-N // 256) * 8
    extra = ptiles * ((K // 32) * 4096 + 2 * 32 * (D + 16) * 2 + 256)
    assert extra <= auto - lean <= extra + 4 * 256 + 256
    # The explicit plan's pass-2 work split differs (partials), within a few MB.
    assert abs(stored - auto) < 0.01 * extra
    # AUTO applies up to D = 128 only.
    assert L.fgmm_iso_workspace_bytes_ex(N, K, 192, A) == L.fgmm_iso_workspace_bytes(N, K, 192)
    # Not stored: D <= 32, K <= 96, or more than 16 GiB of tiles (AUTO: the last).
    for n, k, d in [(N, K, 32), (N, 96, 128), (N, 96, 192), (20_000_000, 1024, 128)]:
        assert L.fgmm_iso_workspace_bytes(n, k, d) == L.fgmm_iso_workspace_bytes_ex(n, k, d, S)
    assert L.fgmm_iso_workspace_bytes(20_000_000, K, D) == L.fgmm_iso_workspace_bytes_ex(20_000_000, K, D, A)
    pairs = -(-N // 128) * 4 * (K // 32)
    # Diagonal: stored for K > 96 at every D.
    d_stored = L.fgmm_diag_workspace_bytes_ex(N, K, 96, S)
    d_lean = L.fgmm_diag_workspace_bytes(N, K, 96)
    assert d_lean == L.fgmm_diag_workspace_bytes_ex(N, K, 96, R) == L.fgmm_diag_workspace_bytes_ex(N, K, 96, 0)
    assert d_stored - d_lean >= pairs * (4096 + 256)
    assert L.fgmm_diag_workspace_bytes(N, 96, 96) == L.fgmm_diag_workspace_bytes_ex(N, 96, 96, S)
    # Diagonal STORE_LOGJOINT_AUTO (D <= 96): the log-joint tiles and per 32-row tile
    # the rows' features [x^2 | x] in three bf16 parts (3 x 32 x (2 D + 16) x 2 bytes)
    # and logZ pairs, tiles rounded to 4 per pass-1 workgroup, and the probe's counts.
    d_auto = L.fgmm_diag_workspace_bytes_ex(N, K, 96, A)
    tiles = -(-N // 128) * 4
    dextra = tiles * ((K // 32) * 4096 + 3 * 32 * (2 * 96 + 16) * 2 + 256)
    assert dextra <= d_auto - d_lean <= dextra + 4 * 256
    assert L.fgmm_diag_workspace_bytes_ex(N, K, 96, A | R) == d_lean
    assert L.fgmm_diag_workspace_bytes_ex(N, K, 96, A | S) == d_stored
    assert L.fgmm_diag_workspace_bytes_ex(N, K, 128, A) == L.fgmm_diag_workspace_bytes(N, K, 128)
    # Full: stored whenever it fits, 32 floats per (32-row tile, component).
    q, qx = L.fgmm_full_workspace_bytes, L.fgmm_full_workspace_bytes_ex
    # Full STORE_LOGJOINT_AUTO (D <= 64, K <= 512): the default plan plus the kept
    # log-joint (tiles rounded to 4 per pass-1 workgroup), the probe's counts and its
    # log-joints of 64 sampled tiles.
    f_lj = -(-250_000 // 128) * 4 * 256 * 32 * 4 + 64 * 256 * 32 * 4
    assert f_lj <= qx(250_000, 256, 64, A) - q(250_000, 256, 64) <= f_lj + 2 * 256
    assert qx(250_000, 256, 96, A) == q(250_000, 256, 96)
    assert qx(250_000, 600, 64, A) == q(250_000, 600, 64)
    assert q(5000, 64, 64) == qx(5000, 64, 64, 0) == qx(5000, 64, 64, R) > 0
    n = 250_000
    lj_bytes = -(-n // 128) * 4 * 256 * 128
    # the stored plan adds the log-joint; the default plan's need words, pass-1
    # bounds and partials are a fraction of it
    assert qx(n, 256, 64, S) >= lj_bytes > 2 * q(n, 256, 64)


# Fake but aligned, non-null addresses: every call below must be rejected by
# argument validation, which happens before any pointer is used.  They only
# run where no GPU is present, so a validation bug cannot turn them into a
# kernel launch on a real device.
no_gpu = pytest.mark.skipif(torch.cuda.is_available(), reason="host-only validation checks")
FAKE = 1 << 20


def _call_iso(**kw):
    a = dict(X=FAKE, ldx=32, N=10, D=32, mu=FAKE, ldmu=32, K=4, lss=FAKE, lpi=FAKE,
             logZ=FAKE, Nk=FAKE, mu_acc=FAKE, sig=FAKE, ws=FAKE, ws_bytes=1 << 40, flags=0)
    a.update(kw)
    L = _lib.lib()
    return L.fgmm_iso_estep_f32(a["X"], a["ldx"], a["N"], a["D"], a["mu"], a["ldmu"], a["K"],
                                a["lss"], a["lpi"], a["logZ"], a["Nk"], a["mu_acc"], a["sig"],
                                a["ws"], a["ws_bytes"], a["flags"], None)


@no_gpu
@pytest.mark.parametrize("kw,status", [
    (dict(N=-1), _lib.FGMM_ERR_INVALID_ARG),
    (dict(D=0), _lib.FGMM_ERR_INVALID_ARG),
    (dict(K=-2), _lib.FGMM_ERR_INVALID_ARG),
    (dict(X=None), _lib.FGMM_ERR_INVALID_ARG),
    (dict(ldx=30), _lib.FGMM_ERR_INVALID_ARG),          # not a multiple of 4
    (dict(ldx=28), _lib.FGMM_ERR_INVALID_ARG),          # shorter than the row
    (dict(X=FAKE + 4), _lib.FGMM_ERR_INVALID_ARG),      # not 16-byte aligned
    (dict(logZ=None), _lib.FGMM_ERR_INVALID_ARG),
    (dict(mu=None), _lib.FGMM_ERR_INVALID_ARG),
    (dict(ldmu=16), _lib.FGMM_ERR_INVALID_ARG),
    (dict(Nk=None), _lib.FGMM_ERR_INVALID_ARG),
    (dict(N=(1 << 37) + 1), _lib.FGMM_ERR_UNSUPPORTED),  # pass-1 grid limit
    (dict(ws_bytes=16), _lib.FGMM_ERR_WORKSPACE),
    (dict(ws=None), _lib.FGMM_ERR_WORKSPACE),
])
def test_iso_rejects_bad_arguments(kw, status):
    assert _call_iso(**kw) == status


def _call_diag(D, flags=0):
    L = _lib.lib()
    ld = (D + 3) // 4 * 4
    return L.fgmm_diag_estep_f32(FAKE, ld, 10, D, FAKE, D, 4, FAKE, D, FAKE, FAKE, FAKE, FAKE, FAKE,
                                 FAKE, 1 << 40, flags, None)


def _call_full(D, flags=0):
    L = _lib.lib()
    ld = (D + 3) // 4 * 4
    return L.fgmm_full_estep_f32(FAKE, ld, 10, D, FAKE, D, 4, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                 FAKE, 1 << 40, flags, None)


@no_gpu
def test_dimension_limits():
    """Largest supported D per covariance model; one past it is UNSUPPORTED.  The
    isotropic and diagonal E-steps (and their bf16 contracts) take any D; the
    full-covariance E-step stops at 4096, its bf16 contract at 128."""
    assert _call_full(4097) == _lib.FGMM_ERR_UNSUPPORTED
    assert _call_full(129, flags=_lib.FLAG_BF16) == _lib.FGMM_ERR_UNSUPPORTED
    # workspace queries accept the supported range
    L = _lib.lib()
    assert L.fgmm_iso_workspace_bytes(100, 10, 4000) > L.fgmm_iso_workspace_bytes(100, 10, 300) > 0
    assert L.fgmm_diag_workspace_bytes(100, 10, 1000) > L.fgmm_diag_workspace_bytes(100, 10, 256) > \
        L.fgmm_diag_workspace_bytes(100, 10, 128) > 0
    assert L.fgmm_full_workspace_bytes(100, 10, 512) > L.fgmm_full_workspace_bytes(100, 10, 300) > \
        L.fgmm_full_workspace_bytes(100, 10, 256) > L.fgmm_full_workspace_bytes(100, 10, 128) > \
        L.fgmm_full_workspace_bytes(100, 10, 64) > 0
    assert L.fgmm_full_workspace_bytes(100, 10, 4096) > 0 == L.fgmm_full_workspace_bytes(100, 10, 4097)
    # the bf16 contracts above D = 256 store the N x K log-joint
    B = _lib.FLAG_BF16
    for q in (L.fgmm_iso_workspace_bytes_ex, L.fgmm_diag_workspace_bytes_ex):
        assert q(4096, 64, 960, B) > q(4096, 64, 300, B) >= 4096 * 64 * 4


def test_python_layer_rejects_cpu_tensors():
    from flash_gmm import FlashGMMError, flash_gmm_estep
    X = torch.zeros(4, 3)
    with pytest.raises(AssertionError):
        flash_gmm_estep(X, torch.zeros(2, 3), torch.zeros(2), torch.zeros(2))
    with pytest.raises(FlashGMMError):
        flash_gmm_estep(X, torch.zeros(2, 3), torch.zeros(2), torch.zeros(2))


def test_reference_module_names_resolve():
    """The reference's module names import and expose its entry points."""
    import importlib
    import flash_gmm
    for mod, fn in (("flash_gmm", "flash_gmm_estep"), ("flash_gmm_h100", "flash_gmm_estep"),
                    ("flash_gmm_diag_h100", "flash_gmm_estep_diag"),
                    ("flash_gmm_full_h100", "flash_gmm_estep_full")):
        m = importlib.import_module(mod)
        assert getattr(m, fn) is getattr(flash_gmm, fn)


def test_gather_slabs_keep_row_state_offsets_in_32_bits():
    """The gathering pass 2 reads a slab's row state through a buffer resource with
    32-bit byte offsets, so no slab may hold more than 2^31 bytes of it.  At large N
    with many components (few slabs wanted) the plan must take more slabs: seen here
    through the workspace, whose slab partials grow with the slab count while the
    other sections it adds between the two sizes are the row state and need words."""
    L = _lib.lib()

    def r8(n):
        return -(-n // 8) * 8

    def r4(n):
        return -(-n // 4) * 4

    # Isotropic: 16 bytes of row state per row; cap = 134,217,696 rows per slab.
    K, D, DP = 16384, 16, 32
    KB, KP = K // 32, K
    N1, N2 = 1 << 26, 1 << 30
    grow = L.fgmm_iso_workspace_bytes(N2, K, D) - L.fgmm_iso_workspace_bytes(N1, K, D)
    fixed = 16 * (N2 - N1) + 4 * KB * (r8(N2 // 32) - r8(N1 // 32))
    per_slab = KP * (DP + 2) * 4
    cap = ((1 << 31) - 256) // 16 // 32 * 32
    slabs_added = -(-N2 // cap) - 4          # 4 slabs at N1 (one group of four)
    assert slabs_added == 5
    assert abs(grow - fixed - slabs_added * per_slab) <= 16 * 256
    # Diagonal: 8 bytes of row state per row; cap = 268,435,424 rows per slab.
    K, D, DP = 16384, 32, 32
    KB, KP = K // 32, K
    N1, N2 = 1 << 26, 1 << 31
    grow = L.fgmm_diag_workspace_bytes(N2, K, D) - L.fgmm_diag_workspace_bytes(N1, K, D)
    fixed = 8 * (N2 - N1) + 8 * KB * (r4(N2 // 32) - r4(N1 // 32))
    per_slab = KP * (2 * DP + 1) * 4
    cap = ((1 << 31) - 256) // 8 // 32 * 32
    slabs_added = -(-N2 // cap) - 4
    assert slabs_added == 5
    assert abs(grow - fixed - slabs_added * per_slab) <= 16 * 256

"""Flash-GMM E-step for AMD Instinct MI355X (gfx950).

Drop-in replacement for the reference's entry points, backed by hand-written
HIP kernels in ``libflashgmm.so`` (C ABI: include/flashgmm.h):

    from flash_gmm import flash_gmm_estep
    logZ, Nk, mu_acc, sig_acc = flash_gmm_estep(X, mu, log_sigma_sq, log_pi)
"""

from ._lib import FlashGMMError  # noqa: F401
from .estep import flash_gmm_estep, iso_estep_into  # noqa: F401

__all__ = ["flash_gmm_estep", "iso_estep_into", "FlashGMMError"]

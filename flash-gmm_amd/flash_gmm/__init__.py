"""Flash-GMM E-step for AMD Instinct MI355X (gfx950).

Drop-in replacement for the reference's entry points, backed by hand-written
HIP kernels in ``libflashgmm.so`` (C ABI: include/flashgmm.h):

    from flash_gmm import flash_gmm_estep
    logZ, Nk, mu_acc, sig_acc = flash_gmm_estep(X, mu, log_sigma_sq, log_pi)
"""

from . import datasets  # noqa: F401
from ._lib import FlashGMMError  # noqa: F401
from .em import (SynthIsoSource, em_diag, em_full, em_iso, mstep_diag, mstep_full,  # noqa: F401
                 mstep_iso, stream_em_iso)
from .estep import (diag_estep_into, flash_gmm_estep, flash_gmm_estep_diag,  # noqa: F401
                    flash_gmm_estep_full, full_estep_into, iso_estep_into)

__all__ = ["flash_gmm_estep", "flash_gmm_estep_diag", "flash_gmm_estep_full",
           "iso_estep_into", "diag_estep_into", "full_estep_into",
           "mstep_iso", "mstep_diag", "mstep_full", "em_iso", "em_diag", "em_full",
           "stream_em_iso", "SynthIsoSource", "FlashGMMError", "datasets"]

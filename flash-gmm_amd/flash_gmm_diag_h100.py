"""Drop-in module name: ``from flash_gmm_diag_h100 import flash_gmm_estep_diag`` as in the
reference (flash_gmm_diag_h100.py:305-384).  Re-exports the gfx950 implementation from the ``flash_gmm``
package."""

from flash_gmm import flash_gmm_estep_diag  # noqa: F401

__all__ = ["flash_gmm_estep_diag"]

"""Drop-in module name: ``from flash_gmm_full_h100 import flash_gmm_estep_full`` as in the
reference (flash_gmm_full_h100.py:235-336).  Re-exports the gfx950 implementation from the ``flash_gmm``
package."""

from flash_gmm import flash_gmm_estep_full  # noqa: F401

__all__ = ["flash_gmm_estep_full"]

"""Drop-in module name: ``from flash_gmm_h100 import flash_gmm_estep`` as in the
reference (flash_gmm_h100.py:254-328, the bf16-operand H100 variant).  Re-exports the
gfx950 implementation from the ``flash_gmm`` package, which computes in fp32."""

from flash_gmm import flash_gmm_estep  # noqa: F401

__all__ = ["flash_gmm_estep"]

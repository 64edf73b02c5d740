"""cufk_amd: MI355X-native NeRF chain reconstruction, a drop-in for ``cufk``'s public surface
(reference ``src/cufk/__init__.py:1-11``)."""

from .reconstruct import BLOCK_SCAN_MAX_POINT_COUNT, reconstruct
from .torsion import compile_torsion

__version__ = "0.1.0"

__all__ = [
    "BLOCK_SCAN_MAX_POINT_COUNT",
    "__version__",
    "compile_torsion",
    "reconstruct",
]

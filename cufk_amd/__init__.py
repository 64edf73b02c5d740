"""cufk_amd: MI355X-native NeRF chain reconstruction, a drop-in for ``cufk``'s public surface
(reference ``src/cufk/__init__.py:1-11``).  ``__all__`` is the reference's; ``reconstruct_long``
(chains past the 2051-point cap), ``reconstruct_loss`` and ``reconstruct_rmsd`` (the
reconstruction fused with a coordinate loss, or with the RMSD after optimal superposition) are
extensions imported by name."""

from .reconstruct import BLOCK_SCAN_MAX_POINT_COUNT, reconstruct, reconstruct_long, reconstruct_loss, reconstruct_rmsd
from .torsion import compile_torsion

__version__ = "0.1.0"

__all__ = [
    "BLOCK_SCAN_MAX_POINT_COUNT",
    "__version__",
    "compile_torsion",
    "reconstruct",
]

"""Torsion-only path: ``compile_torsion(bond_lengths, bond_angles)(raw_pairs)``.

Mirrors the reference ``src/cufk/torsion.py:63-135``.  The reference formats the constants
with ``.17g`` into ``-D`` macros and JIT-compiles a CUDA module per constant set; here the
same values (bond lengths rounded to float, bond-angle sin/cos in float64) are passed to a
prebuilt HIP kernel as arguments, so "compiling" is constructing a ``_C.TorsionModule``.
The returned callable is cached per ``(bond_lengths, bond_angles)`` key, like
``_TORSION_CALLS`` (torsion.py:50,117-135).
"""

from __future__ import annotations

import math
from typing import Final, Protocol

import torch

from ._native import _C


class TorsionReconstructor(Protocol):
    def __call__(self, raw_pairs: torch.Tensor) -> torch.Tensor:
        r"""Reconstruct ``(B, N, 3)`` coordinates from interleaved raw ``(sin, cos)`` pairs
        shaped ``(B, 2 * (N - 3))``; each pair is normalised inside the kernel.  Gradients
        flow to ``raw_pairs``."""
        ...


class _TorsionCall:
    """The callable ``compile_torsion`` returns: calling it is the reference's module ``apply``
    (torsion.py:134-135).  ``loss`` and ``rmsd`` are extensions with no reference counterpart:
    the torsion path fused with a per-chain loss against a target, whose backward forms
    ``grad_xyz`` inside the kernel (the reference's torsion backward, torsion.cu:297-381, reads
    a materialised one)."""

    __slots__ = ("_module", "_apply")

    def __init__(self, module):
        self._module = module
        self._apply = module.apply

    def __call__(self, raw_pairs: torch.Tensor) -> torch.Tensor:
        return self._apply(raw_pairs)

    def loss(self, raw_pairs: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        r"""Per-chain :math:`\sum_i \lVert x_i - t_i \rVert^2` of the reconstruction of
        ``raw_pairs`` against ``target`` ``(B, N, 3)`` (same dtype and device, no gradient),
        ``(B,)``; gradients flow to ``raw_pairs``."""
        return self._module.loss(raw_pairs, target.contiguous(), 0)

    def rmsd(self, raw_pairs: torch.Tensor, target: torch.Tensor, squared: bool = False) -> torch.Tensor:
        r"""Per-chain RMSD of the reconstruction from ``target`` after optimal superposition (the
        mean squared deviation with ``squared=True``), ``(B,)``; as
        :func:`cufk_amd.reconstruct_rmsd` for the torsion path."""
        return self._module.loss(raw_pairs, target.contiguous(), 1 if squared else 2)


_TORSION_CALLS: dict[tuple[tuple[float, float, float], tuple[float, float, float]], TorsionReconstructor] = {}
_TORSION_MODULES: dict[tuple[tuple[float, float, float], tuple[float, float, float]], object] = {}


def _format_float(value: float) -> str:
    """torsion.py:63-64."""
    return format(float(value), ".17g")


def _as_triple(values: tuple[float, float, float], label: str) -> tuple[float, float, float]:
    """torsion.py:67-69."""
    assert len(values) == 3, f"{label} must have 3 elements"
    return (values[0], values[1], values[2])


def _constants(
    lengths: tuple[float, float, float], angles: tuple[float, float, float]
) -> tuple[list[float], list[float], list[float]]:
    """The values the reference compiles in (torsion.py:81-86, torsion.cu:43-53): each
    value passes through its ``.17g`` text; lengths are later rounded to float."""
    ls = [float(_format_float(v)) for v in lengths]
    ss = [float(_format_float(math.sin(a))) for a in angles]
    cs = [float(_format_float(math.cos(a))) for a in angles]
    return ls, ss, cs


def compile_torsion(
    bond_lengths: tuple[float, float, float],
    bond_angles: tuple[float, float, float],
) -> TorsionReconstructor:
    r"""Build (once per constant set) a torsion-only reconstructor for fixed backbone geometry.

    Args:
        bond_lengths: Three repeating bond lengths (rounded to float inside the kernel).
        bond_angles: Three repeating bond angles in radians; their sin/cos are taken in
            float64 here.

    Returns:
        A cached callable ``reconstruct(raw_pairs) -> xyz``.  Equal arguments return the
        same callable object.  It also offers the fused losses ``.loss(raw_pairs, target)``
        and ``.rmsd(raw_pairs, target, squared=False)`` (extensions).
    """
    lengths = _as_triple(bond_lengths, "bond_lengths")
    angles = _as_triple(bond_angles, "bond_angles")
    key = (lengths, angles)
    if key not in _TORSION_CALLS:
        module = _C.TorsionModule(*_constants(lengths, angles))
        _TORSION_MODULES[key] = module
        _TORSION_CALLS[key] = _TorsionCall(module)
    return _TORSION_CALLS[key]

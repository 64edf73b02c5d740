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
        same callable object.
    """
    lengths = _as_triple(bond_lengths, "bond_lengths")
    angles = _as_triple(bond_angles, "bond_angles")
    key = (lengths, angles)
    if key not in _TORSION_CALLS:
        module = _C.TorsionModule(*_constants(lengths, angles))
        _TORSION_MODULES[key] = module
        _TORSION_CALLS[key] = module.apply
    return _TORSION_CALLS[key]

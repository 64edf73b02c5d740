"""Generic reconstruction path: ``reconstruct(lengths, angles, dihedrals, p0, first_direction, initial_normal)``.

Mirrors the reference ``src/cufk/reconstruct.py:1-81``: same batching of 1-D inputs, same
default anchors, same contiguity handling, same call into ``_C.apply`` (a C++
``torch::autograd::Function`` over the HIP C ABI).
"""

from __future__ import annotations

import torch

from ._native import _C

# reconstruct.py:5: N <= 2051 points (2048 local transforms).
BLOCK_SCAN_MAX_POINT_COUNT = 2051


def _batched_inputs(
    lengths: torch.Tensor,
    angles: torch.Tensor,
    dihedrals: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, bool]:
    """reconstruct.py:8-16: add a batch axis when ``lengths`` is 1-D."""
    single = lengths.dim() == 1
    if single:
        lengths, angles, dihedrals = lengths[None], angles[None], dihedrals[None]
    return lengths, angles, dihedrals, single


_DEFAULT_ANCHORS: dict[tuple[torch.device, torch.dtype, tuple[float, float, float]], torch.Tensor] = {}


def _anchor(x: torch.Tensor | None, vals: tuple[float, float, float], ref: torch.Tensor) -> torch.Tensor:
    """reconstruct.py:19-26: default anchor on ``ref``'s device and dtype.

    The reference builds it with a host-to-device copy on every call.  Here it is built once per
    device, dtype and value and reused: the kernels only read it and it never requires grad, so
    the values and gradients are the same, and a call with default anchors saves three small
    copies (about 45 us of host time at C1's size).

    The cached tensor is always made outside inference mode: a tensor made inside it is an
    inference tensor, which ``save_for_backward`` refuses, so a first call under
    ``torch.inference_mode()`` would otherwise break every later call that needs gradients."""
    if x is None:
        key = (ref.device, ref.dtype, vals)
        x = _DEFAULT_ANCHORS.get(key)
        if x is None:
            with torch.inference_mode(False):
                made = torch.tensor(vals, device=ref.device, dtype=ref.dtype)
            x = _DEFAULT_ANCHORS.setdefault(key, made)
    return x


def reconstruct(
    lengths: torch.Tensor,
    angles: torch.Tensor,
    dihedrals: torch.Tensor,
    p0: torch.Tensor | None = None,
    first_direction: torch.Tensor | None = None,
    initial_normal: torch.Tensor | None = None,
    *,
    anchor_grads: bool = False,
) -> torch.Tensor:
    r"""Reconstruct Cartesian coordinates from full internal coordinates.

    Args:
        lengths: Bond lengths, GPU tensor ``(N - 1,)`` for one chain or ``(B, N - 1)``.
        angles: Bond angles in radians, ``(N - 2,)`` or ``(B, N - 2)``.
        dihedrals: Dihedral angles in radians, ``(N - 3,)`` or ``(B, N - 3)``.
        p0: Optional first point ``(3,)``; defaults to ``(0, 0, 0)``.
        first_direction: Optional first-bond direction ``(3,)``; defaults to ``(1, 0, 0)``.
        initial_normal: Optional initial plane normal ``(3,)``; defaults to ``(0, 0, 1)``.

    Returns:
        ``(N, 3)`` for one chain or ``(B, N, 3)``, dtype of ``lengths``.

    All inputs are GPU tensors of one dtype (float16, bfloat16, float32 or float64),
    4 <= N <= 2051.  Gradients flow to lengths, angles and dihedrals; anchors must not
    require grad, as in the reference.  With ``anchor_grads=True`` (an extension, keyword
    only) the anchors may require grad and receive gradients too (assuming
    ``|first_direction| >= 1e-6``; an ``initial_normal`` parallel to ``first_direction`` gets
    a zero gradient, the normal then coming from a fixed helper axis).
    """
    lengths, angles, dihedrals, single = _batched_inputs(lengths, angles, dihedrals)
    p0 = _anchor(p0, (0.0, 0.0, 0.0), lengths)
    first_direction = _anchor(first_direction, (1.0, 0.0, 0.0), lengths)
    initial_normal = _anchor(initial_normal, (0.0, 0.0, 1.0), lengths)

    apply = _C.apply_anchored if anchor_grads else _C.apply
    xyz = apply(
        lengths.contiguous(),
        angles.contiguous(),
        dihedrals.contiguous(),
        p0,
        first_direction,
        initial_normal,
    )
    return xyz[0] if single else xyz


def reconstruct_long(
    lengths: torch.Tensor,
    angles: torch.Tensor,
    dihedrals: torch.Tensor,
    p0: torch.Tensor | None = None,
    first_direction: torch.Tensor | None = None,
    initial_normal: torch.Tensor | None = None,
    segment_steps: int | None = None,
    *,
    anchor_grads: bool = False,
) -> torch.Tensor:
    r"""``reconstruct`` for chains of any length (N >= 4, no 2051-point cap).

    Same arguments, defaults, validation and gradients as :func:`reconstruct` (including
    ``anchor_grads``).  The chain is cut into segments of ``segment_steps`` local transforms
    (1..2048; by default 2048, halved down to 256 while fewer than 1024 segments would run),
    each reconstructed by one workgroup and joined in float64.  The backward takes, per
    segment, the position-based adjoint over the segment's own local positions where the
    forward's tests passed for it and for the segment before it, and the exact adjoint
    elsewhere.  Without ``segment_steps``, chains of at most 2051 points take
    :func:`reconstruct` itself.

    The reference has no counterpart (its README leaves long chains to a separate
    repository); this extends its interface rather than mirroring it.
    """
    if segment_steps is None and lengths.shape[-1] + 1 <= BLOCK_SCAN_MAX_POINT_COUNT:
        return reconstruct(lengths, angles, dihedrals, p0, first_direction, initial_normal, anchor_grads=anchor_grads)
    lengths, angles, dihedrals, single = _batched_inputs(lengths, angles, dihedrals)
    p0 = _anchor(p0, (0.0, 0.0, 0.0), lengths)
    first_direction = _anchor(first_direction, (1.0, 0.0, 0.0), lengths)
    initial_normal = _anchor(initial_normal, (0.0, 0.0, 1.0), lengths)
    xyz = _C.apply_long(
        lengths.contiguous(),
        angles.contiguous(),
        dihedrals.contiguous(),
        p0,
        first_direction,
        initial_normal,
        0 if segment_steps is None else int(segment_steps),
        anchor_grads,
    )
    return xyz[0] if single else xyz


def reconstruct_loss(
    lengths: torch.Tensor,
    angles: torch.Tensor,
    dihedrals: torch.Tensor,
    target: torch.Tensor,
    p0: torch.Tensor | None = None,
    first_direction: torch.Tensor | None = None,
    initial_normal: torch.Tensor | None = None,
    *,
    anchor_grads: bool = False,
) -> torch.Tensor:
    r"""Per-chain coordinate loss :math:`\sum_i \lVert x_i - t_i \rVert^2` of the reconstruction,
    fused with it.

    Equal to ``((reconstruct(lengths, angles, dihedrals, ...) - target) ** 2).sum((-2, -1))``,
    but ``grad_xyz`` never exists in memory: the forward reduces the loss from the positions in
    registers (it also writes the positions, kept for the backward, not returned), and the
    backward forms each point's gradient from its saved position and target inside the kernel.

    Args:
        lengths, angles, dihedrals, p0, first_direction, initial_normal: as for
            :func:`reconstruct` (4 <= N <= 2051).
        target: ``(N, 3)`` or ``(B, N, 3)``, dtype and device of ``lengths``; no gradient.
        anchor_grads: as for :func:`reconstruct`: the anchors may require grad and receive
            gradients.

    Returns:
        ``(B,)`` losses, or a 0-d tensor for one chain.  Gradients flow to lengths, angles and
        dihedrals.  The reference has no counterpart (it leaves the loss to PyTorch).
    """
    lengths, angles, dihedrals, single = _batched_inputs(lengths, angles, dihedrals)
    if single:
        target = target[None]
    p0 = _anchor(p0, (0.0, 0.0, 0.0), lengths)
    first_direction = _anchor(first_direction, (1.0, 0.0, 0.0), lengths)
    initial_normal = _anchor(initial_normal, (0.0, 0.0, 1.0), lengths)
    loss = _C.apply_loss(
        lengths.contiguous(),
        angles.contiguous(),
        dihedrals.contiguous(),
        target.contiguous(),
        p0,
        first_direction,
        initial_normal,
        anchor_grads,
    )
    return loss[0] if single else loss


def reconstruct_rmsd(
    lengths: torch.Tensor,
    angles: torch.Tensor,
    dihedrals: torch.Tensor,
    target: torch.Tensor,
    p0: torch.Tensor | None = None,
    first_direction: torch.Tensor | None = None,
    initial_normal: torch.Tensor | None = None,
    *,
    squared: bool = False,
) -> torch.Tensor:
    r"""Per-chain RMSD of the reconstruction from ``target`` after optimal superposition, fused
    with the reconstruction.

    For each chain, :math:`\min_R \sqrt{\tfrac1N \sum_i \lVert R (x_i - \bar x) - (t_i - \bar t)
    \rVert^2}` over proper rotations (the Kabsch / Horn superposition, solved per chain in double
    inside the forward kernel), or the mean squared deviation itself with ``squared=True``.  The
    backward forms ``grad_xyz`` inside the kernel from the saved positions, the target and the
    chain's optimal rotation (the rotation's own dependence drops out at the optimum), so it
    never exists in memory.  Where the RMSD is 0 its gradient is taken as 0.

    Args:
        lengths, angles, dihedrals, p0, first_direction, initial_normal: as for
            :func:`reconstruct` (4 <= N <= 2051).
        target: ``(N, 3)`` or ``(B, N, 3)``, dtype and device of ``lengths``; no gradient.
        squared: return the mean squared deviation instead of its square root.

    Returns:
        ``(B,)`` values, or a 0-d tensor for one chain; the positions as stored (rounded to the
        dtype) are the ones superposed.  The reference has no counterpart.
    """
    lengths, angles, dihedrals, single = _batched_inputs(lengths, angles, dihedrals)
    if single:
        target = target[None]
    p0 = _anchor(p0, (0.0, 0.0, 0.0), lengths)
    first_direction = _anchor(first_direction, (1.0, 0.0, 0.0), lengths)
    initial_normal = _anchor(initial_normal, (0.0, 0.0, 1.0), lengths)
    loss = _C.apply_superposed(
        lengths.contiguous(),
        angles.contiguous(),
        dihedrals.contiguous(),
        target.contiguous(),
        p0,
        first_direction,
        initial_normal,
        1 if squared else 2,
    )
    return loss[0] if single else loss

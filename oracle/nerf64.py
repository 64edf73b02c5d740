"""Float64 CPU oracle for cufk's reconstruction path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker or the timed CPU
baseline.  The product (``cufk_amd``) never imports it and fails loudly when
its HIP library is missing.

Every function restates the reference's arithmetic in float64, vectorised over
the batch axis and serial over chain steps.  Citations are to files under the
reference tree ``src/cufk/``.

Pinning (how each function is checked, see ``tests/test_oracle.py``):

* ``reconstruct_forward``: against classic serial Parsons NeRF
  (``nerf_serial``, a different algorithm), the internal-coordinate round trip
  (``measure_internal``: bond lengths, interior angles and IUPAC atan2
  dihedrals), the default-frame closed forms and rigid-motion covariance of the
  anchors.
* ``reconstruct_backward`` (reference form), ``reconstruct_backward_world``
  and ``reconstruct_backward_frames``: against torch.autograd through an
  independent torch restatement of the NeRF recurrence, central finite
  differences, and each other.
* ``torsion_forward`` / ``torsion_backward``: against ``reconstruct_forward``
  with tiled constants and ``D = atan2(rs, rc)``, and the chain rule through
  the pair normalisation, and finite differences.
* ``anchor_gradients``: central finite differences of ``reconstruct_forward``
  in each anchor component, for generic anchors and the degenerate-normal
  branch, and torch.autograd through the torch restatement with its anchors.
* ``torsion_constants``: closed form (float rounding of lengths, float64
  ``math.sin``/``math.cos`` of the angles printed with ``.17g``).
* ``superpose`` / ``superposed_loss`` / ``superposed_grad_xyz`` (the fused RMSD losses, no
  reference counterpart): zero for rigidly moved copies, invariance under rigid motions of
  either side and symmetry in its arguments, a proper rotation for mirrored targets, a brute
  search over rotations, central finite differences of the loss in x and, composed with the
  forward and backward, in the internal coordinates.

No reference golden vectors exist (the reference ships no tests), so parity of
bit-level fp32/fp16/bf16 rounding with the CUDA build is unpinned; those
dtypes are gated by tolerance against this float64 oracle.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

# block.cu:41 ``kEps`` and frame_utils.cuh:7 ``kFrameEps`` are float literals
# 1e-12f; compared/used after promotion to the working precision.
K_EPS = float(np.float32(1.0e-12))
# torsion.cu:35 kNormEps = 1e-8f; the clamp is kNormEps*kNormEps formed in float.
K_NORM_EPS2 = float(np.float32(np.float32(1.0e-8) * np.float32(1.0e-8)))

DEFAULT_P0 = (0.0, 0.0, 0.0)  # reconstruct.py:69
DEFAULT_FIRST_DIRECTION = (1.0, 0.0, 0.0)  # reconstruct.py:70
DEFAULT_INITIAL_NORMAL = (0.0, 0.0, 1.0)  # reconstruct.py:71


# ---------------------------------------------------------------- helpers


def _dot(a, b):
    return np.sum(a * b, axis=-1)


def _cross(a, b):
    return np.cross(a, b)


def _normalized(v, eps=K_EPS):
    """frame_utils.cuh:17-21: v / sqrt(max(v.v, eps))."""
    n2 = _dot(v, v)
    return v / np.sqrt(np.maximum(n2, eps))[..., None]


def _stable_perpendicular(v):
    """frame_utils.cuh:23-31: normalized(v x helper), helper = e_x or e_y if |v_x| >= 0.9."""
    helper = np.zeros_like(v)
    use_y = np.abs(v[..., 0]) >= 0.9
    helper[..., 0] = np.where(use_y, 0.0, 1.0)
    helper[..., 1] = np.where(use_y, 1.0, 0.0)
    return _normalized(_cross(v, helper))


@dataclass
class FirstFrame:
    p1: np.ndarray
    p2: np.ndarray
    dir0: np.ndarray
    turn0: np.ndarray
    dir1: np.ndarray
    normal: np.ndarray
    frame: np.ndarray  # (B, 3, 3) columns (dir1, side, normal)


def first_frame(L0, L1, A0, p0, first_direction, initial_normal) -> FirstFrame:
    """block.cu:113-148 ``compute_first_frame`` (A.2).

    L0, L1, A0: (B,) arrays; anchors: (3,) arrays shared by the batch.
    """
    B = L0.shape[0]
    origin = np.broadcast_to(np.asarray(p0, np.float64), (B, 3))
    dir0 = _normalized(np.broadcast_to(np.asarray(first_direction, np.float64), (B, 3)).copy())
    p1 = origin + L0[:, None] * dir0
    normal0 = np.broadcast_to(np.asarray(initial_normal, np.float64), (B, 3)).copy()
    normal0 = normal0 - _dot(normal0, dir0)[:, None] * dir0
    degenerate = _dot(normal0, normal0) < K_EPS
    normal0 = np.where(degenerate[:, None], _stable_perpendicular(dir0), _normalized(normal0))
    turn0 = _normalized(_cross(normal0, dir0))
    s, c = np.sin(A0), np.cos(A0)
    dir1 = -c[:, None] * dir0 + s[:, None] * turn0
    p2 = p1 + L1[:, None] * dir1
    normal = _normalized(_cross(dir0, dir1))
    side = _cross(normal, dir1)
    frame = np.stack([dir1, side, normal], axis=-1)
    return FirstFrame(p1, p2, dir0, turn0, dir1, normal, frame)


def local_transform(length, theta, phi):
    """affine.cuh:24-51 (A.3): rows [[-c,-s,0],[sC,-cC,-S],[sS,-cS,C]], v = l*M[:,0]."""
    s, c = np.sin(theta), np.cos(theta)
    S, C = np.sin(phi), np.cos(phi)
    return _local_from_sincos(length, s, c, S, C)


def _local_from_sincos(length, s, c, S, C):
    z = np.zeros_like(s)
    m = np.stack(
        [
            np.stack([-c, -s, z], axis=-1),
            np.stack([s * C, -c * C, -S], axis=-1),
            np.stack([s * S, -c * S, C], axis=-1),
        ],
        axis=-2,
    )
    v = length[..., None] * np.stack([-c, s * C, s * S], axis=-1)
    return m, v


def _compose(am, av, bm, bv):
    """affine.cuh:53-58: (a.m b.m, a.v + a.m b.v); a is the earlier element."""
    return am @ bm, av + np.einsum("bij,bj->bi", am, bv)


def _as_batch(x):
    x = np.asarray(x, np.float64)
    return (x[None], True) if x.ndim == 1 else (x, False)


def _anchors(p0, first_direction, initial_normal):
    p0 = DEFAULT_P0 if p0 is None else p0
    first_direction = DEFAULT_FIRST_DIRECTION if first_direction is None else first_direction
    initial_normal = DEFAULT_INITIAL_NORMAL if initial_normal is None else initial_normal
    return (np.asarray(p0, np.float64), np.asarray(first_direction, np.float64), np.asarray(initial_normal, np.float64))


# ---------------------------------------------------------------- reconstruct


def _prefix_affines(L, A, D):
    """Inclusive prefix P_k = A_0 o ... o A_k for every step (A.4), (B,S,3,3),(B,S,3)."""
    B, S = D.shape
    Pm = np.empty((B, S, 3, 3))
    Pv = np.empty((B, S, 3))
    m = np.broadcast_to(np.eye(3), (B, 3, 3)).copy()
    v = np.zeros((B, 3))
    for k in range(S):
        lm, lv = local_transform(L[:, k + 2], A[:, k + 1], D[:, k])
        m, v = _compose(m, v, lm, lv)
        Pm[:, k] = m
        Pv[:, k] = v
    return Pm, Pv


def reconstruct_forward(lengths, angles, dihedrals, p0=None, first_direction=None, initial_normal=None):
    """block.cu:157-204 ``block_forward_kernel`` + reconstruct.py:68-81 batching.

    x0 = p0, x1, x2 from the first frame, x_{k+3} = p2 + F . P_k.v.
    """
    L, single = _as_batch(lengths)
    A, _ = _as_batch(angles)
    D, _ = _as_batch(dihedrals)
    p0, fd, n0 = _anchors(p0, first_direction, initial_normal)
    B, S = D.shape
    ff = first_frame(L[:, 0], L[:, 1], A[:, 0], p0, fd, n0)
    _, Pv = _prefix_affines(L, A, D)
    xyz = np.empty((B, S + 3, 3))
    xyz[:, 0] = p0
    xyz[:, 1] = ff.p1
    xyz[:, 2] = ff.p2
    xyz[:, 3:] = ff.p2[:, None, :] + np.einsum("bij,bkj->bki", ff.frame, Pv)
    return xyz[0] if single else xyz


def reconstruct_backward(lengths, angles, dihedrals, grad_xyz, p0=None, first_direction=None, initial_normal=None):
    """Reference-form adjoint (A.5): block.cu:230-313, affine.cuh:64-77,114-140, block.cu:206-228.

    Returns (grad_lengths, grad_angles, grad_dihedrals).  Anchors get no gradient.
    """
    L, single = _as_batch(lengths)
    A, _ = _as_batch(angles)
    D, _ = _as_batch(dihedrals)
    g, _ = _as_batch(grad_xyz)
    if single:
        g = g.reshape(1, -1, 3) if g.ndim == 2 else g
    p0, fd, n0 = _anchors(p0, first_direction, initial_normal)
    B, S = D.shape
    ff = first_frame(L[:, 0], L[:, 1], A[:, 0], p0, fd, n0)
    Pm, Pv = _prefix_affines(L, A, D)
    gL = np.zeros_like(L)
    gA = np.zeros_like(A)
    gD = np.zeros_like(D)
    # Suffix elements (Ft g_{j+3} (x) P_j.v, Ft g_{j+3}) summed from the tail (affine.cuh:64-73).
    Sm = np.zeros((B, 3, 3))
    Sv = np.zeros((B, 3))
    eye = np.broadcast_to(np.eye(3), (B, 3, 3))
    for k in range(S - 1, -1, -1):
        G = np.einsum("bji,bj->bi", ff.frame, g[:, k + 3])
        Sm = Sm + G[:, :, None] * Pv[:, k][:, None, :]
        Sv = Sv + G
        prev_m = eye if k == 0 else Pm[:, k - 1]
        curr_m, curr_v = Pm[:, k], Pv[:, k]
        grad_t = np.einsum("bji,bj->bi", prev_m, Sv)
        centered = Sm - Sv[:, :, None] * curr_v[:, None, :]
        grad_r = np.swapaxes(prev_m, 1, 2) @ centered @ curr_m
        ell = L[:, k + 2]
        grad_r[:, :, 0] += ell[:, None] * grad_t
        s, c = np.sin(A[:, k + 1]), np.cos(A[:, k + 1])
        Sd, Cd = np.sin(D[:, k]), np.cos(D[:, k])
        z = np.zeros_like(s)
        direction = np.stack([-c, s * Cd, s * Sd], -1)
        dth0 = np.stack([s, c * Cd, c * Sd], -1)
        dth1 = np.stack([-c, s * Cd, s * Sd], -1)
        dph0 = np.stack([z, -s * Sd, s * Cd], -1)
        dph1 = np.stack([z, c * Sd, -c * Cd], -1)
        dph2 = np.stack([z, -Cd, -Sd], -1)
        gL[:, k + 2] = _dot(grad_t, direction)
        gA[:, k + 1] = _dot(grad_r[:, :, 0], dth0) + _dot(grad_r[:, :, 1], dth1)
        gD[:, k] = _dot(grad_r[:, :, 0], dph0) + _dot(grad_r[:, :, 1], dph1) + _dot(grad_r[:, :, 2], dph2)
    # First-frame parameters (block.cu:206-228) from S_0.
    tail_v = np.einsum("bij,bj->bi", ff.frame, Sv)
    tail_a = ff.frame @ Sm
    grad_p2 = g[:, 2] + tail_v
    gL[:, 0] = _dot(g[:, 1] + grad_p2, ff.dir0)
    gL[:, 1] = _dot(grad_p2, ff.dir1)
    s, c = np.sin(A[:, 0]), np.cos(A[:, 0])
    d_dir = s[:, None] * ff.dir0 + c[:, None] * ff.turn0
    d_side = _cross(ff.normal, d_dir)
    gA[:, 0] = L[:, 1] * _dot(grad_p2, d_dir) + _dot(tail_a[:, :, 0], d_dir) + _dot(tail_a[:, :, 1], d_side)
    if single:
        return gL[0], gA[0], gD[0]
    return gL, gA, gD


def _suffix_force_moment(xyz, g):
    """F_i = sum_{j>=i} g_j, M_i = sum_{j>=i} x_j x g_j (torsion.cu:184-211), (B,N+1,3) each."""
    B, N, _ = xyz.shape
    F = np.zeros((B, N + 1, 3))
    M = np.zeros((B, N + 1, 3))
    F[:, :N] = np.cumsum(g[:, ::-1], axis=1)[:, ::-1]
    M[:, :N] = np.cumsum(_cross(xyz, g)[:, ::-1], axis=1)[:, ::-1]
    return F, M


def _unit(v):
    return v / np.linalg.norm(v, axis=-1, keepdims=True)


def reconstruct_backward_world(lengths, angles, dihedrals, grad_xyz, p0=None, first_direction=None, initial_normal=None):
    """World-frame adjoint (A.6) from the forward positions.

    gL[i] = u(x_{i+1}-x_i).F_{i+1}; gA[i] = u((x_i-x_{i+1}) x (x_{i+2}-x_{i+1})).tau_{i+2}(x_{i+1});
    gD[i] = u(x_{i+2}-x_{i+1}).tau_{i+3}(x_{i+2}), tau_i(q) = M_i - q x F_i.
    Valid for positive bond lengths and angles in (0, pi); the reference's
    torsion backward uses the same form for dL/dphi (torsion.cu:204-217).
    """
    L, single = _as_batch(lengths)
    A, _ = _as_batch(angles)
    D, _ = _as_batch(dihedrals)
    g = np.asarray(grad_xyz, np.float64)
    g = g[None] if single else g
    x = reconstruct_forward(L, A, D, p0, first_direction, initial_normal)
    F, M = _suffix_force_moment(x, g)
    N = x.shape[1]
    i = np.arange(N - 1)
    gL = _dot(_unit(x[:, i + 1] - x[:, i]), F[:, i + 1])
    i = np.arange(N - 2)
    axis = _unit(_cross(x[:, i] - x[:, i + 1], x[:, i + 2] - x[:, i + 1]))
    tau = M[:, i + 2] - _cross(x[:, i + 1], F[:, i + 2])
    gA = _dot(axis, tau)
    i = np.arange(N - 3)
    tau = M[:, i + 3] - _cross(x[:, i + 2], F[:, i + 3])
    gD = _dot(_unit(x[:, i + 2] - x[:, i + 1]), tau)
    if single:
        return gL[0], gA[0], gD[0]
    return gL, gA, gD


def reconstruct_backward_frames(lengths, angles, dihedrals, grad_xyz, p0=None, first_direction=None, initial_normal=None):
    """World-frame adjoint with exact frame axes (the form the HIP backward evaluates).

    With R_k the world rotation after step k (R_{-1} = F), x_{k+3} = x_{k+2} + l_k R_k[:,0]:
    gL[k+2] = R_k[:,0].F_{k+3}; gA[k+1] = -R_k[:,2].tau_{k+3}(x_{k+2});
    gD[k] = R_{k-1}[:,0].tau_{k+3}(x_{k+2}); first frame: gL[0] = d0.F_1, gL[1] = d1.F_2,
    gA[0] = -(d0 x t0).tau_2(x_1).  Equal to the reference form for every finite input
    (no normalisation of point differences, so no sign or degeneracy cases).
    """
    L, single = _as_batch(lengths)
    A, _ = _as_batch(angles)
    D, _ = _as_batch(dihedrals)
    g = np.asarray(grad_xyz, np.float64)
    g = g[None] if single else g
    p0, fd, n0 = _anchors(p0, first_direction, initial_normal)
    B, S = D.shape
    ff = first_frame(L[:, 0], L[:, 1], A[:, 0], p0, fd, n0)
    Pm, _ = _prefix_affines(L, A, D)
    x = reconstruct_forward(L, A, D, p0, fd, n0)
    F, M = _suffix_force_moment(x, g)
    R = np.einsum("bij,bkjl->bkil", ff.frame, Pm)  # world rotation after each step
    Rprev = np.concatenate([ff.frame[:, None], R[:, :-1]], axis=1)
    k = np.arange(S)
    tau = M[:, k + 3] - _cross(x[:, k + 2], F[:, k + 3])
    gL = np.zeros_like(L)
    gA = np.zeros_like(A)
    gD = np.zeros_like(D)
    gL[:, k + 2] = _dot(R[:, :, :, 0], F[:, k + 3])
    gA[:, k + 1] = -_dot(R[:, :, :, 2], tau)
    gD[:, k] = _dot(Rprev[:, :, :, 0], tau)
    gL[:, 0] = _dot(ff.dir0, F[:, 1])
    gL[:, 1] = _dot(ff.dir1, F[:, 2])
    tau2 = M[:, 2] - _cross(x[:, 1], F[:, 2])
    gA[:, 0] = -_dot(_cross(ff.dir0, ff.turn0), tau2)
    if single:
        return gL[0], gA[0], gD[0]
    return gL, gA, gD


# ---------------------------------------------------------------- independent checks


def anchor_gradients(lengths, angles, dihedrals, grad_xyz, p0=None, first_direction=None, initial_normal=None):
    """Gradients of sum(grad_xyz * xyz) with respect to the three anchors, summed over the batch
    (the anchors are shared).  No reference counterpart: the reference rejects anchors that
    require grad (extension_utils.cuh:81).

    Every point is p0 + Q c_i with Q = [d, t, n] the orthonormal frame of first_frame
    (d = first_direction normalised, n its Gram-Schmidt normal, t = n x d) and c_i independent
    of the anchors, because every step of block.cu:113-148 and the scan commutes with
    rotations.  So dL/dp0 = F = sum g, and an infinitesimal rotation w of Q changes L by
    w . tau, tau = sum (x - p0) x g.  Expressing w through d and n (w x d = dd, w x n = dn)
    gives dL = dd . (tau x d) - (tau . d)(dn . t), then the chain rule through the
    normalisation of first_direction and the Gram-Schmidt step (or, for the degenerate normal,
    stable_perpendicular(d) with its fixed helper axis).  Assumes |first_direction| >= 1e-6.

    Returns (grad_p0, grad_first_direction, grad_initial_normal), each (3,).
    """
    L, _ = _as_batch(lengths)
    A, _ = _as_batch(angles)
    D, _ = _as_batch(dihedrals)
    g = np.asarray(grad_xyz, np.float64).reshape(L.shape[0], -1, 3)
    p0, fd, n0 = _anchors(p0, first_direction, initial_normal)
    x = reconstruct_forward(L, A, D, p0, fd, n0).reshape(g.shape)
    F = g.sum(axis=(0, 1))
    tau = np.cross(x - p0, g).sum(axis=(0, 1))
    dnorm = math.sqrt(max(float(fd @ fd), K_EPS))
    d = fd / dnorm
    n_raw = n0 - float(n0 @ d) * d
    if float(n_raw @ n_raw) < K_EPS:  # degenerate: n = stable_perpendicular(d)
        h = np.array([0.0, 1.0, 0.0]) if abs(d[0]) >= 0.9 else np.array([1.0, 0.0, 0.0])
        dh = np.cross(d, h)
        n = dh / math.sqrt(max(float(dh @ dh), K_EPS))
        t = np.cross(n, d)
        v = np.cross(tau, d) - float(tau @ d) * np.cross(h, t) / math.sqrt(float(dh @ dh))
        grad_fd = (v - float(v @ d) * d) / dnorm
        grad_n0 = np.zeros(3)
    else:
        nn = math.sqrt(float(n_raw @ n_raw))
        n = n_raw / nn
        t = np.cross(n, d)
        grad_fd = (np.cross(tau, d) + float(tau @ d) * float(n0 @ d) / nn * t) / dnorm
        grad_n0 = -float(tau @ d) / nn * t
    return F, grad_fd, grad_n0


def nerf_serial(lengths, angles, dihedrals, p0=None, first_direction=None, initial_normal=None):
    """Classic serial NeRF (Parsons et al. 2005) from the first three points.

    d = c + [bc, n x bc, n] (-l cos t, l sin t cos p, l sin t sin p) with
    bc = unit(c - b), n = unit((b - a) x bc).  An independent algorithm used to
    pin ``reconstruct_forward``.
    """
    L, single = _as_batch(lengths)
    A, _ = _as_batch(angles)
    D, _ = _as_batch(dihedrals)
    p0, fd, n0 = _anchors(p0, first_direction, initial_normal)
    B, S = D.shape
    ff = first_frame(L[:, 0], L[:, 1], A[:, 0], p0, fd, n0)
    x = np.empty((B, S + 3, 3))
    x[:, 0] = p0
    x[:, 1] = ff.p1
    x[:, 2] = ff.p2
    for k in range(S):
        a, b, c = x[:, k], x[:, k + 1], x[:, k + 2]
        bc = _unit(c - b)
        n = _unit(_cross(b - a, bc))
        m = np.stack([bc, _cross(n, bc), n], axis=-1)
        l, t, p = L[:, k + 2], A[:, k + 1], D[:, k]
        d2 = np.stack([-l * np.cos(t), l * np.sin(t) * np.cos(p), l * np.sin(t) * np.sin(p)], -1)
        x[:, k + 3] = c + np.einsum("bij,bj->bi", m, d2)
    return x[0] if single else x


def measure_internal(xyz):
    """Bond lengths, interior angles and IUPAC atan2 dihedrals of a (B,N,3) polyline."""
    x = np.asarray(xyz, np.float64)
    b = x[:, 1:] - x[:, :-1]
    L = np.linalg.norm(b, axis=-1)
    u, w = -b[:, :-1], b[:, 1:]
    A = np.arctan2(np.linalg.norm(_cross(u, w), axis=-1), _dot(u, w))
    b1, b2, b3 = b[:, :-2], b[:, 1:-1], b[:, 2:]
    n1, n2 = _cross(b1, b2), _cross(b2, b3)
    D = np.arctan2(np.linalg.norm(b2, axis=-1) * _dot(b1, n2), _dot(n1, n2))
    return L, A, D


# ---------------------------------------------------------------- torsion


@dataclass(frozen=True)
class TorsionConstants:
    lengths: tuple  # float-rounded bond lengths (torsion.cu:43-47)
    sin: tuple  # float64 sin of bond angles (torsion.py:84-85)
    cos: tuple


def torsion_constants(bond_lengths, bond_angles) -> TorsionConstants:
    """torsion.py:63-86 + torsion.cu:43-53: lengths rounded to float, sin/cos in float64."""
    assert len(bond_lengths) == 3 and len(bond_angles) == 3
    lengths = tuple(float(np.float32(float(format(float(v), ".17g")))) for v in bond_lengths)
    sins = tuple(float(format(math.sin(a), ".17g")) for a in bond_angles)
    coss = tuple(float(format(math.cos(a), ".17g")) for a in bond_angles)
    return TorsionConstants(lengths, sins, coss)


def _normalize_pairs(raw):
    """torsion.cu:119-141: (rs, rc) / sqrt(max(rs^2 + rc^2, 1e-16))."""
    rs, rc = raw[..., 0::2], raw[..., 1::2]
    n2 = np.maximum(rs * rs + rc * rc, K_NORM_EPS2)
    r = 1.0 / np.sqrt(n2)
    return rs * r, rc * r, n2


def torsion_base(consts: TorsionConstants):
    """torsion.cu:149-166: x0 = 0, x1 = (l0,0,0), x2 = (l0 - l1 c0, l1 s0, 0), F columns."""
    l0, l1 = consts.lengths[0], consts.lengths[1]
    s, c = consts.sin[0], consts.cos[0]
    p1 = np.array([l0, 0.0, 0.0])
    p2 = np.array([l0 - l1 * c, l1 * s, 0.0])
    frame = np.array([[-c, -s, 0.0], [s, -c, 0.0], [0.0, 0.0, 1.0]])
    return p1, p2, frame


def torsion_forward(raw_pairs, consts: TorsionConstants):
    """torsion.cu:254-295: step k uses l_{(k+2)%3}, angle_{(k+1)%3}, normalised raw pair k."""
    raw = np.asarray(raw_pairs, np.float64)
    B, K = raw.shape
    S = K // 2
    Sn, Cn, _ = _normalize_pairs(raw)
    p1, p2, frame = torsion_base(consts)
    x = np.empty((B, S + 3, 3))
    x[:, 0] = 0.0
    x[:, 1] = p1
    x[:, 2] = p2
    m = np.broadcast_to(np.eye(3), (B, 3, 3)).copy()
    v = np.zeros((B, 3))
    for k in range(S):
        lp, ap = (k + 2) % 3, (k + 1) % 3
        ell = np.full(B, consts.lengths[lp])
        s = np.full(B, consts.sin[ap])
        c = np.full(B, consts.cos[ap])
        lm, lv = _local_from_sincos(ell, s, c, Sn[:, k], Cn[:, k])
        m, v = _compose(m, v, lm, lv)
        x[:, k + 3] = p2 + v @ frame.T
    return x


def torsion_backward(raw_pairs, xyz, grad_xyz, consts: TorsionConstants):
    """torsion.cu:297-381 + 173-182 + 213-217.

    dphi_k = (1/l_{(k+1)%3}) (x_{k+2} - x_{k+1}) . (M_{k+3} - x_{k+2} x F_{k+3});
    raw grad = dphi (rc, -rs) / max(rs^2 + rc^2, 1e-16).  x_1 for k = 0 is the constant base point.
    The reciprocal 1/l is formed in float (torsion.cu:216) even for float64.
    """
    raw = np.asarray(raw_pairs, np.float64)
    x = np.asarray(xyz, np.float64)
    g = np.asarray(grad_xyz, np.float64)
    B, K = raw.shape
    S = K // 2
    F, M = _suffix_force_moment(x, g)
    k = np.arange(S)
    inv_len = np.array([float(np.float32(1.0) / np.float32(consts.lengths[(p + 1) % 3])) for p in range(3)])
    prev = x[:, k + 1].copy()
    prev[:, 0] = torsion_base(consts)[0]
    pivot = x[:, k + 2]
    tau = M[:, k + 3] - _cross(pivot, F[:, k + 3])
    dphi = inv_len[k % 3][None] * _dot(pivot - prev, tau)
    rs, rc = raw[:, 0::2], raw[:, 1::2]
    n2 = np.maximum(rs * rs + rc * rc, K_NORM_EPS2)
    scale = dphi / n2
    out = np.empty_like(raw)
    out[:, 0::2] = rc * scale
    out[:, 1::2] = -rs * scale
    return out


# ---------------------------------------------------------------- superposed losses
#
# No reference counterpart (the reference leaves losses to PyTorch): the fused RMSD losses of
# cufk_amd.  Restated here with the SVD form of the Kabsch algorithm (W. Kabsch, Acta Cryst. A32,
# 1976; A34, 1978), an independent route from the kernels' quaternion eigenproblem.


def superpose(xyz, target):
    """Optimal proper rotation of each chain onto its target: returns R (B, 3, 3) with
    R (x_i - xbar) ~ t_i - tbar, the centroids xbar, tbar (B, 3) and the mean squared deviation
    after superposition (B,)."""
    x = np.asarray(xyz, np.float64)
    t = np.asarray(target, np.float64)
    xb, tb = x.mean(axis=1), t.mean(axis=1)
    xc, tc = x - xb[:, None], t - tb[:, None]
    H = np.einsum("bia,bic->bac", xc, tc)  # sum_i x'_a t'_c
    U, _, Vt = np.linalg.svd(H)
    d = np.sign(np.linalg.det(np.einsum("bji,bkj->bik", Vt, U)))  # det(V U^T)
    d = np.where(d == 0, 1.0, d)
    D = np.zeros_like(H)
    D[:, 0, 0] = D[:, 1, 1] = 1.0
    D[:, 2, 2] = d
    R = np.einsum("bji,bjk,blk->bil", Vt, D, U)  # V D U^T
    resid = np.einsum("bac,bic->bia", R, xc) - tc
    msd = np.mean(np.sum(resid**2, axis=-1), axis=1)
    return R, xb, tb, msd


def superposed_loss(xyz, target, squared=False):
    """Per-chain mean squared deviation after optimal superposition, or its square root."""
    msd = superpose(xyz, target)[3]
    return msd if squared else np.sqrt(msd)


def superposed_grad_xyz(xyz, target, grad_loss=None, squared=False):
    """dL/dx of the superposed loss: (2/N) w ((x_i - xbar) - R^T (t_i - tbar)), divided by
    2 rmsd for the RMSD (0 where it is 0).  The rotation's own dependence on x drops out at
    the optimum (envelope theorem)."""
    x = np.asarray(xyz, np.float64)
    R, xb, tb, msd = superpose(x, target)
    n = x.shape[1]
    w = np.ones(x.shape[0]) if grad_loss is None else np.asarray(grad_loss, np.float64)
    c = 2.0 * w / n
    if not squared:
        rmsd = np.sqrt(msd)
        c = np.where(rmsd > 0, c / (2.0 * np.where(rmsd > 0, rmsd, 1.0)), 0.0)
    tc = np.asarray(target, np.float64) - tb[:, None]
    return c[:, None, None] * ((x - xb[:, None]) - np.einsum("bca,bic->bia", R, tc))


# ---------------------------------------------------------------- synthetic inputs


def synthetic_inputs(B, N, seed, anchors=False):
    """Config draws: lengths ~N(0.145, 0.01) clipped to [0.12, 0.17], angles ~N(2.05, 0.08),
    dihedrals ~U(-pi, pi), upstream grad ~N(0, 1); optional random anchors (p0 ~ N(0, I),
    first_direction / initial_normal = columns 0 and 1 of Q from QR of a 3x3 normal matrix)."""
    rng = np.random.default_rng(seed)
    L = np.clip(rng.normal(0.145, 0.01, (B, N - 1)), 0.12, 0.17)
    A = rng.normal(2.05, 0.08, (B, N - 2))
    D = rng.uniform(-np.pi, np.pi, (B, N - 3))
    g = rng.normal(0.0, 1.0, (B, N, 3))
    out = {"lengths": L, "angles": A, "dihedrals": D, "grad": g}
    if anchors:
        out["p0"] = rng.normal(0.0, 1.0, 3)
        q, _ = np.linalg.qr(rng.normal(0.0, 1.0, (3, 3)))
        out["first_direction"] = q[:, 0].copy()
        out["initial_normal"] = q[:, 1].copy()
    return out

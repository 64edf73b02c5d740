"""Pins for the float64 oracle (CPU only).

Each oracle function is checked against something other than its own formula: an
independent algorithm (serial Parsons NeRF, torch autograd through that NeRF, finite
differences, the chain rule through atan2), an invariant (internal-coordinate round trip,
rigid-motion covariance), or a closed form.  The mutation tests at the end plant plausible
mistakes in copies of the oracle and show that these checks catch them.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import nerf64 as o

BOND_LENGTHS = (0.14685231, 0.15365194, 0.13405086)
BOND_ANGLES = (1.9676635, 2.062335, 2.164016)


def _anchors(d):
    return dict(p0=d["p0"], first_direction=d["first_direction"], initial_normal=d["initial_normal"])


def _wrap(a):
    return np.angle(np.exp(1j * a))


# ------------------------------------------------------------------ forward


@pytest.mark.parametrize("N", [4, 5, 17, 64, 300])
@pytest.mark.parametrize("anchors", [False, True])
def test_forward_equals_serial_nerf(N, anchors):
    d = o.synthetic_inputs(3, N, seed=N, anchors=anchors)
    an = _anchors(d) if anchors else {}
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **an)
    y = o.nerf_serial(d["lengths"], d["angles"], d["dihedrals"], **an)
    assert np.abs(x - y).max() < 1e-12


@pytest.mark.parametrize("N", [4, 40, 500])
def test_internal_coordinate_round_trip(N):
    d = o.synthetic_inputs(2, N, seed=1, anchors=True)
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchors(d))
    L, A, D = o.measure_internal(x)
    assert np.abs(L - d["lengths"]).max() < 1e-12
    assert np.abs(A - d["angles"]).max() < 1e-11
    # IUPAC sign convention: atan2(|b2| b1.(b2 x b3), (b1 x b2).(b2 x b3)).
    assert np.abs(_wrap(D - d["dihedrals"])).max() < 1e-11


def test_default_frame_closed_form():
    d = o.synthetic_inputs(4, 10, seed=3, anchors=False)
    L, A = d["lengths"], d["angles"]
    x = o.reconstruct_forward(L, A, d["dihedrals"])
    assert np.abs(x[:, 0]).max() == 0.0
    np.testing.assert_allclose(x[:, 1], np.stack([L[:, 0], 0 * L[:, 0], 0 * L[:, 0]], -1), atol=1e-15)
    x2 = np.stack([L[:, 0] - L[:, 1] * np.cos(A[:, 0]), L[:, 1] * np.sin(A[:, 0]), 0 * L[:, 0]], -1)
    np.testing.assert_allclose(x[:, 2], x2, atol=1e-15)


def test_anchor_covariance():
    d = o.synthetic_inputs(3, 50, seed=4, anchors=True)
    x0 = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"])
    # Unnormalised anchors: the oracle must normalise and Gram-Schmidt them.
    fd = 3.0 * d["first_direction"]
    n0 = 0.5 * d["initial_normal"] + 0.7 * d["first_direction"]
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], p0=d["p0"], first_direction=fd, initial_normal=n0)
    dh = fd / np.linalg.norm(fd)
    nh = n0 - (n0 @ dh) * dh
    nh /= np.linalg.norm(nh)
    R = np.stack([dh, np.cross(nh, dh), nh], axis=-1)
    np.testing.assert_allclose(x, d["p0"] + x0 @ R.T, atol=1e-13)


@pytest.mark.parametrize("fd", [(0.0, 0.0, 1.0), (1.0, 0.0, 0.0), (0.95, 0.1, 0.0)])
def test_degenerate_normal_uses_stable_perpendicular(fd):
    # initial_normal parallel to first_direction: block.cu:126 falls back to
    # normalized(d0 x helper), helper = e_x unless |d0_x| >= 0.9 (frame_utils.cuh:23-31).
    d = o.synthetic_inputs(1, 8, seed=5, anchors=False)
    fd = np.array(fd)
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], first_direction=fd, initial_normal=2 * fd)
    dh = fd / np.linalg.norm(fd)
    helper = np.array([0.0, 1.0, 0.0]) if abs(dh[0]) >= 0.9 else np.array([1.0, 0.0, 0.0])
    nh = np.cross(dh, helper)
    nh /= np.linalg.norm(nh)
    th = np.cross(nh, dh)
    a0, l1 = d["angles"][0, 0], d["lengths"][0, 1]
    x2 = d["lengths"][0, 0] * dh + l1 * (-math.cos(a0) * dh + math.sin(a0) * th)
    np.testing.assert_allclose(x[0, 2], x2, atol=1e-15)


# ------------------------------------------------------------------ backward


def _torch_nerf(L, A, D):
    """Serial NeRF in torch (independent of the oracle's affine scan), default anchors."""
    B = L.shape[0]
    z = torch.zeros(B, dtype=L.dtype)
    pts = [torch.zeros(B, 3, dtype=L.dtype), torch.stack([L[:, 0], z, z], -1)]
    pts.append(torch.stack([L[:, 0] - L[:, 1] * torch.cos(A[:, 0]), L[:, 1] * torch.sin(A[:, 0]), z], -1))
    for k in range(D.shape[1]):
        a, b, c = pts[k], pts[k + 1], pts[k + 2]
        bc = (c - b) / torch.linalg.norm(c - b, dim=-1, keepdim=True)
        n = torch.cross(b - a, bc, dim=-1)
        n = n / torch.linalg.norm(n, dim=-1, keepdim=True)
        m = torch.stack([bc, torch.cross(n, bc, dim=-1), n], -1)
        l, t, p = L[:, k + 2], A[:, k + 1], D[:, k]
        d2 = torch.stack([-l * torch.cos(t), l * torch.sin(t) * torch.cos(p), l * torch.sin(t) * torch.sin(p)], -1)
        pts.append(c + torch.einsum("bij,bj->bi", m, d2))
    return torch.stack(pts, 1)


@pytest.mark.parametrize("N", [4, 6, 25])
def test_backward_matches_torch_autograd_of_serial_nerf(N):
    d = o.synthetic_inputs(3, N, seed=20 + N, anchors=False)
    L, A, D = (torch.tensor(d[k], requires_grad=True) for k in ("lengths", "angles", "dihedrals"))
    x = _torch_nerf(L, A, D)
    gt = torch.autograd.grad(x, (L, A, D), torch.tensor(d["grad"]))
    go = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"])
    for a, b in zip(gt, go):
        assert np.abs(a.numpy() - b).max() < 1e-12


def test_backward_matches_finite_differences_with_anchors():
    d = o.synthetic_inputs(1, 14, seed=6, anchors=True)
    an = _anchors(d)
    g = d["grad"]
    grads = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], g, **an)
    h = 1e-6
    for idx, key in enumerate(("lengths", "angles", "dihedrals")):
        fd = np.zeros_like(d[key])
        for j in range(d[key].shape[1]):
            plus = {k: d[k].copy() for k in ("lengths", "angles", "dihedrals")}
            minus = {k: d[k].copy() for k in ("lengths", "angles", "dihedrals")}
            plus[key][0, j] += h
            minus[key][0, j] -= h
            fp = np.sum(o.reconstruct_forward(plus["lengths"], plus["angles"], plus["dihedrals"], **an) * g)
            fm = np.sum(o.reconstruct_forward(minus["lengths"], minus["angles"], minus["dihedrals"], **an) * g)
            fd[0, j] = (fp - fm) / (2 * h)
        assert np.abs(fd - grads[idx]).max() < 1e-7


@pytest.mark.parametrize(
    "fd,n0",
    [
        (None, None),  # random anchors from the seed
        ([0.3, -1.7, 0.4], [2.0, 0.1, -0.5]),  # neither unit length nor orthogonal
        ([0.0, 0.0, 2.0], [0.0, 0.0, -3.0]),  # parallel: degenerate normal, helper e_x
        ([1.5, 0.2, 0.0], [3.0, 0.4, 0.0]),  # parallel with |d_x| >= 0.9: helper e_y
    ],
)
def test_anchor_gradients_match_finite_differences(fd, n0):
    d = o.synthetic_inputs(3, 12, seed=31, anchors=True)
    if fd is not None:
        d["first_direction"], d["initial_normal"] = np.array(fd, float), np.array(n0, float)
    an = _anchors(d)
    g = d["grad"]
    got = o.anchor_gradients(d["lengths"], d["angles"], d["dihedrals"], g, **an)
    # The degenerate branch holds while |n0 - (n0.d) d|^2 < 1e-12: steps small enough to stay
    # in it, with the larger roundoff that brings.
    degenerate = fd is not None and abs(np.dot(np.cross(fd, n0), np.cross(fd, n0))) < 1e-20
    h, tol = (1e-8, 1e-5) if degenerate else (1e-6, 1e-6)
    for key, want in zip(("p0", "first_direction", "initial_normal"), got):
        num = np.zeros(3)
        for j in range(3):
            plus, minus = dict(an), dict(an)
            plus[key] = an[key].copy()
            minus[key] = an[key].copy()
            plus[key][j] += h
            minus[key][j] -= h
            fp = np.sum(o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **plus) * g)
            fm = np.sum(o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **minus) * g)
            num[j] = (fp - fm) / (2 * h)
        assert np.abs(num - want).max() < tol * max(1.0, np.abs(want).max()), (key, num, want)


def test_anchor_gradients_match_torch_autograd():
    """The torch restatement of the recurrence, started from first-frame points built in
    torch from anchors that require grad."""
    d = o.synthetic_inputs(2, 9, seed=33, anchors=True)
    p0, fd, n0 = (torch.tensor(d[k], requires_grad=True) for k in ("p0", "first_direction", "initial_normal"))
    L, A, D = (torch.tensor(d[k]) for k in ("lengths", "angles", "dihedrals"))
    dd = fd / fd.norm()
    nr = n0 - (n0 @ dd) * dd
    nn = nr / nr.norm()
    t = torch.linalg.cross(nn, dd)
    xs = []
    for b in range(L.shape[0]):
        x1 = p0 + L[b, 0] * dd
        dir1 = -torch.cos(A[b, 0]) * dd + torch.sin(A[b, 0]) * t
        pts = [p0, x1, x1 + L[b, 1] * dir1]
        for k in range(L.shape[1] - 2):  # classic NeRF placement, step k uses L[k+2], A[k+1], D[k]
            a, bb, c = pts[-3], pts[-2], pts[-1]
            bc = (c - bb) / (c - bb).norm()
            nv = torch.linalg.cross(bb - a, bc)
            nv = nv / nv.norm()
            m = torch.stack([bc, torch.linalg.cross(nv, bc), nv], dim=1)
            th, ph = A[b, k + 1], D[b, k]
            loc = L[b, k + 2] * torch.stack([-torch.cos(th), torch.sin(th) * torch.cos(ph), torch.sin(th) * torch.sin(ph)])
            pts.append(c + m @ loc)
        xs.append(torch.stack(pts))
    x = torch.stack(xs)
    assert np.abs(x.detach().numpy() - o.reconstruct_forward(**{k: d[k] for k in ("lengths", "angles", "dihedrals")},
                                                                 p0=d["p0"], first_direction=d["first_direction"],
                                                                 initial_normal=d["initial_normal"])).max() < 1e-12
    got_t = torch.autograd.grad(x, (p0, fd, n0), torch.tensor(d["grad"]))
    got_o = o.anchor_gradients(d["lengths"], d["angles"], d["dihedrals"], d["grad"], p0=d["p0"],
                               first_direction=d["first_direction"], initial_normal=d["initial_normal"])
    for a, b in zip(got_t, got_o):
        assert np.abs(a.numpy() - b).max() < 1e-11


def test_adjoint_forms_agree():
    d = o.synthetic_inputs(3, 60, seed=7, anchors=True)
    args = (d["lengths"], d["angles"], d["dihedrals"], d["grad"])
    ref = o.reconstruct_backward(*args, **_anchors(d))
    world = o.reconstruct_backward_world(*args, **_anchors(d))
    frames = o.reconstruct_backward_frames(*args, **_anchors(d))
    for a, b, c in zip(ref, world, frames):
        assert np.abs(a - b).max() < 1e-12 * max(1, np.abs(a).max())
        assert np.abs(a - c).max() < 1e-12 * max(1, np.abs(a).max())


def test_frame_adjoint_handles_signs_the_world_form_cannot():
    d = o.synthetic_inputs(2, 20, seed=8, anchors=True)
    d["lengths"][:, 4] *= -1
    d["angles"][:, 0] = -0.6
    d["angles"][:, 6] = 3.6
    args = (d["lengths"], d["angles"], d["dihedrals"], d["grad"])
    ref = o.reconstruct_backward(*args, **_anchors(d))
    frames = o.reconstruct_backward_frames(*args, **_anchors(d))
    world = o.reconstruct_backward_world(*args, **_anchors(d))
    for a, c in zip(ref, frames):
        assert np.abs(a - c).max() < 1e-12 * max(1, np.abs(a).max())
    assert max(np.abs(a - w).max() for a, w in zip(ref, world)) > 1e-3


# ------------------------------------------------------------------ torsion


def test_torsion_constants_closed_form():
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    assert c.lengths == tuple(float(np.float32(v)) for v in BOND_LENGTHS)
    assert c.sin == tuple(math.sin(a) for a in BOND_ANGLES)
    assert c.cos == tuple(math.cos(a) for a in BOND_ANGLES)
    with pytest.raises(AssertionError):
        o.torsion_constants((1.0, 2.0), BOND_ANGLES)


def _tiled(c, B, N):
    L = np.array([c.lengths[i % 3] for i in range(N - 1)])[None].repeat(B, 0)
    A = np.array([math.atan2(c.sin[i % 3], c.cos[i % 3]) for i in range(N - 2)])[None].repeat(B, 0)
    return L, A


@pytest.mark.parametrize("N", [4, 5, 6, 47])
def test_torsion_equals_reconstruct_with_tiled_constants(N):
    rng = np.random.default_rng(N)
    raw = rng.normal(size=(2, 2 * (N - 3)))
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    L, A = _tiled(c, 2, N)
    D = np.arctan2(raw[:, 0::2], raw[:, 1::2])
    np.testing.assert_allclose(o.torsion_forward(raw, c), o.reconstruct_forward(L, A, D), atol=1e-14)


def test_torsion_backward_is_chain_rule_through_atan2():
    rng = np.random.default_rng(9)
    B, N = 2, 31
    raw = rng.normal(size=(B, 2 * (N - 3)))
    g = rng.normal(size=(B, N, 3))
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    L, A = _tiled(c, B, N)
    rs, rc = raw[:, 0::2], raw[:, 1::2]
    _, _, gD = o.reconstruct_backward(L, A, np.arctan2(rs, rc), g)
    n2 = rs * rs + rc * rc
    expect = np.empty_like(raw)
    expect[:, 0::2] = gD * rc / n2
    expect[:, 1::2] = -gD * rs / n2
    got = o.torsion_backward(raw, o.torsion_forward(raw, c), g, c)
    # 1/l is formed in float (torsion.cu:216): relative differences ~1e-8 are expected.
    assert np.abs(got - expect).max() <= 1e-7 * np.abs(expect).max()


def test_torsion_backward_finite_differences():
    rng = np.random.default_rng(10)
    raw = rng.normal(size=(1, 2 * 9))
    g = rng.normal(size=(1, 12, 3))
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    got = o.torsion_backward(raw, o.torsion_forward(raw, c), g, c)
    h = 1e-6
    fd = np.zeros_like(raw)
    for j in range(raw.shape[1]):
        p, m = raw.copy(), raw.copy()
        p[0, j] += h
        m[0, j] -= h
        fd[0, j] = (np.sum(o.torsion_forward(p, c) * g) - np.sum(o.torsion_forward(m, c) * g)) / (2 * h)
    assert np.abs(fd - got).max() < 1e-6 * max(1, np.abs(got).max())


def test_torsion_clamps_tiny_pairs():
    raw = np.zeros((1, 6))
    raw[0, 2:4] = (1e-10, -2e-10)
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    S, C, n2 = o._normalize_pairs(raw)
    assert n2[0, 0] == o.K_NORM_EPS2 and S[0, 0] == 0.0 and C[0, 0] == 0.0
    assert np.all(np.isfinite(o.torsion_forward(raw, c)))


# ------------------------------------------------------------------ golden fixtures (regression)


def test_golden_c0_regenerates(golden_c0):
    g = golden_c0
    np.testing.assert_array_equal(o.reconstruct_forward(g["lengths"], g["angles"], g["dihedrals"]), g["xyz"])
    gL, gA, gD = o.reconstruct_backward(g["lengths"], g["angles"], g["dihedrals"], g["grad"])
    np.testing.assert_array_equal(gL, g["grad_lengths"])
    np.testing.assert_array_equal(gD, g["grad_dihedrals"])
    L, A, D = o.measure_internal(g["xyz"])
    assert np.abs(_wrap(D - g["dihedrals"])).max() < 1e-11


def test_golden_anchored_regenerates(golden_anchored):
    g = golden_anchored
    an = dict(p0=g["p0"], first_direction=g["first_direction"], initial_normal=g["initial_normal"])
    np.testing.assert_allclose(o.reconstruct_forward(g["lengths"], g["angles"], g["dihedrals"], **an), g["xyz"], atol=0)
    np.testing.assert_allclose(o.nerf_serial(g["lengths"], g["angles"], g["dihedrals"], **an), g["xyz"], atol=1e-13)


def test_golden_torsion_regenerates(golden_torsion):
    g = golden_torsion
    c = o.torsion_constants(tuple(g["bond_lengths"]), tuple(g["bond_angles"]))
    np.testing.assert_array_equal(o.torsion_forward(g["raw_pairs"], c), g["xyz"])
    np.testing.assert_array_equal(o.torsion_backward(g["raw_pairs"], g["xyz"], g["grad"], c), g["grad_raw"])


# ------------------------------------------------------------------ planted mistakes


def test_checks_catch_a_flipped_dihedral_sign(monkeypatch):
    real = o.local_transform
    monkeypatch.setattr(o, "local_transform", lambda l, t, p: real(l, t, -p))
    d = o.synthetic_inputs(1, 30, seed=11, anchors=False)
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"])
    _, _, D = o.measure_internal(x)
    assert np.abs(_wrap(D - d["dihedrals"])).max() > 1e-3
    assert np.abs(x - o.nerf_serial(d["lengths"], d["angles"], d["dihedrals"])).max() > 1e-3


def test_checks_catch_a_transposed_compose(monkeypatch):
    monkeypatch.setattr(o, "_compose", lambda am, av, bm, bv: (bm @ am, bv + np.einsum("bij,bj->bi", bm, av)))
    d = o.synthetic_inputs(1, 30, seed=12, anchors=False)
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"])
    assert np.abs(x - o.nerf_serial(d["lengths"], d["angles"], d["dihedrals"])).max() > 1e-3


def test_checks_catch_a_dropped_first_frame_gradient_term():
    d = o.synthetic_inputs(2, 12, seed=13, anchors=False)
    gL, gA, gD = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"])
    L, A, D = (torch.tensor(d[k], requires_grad=True) for k in ("lengths", "angles", "dihedrals"))
    tA = torch.autograd.grad(_torch_nerf(L, A, D), (A,), torch.tensor(d["grad"]))[0].numpy()
    # Dropping the l1 * grad_p2 . d_dir term of block.cu:227 breaks agreement with autograd.
    ff = o.first_frame(d["lengths"][:, 0], d["lengths"][:, 1], d["angles"][:, 0], (0, 0, 0), (1, 0, 0), (0, 0, 1))
    s, c = np.sin(d["angles"][:, 0]), np.cos(d["angles"][:, 0])
    d_dir = s[:, None] * ff.dir0 + c[:, None] * ff.turn0
    F2 = d["grad"][:, 2:].sum(1)
    dropped = gA[:, 0] - d["lengths"][:, 1] * np.sum(F2 * d_dir, -1)
    assert np.abs(gA[:, 0] - tA[:, 0]).max() < 1e-12
    assert np.abs(dropped - tA[:, 0]).max() > 1e-3


# ------------------------------------------------------------------ the CPU baseline (PyTorch)


def _torch_inputs(d):
    return {k: torch.tensor(v, dtype=torch.float64) for k, v in d.items()}


@pytest.mark.parametrize("N", [4, 5, 64, 300])
def test_cpu_torch_baseline_matches_the_oracle(N):
    """bench.py's CPU baseline (oracle/cpu_torch.py) equals the pinned float64 oracle: forward
    within 1e-12, world-frame adjoint within 1e-10 relative of the reference-form backward."""
    from oracle import cpu_torch as ct

    d = o.synthetic_inputs(4, N, seed=50 + N, anchors=True)
    t = _torch_inputs(d)
    x = ct.forward(t["lengths"], t["angles"], t["dihedrals"], t["p0"], t["first_direction"], t["initial_normal"])
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchors(d))
    assert np.abs(x.numpy() - ref).max() <= 1e-12
    got = ct.backward(x, t["grad"])
    want = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchors(d))
    for a, b in zip(got, want):
        assert np.abs(a.numpy() - b).max() <= 1e-10 * np.abs(b).max()


@pytest.mark.parametrize("fd", [[0.0, 0.0, 2.0], [1.0, 0.1, 0.0]])
def test_cpu_torch_baseline_degenerate_normal(fd):
    from oracle import cpu_torch as ct

    d = o.synthetic_inputs(2, 30, seed=8, anchors=True)
    d["first_direction"] = np.array(fd)
    d["initial_normal"] = np.array(fd) * -3.0
    t = _torch_inputs(d)
    x = ct.forward(t["lengths"], t["angles"], t["dihedrals"], t["p0"], t["first_direction"], t["initial_normal"])
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchors(d))
    assert np.abs(x.numpy() - ref).max() <= 1e-12


def test_cpu_torch_torsion_matches_the_oracle():
    """Torsion forward and backward, with a zero pair and a pair below the 1e-8 clamp."""
    from oracle import cpu_torch as ct

    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    rng = np.random.default_rng(12)
    raw = rng.normal(size=(4, 2 * 50))
    raw[0, 4:6] = 0.0
    raw[1, 6:8] = (1e-9, 0.0)
    g = rng.normal(size=(4, 53, 3))
    x = ct.torsion_forward(torch.tensor(raw), c.lengths, c.sin, c.cos)
    xr = o.torsion_forward(raw, c)
    assert np.abs(x.numpy() - xr).max() <= 1e-12
    gr = o.torsion_backward(raw, xr, g, c)
    got = ct.torsion_backward(torch.tensor(raw), x, torch.tensor(g), c.lengths)
    assert np.abs(got.numpy() - gr).max() <= 1e-10 * np.abs(gr).max()


# ------------------------------------------------------------------ superposed losses


def _rot(rng):
    q, _ = np.linalg.qr(rng.normal(size=(3, 3)))
    return q * np.sign(np.linalg.det(q))


def test_superpose_zero_for_rigid_copies_and_invariant():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(4, 30, 3)) * 2.0
    Q = np.stack([_rot(rng) for _ in range(4)])
    moved = np.einsum("bij,bkj->bki", Q, x) + rng.normal(size=(4, 1, 3)) * 5
    assert np.abs(o.superposed_loss(x, moved, squared=True)).max() < 1e-20
    t = rng.normal(size=x.shape)
    base = o.superposed_loss(x, t)
    Q2 = np.stack([_rot(rng) for _ in range(4)])
    t_moved = np.einsum("bij,bkj->bki", Q2, t) - 3.0
    assert np.allclose(o.superposed_loss(x, t_moved), base, rtol=1e-12)
    assert np.allclose(o.superposed_loss(t, x), base, rtol=1e-12)  # symmetric in its arguments


def test_superpose_is_a_proper_rotation_for_mirrored_targets():
    rng = np.random.default_rng(4)
    x = rng.normal(size=(3, 25, 3)) * [3.0, 2.0, 1.0]
    mirrored = x * [1.0, 1.0, -1.0]  # a reflection: no proper rotation maps x onto it
    R, _, _, msd = o.superpose(x, mirrored)
    assert np.allclose(np.linalg.det(R), 1.0)
    assert np.all(msd > 0.1)


def test_superpose_beats_every_sampled_rotation():
    """Optimality: no sampled proper rotation (uniform quaternions) and no small perturbation
    of the solution does better."""
    rng = np.random.default_rng(5)
    x = rng.normal(size=(1, 40, 3))
    t = np.einsum("ij,bkj->bki", _rot(rng), x) + 0.3 * rng.normal(size=x.shape)
    R, xb, tb, msd = o.superpose(x, t)
    xc, tc = x[0] - xb[0], t[0] - tb[0]

    def msd_of(Rm):
        return np.mean(np.sum((xc @ Rm.T - tc) ** 2, axis=1))

    q = rng.normal(size=(20000, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    w, a, b, c = q.T
    Rs = np.stack([np.stack([w*w+a*a-b*b-c*c, 2*(a*b-w*c), 2*(a*c+w*b)], -1),
                   np.stack([2*(b*a+w*c), w*w-a*a+b*b-c*c, 2*(b*c-w*a)], -1),
                   np.stack([2*(c*a-w*b), 2*(c*b+w*a), w*w-a*a-b*b+c*c], -1)], -2)
    sampled = np.mean(np.sum((np.einsum("rij,kj->rki", Rs, xc) - tc) ** 2, axis=-1), axis=1)
    assert msd[0] <= sampled.min() + 1e-12
    for _ in range(20):
        k = rng.normal(size=3) * 1e-3
        K = np.array([[0, -k[2], k[1]], [k[2], 0, -k[0]], [-k[1], k[0], 0]])
        assert msd_of(R[0] @ (np.eye(3) + K + K @ K / 2)) >= msd[0] - 1e-15


@pytest.mark.parametrize("squared", [True, False])
def test_superposed_gradient_finite_differences(squared):
    rng = np.random.default_rng(6)
    x = rng.normal(size=(2, 15, 3))
    t = rng.normal(size=(2, 15, 3))
    w = np.array([1.5, -0.5])
    g = o.superposed_grad_xyz(x, t, w, squared)
    h = 1e-6
    for b, i, a in [(0, 0, 0), (0, 7, 2), (1, 14, 1), (1, 3, 0)]:
        xp, xm = x.copy(), x.copy()
        xp[b, i, a] += h
        xm[b, i, a] -= h
        fd = w[b] * (o.superposed_loss(xp, t, squared)[b] - o.superposed_loss(xm, t, squared)[b]) / (2 * h)
        assert abs(fd - g[b, i, a]) <= 1e-7 * max(1.0, abs(fd))


@pytest.mark.parametrize("squared", [True, False])
def test_superposed_loss_through_the_chain_finite_differences(squared):
    """The composition the fused kernels compute: the forward, the superposed loss, and the
    reference backward fed with superposed_grad_xyz, against central differences in L, A, D."""
    d = o.synthetic_inputs(2, 14, seed=9, anchors=True)
    an = _anchors(d)
    t = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **an)
    t = t + np.random.default_rng(1).normal(0.0, 0.2, t.shape)

    def loss(L, A, D):
        return o.superposed_loss(o.reconstruct_forward(L, A, D, **an), t, squared).sum()

    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **an)
    grads = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], o.superposed_grad_xyz(x, t, None, squared),
                                   **an)
    h = 1e-6
    for k, (name, g) in enumerate(zip(("lengths", "angles", "dihedrals"), grads)):
        for b, j in [(0, 0), (1, 5), (0, g.shape[1] - 1)]:
            args = [d["lengths"].copy(), d["angles"].copy(), d["dihedrals"].copy()]
            args[k][b, j] += h
            fp = loss(*args)
            args[k][b, j] -= 2 * h
            fm = loss(*args)
            assert abs((fp - fm) / (2 * h) - g[b, j]) <= 1e-6 * max(1.0, abs(g[b, j])), (name, b, j)


def test_torsion_losses_through_the_chain_finite_differences():
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    rng = np.random.default_rng(10)
    raw = rng.normal(size=(2, 2 * 12))
    t = o.torsion_forward(raw, c) + rng.normal(0.0, 0.2, (2, 15, 3))
    x = o.torsion_forward(raw, c)
    for kind in ("squared_distance", "msd", "rmsd"):
        if kind == "squared_distance":
            f = lambda r: ((o.torsion_forward(r, c) - t) ** 2).sum()  # noqa: E731
            gx = 2.0 * (x - t)
        else:
            sq = kind == "msd"
            f = lambda r: o.superposed_loss(o.torsion_forward(r, c), t, sq).sum()  # noqa: E731
            gx = o.superposed_grad_xyz(x, t, None, sq)
        g = o.torsion_backward(raw, x, gx, c)
        h = 1e-6
        for b, j in [(0, 0), (1, 7), (0, 23)]:
            rp, rm = raw.copy(), raw.copy()
            rp[b, j] += h
            rm[b, j] -= h
            fd = (f(rp) - f(rm)) / (2 * h)
            # torsion_backward forms 1/l in float (torsion.cu:216), a 1e-8 relative effect.
            assert abs(fd - g[b, j]) <= 1e-6 * max(1.0, abs(fd)), (kind, b, j)


def test_superpose_header_matches_the_oracle(tmp_path):
    """cufk_amd/csrc/superpose.h (Horn's quaternion eigenproblem, as the kernels run it) built
    for the host with g++, against the SVD oracle: msd to 1e-10 relative, R^T and the offset
    to 1e-9, for generic, well-fitted, mirrored and collinear chains."""
    import shutil
    import subprocess

    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no host C++ compiler")
    root = Path(__file__).resolve().parent.parent
    src = tmp_path / "sp.cpp"
    src.write_text(
        '#include "superpose.h"\n#include <cstdio>\nusing namespace cufk_amd;\n'
        "int main() { int n; double cx[3], ct[3];\n"
        '  while (scanf("%d %lf %lf %lf %lf %lf %lf", &n, cx, cx + 1, cx + 2, ct, ct + 1, ct + 2) == 7) {\n'
        "    double s[kSuperposeSums] = {};\n"
        "    for (int i = 0; i < n; ++i) { double x[3], t[3];\n"
        '      if (scanf("%lf %lf %lf %lf %lf %lf", x, x + 1, x + 2, t, t + 1, t + 2) != 6) return 1;\n'
        "      for (int k = 0; k < 3; ++k) { x[k] -= cx[k]; t[k] -= ct[k]; }\n"
        "      superpose_add(s, x, t); }\n"
        "    double out[kSuperposeRecord]; superpose_solve(s, n, cx, ct, out);\n"
        '    for (int i = 0; i < 13; ++i) printf("%.17g ", out[i]); printf("\\n"); }\n  return 0; }\n'
    )
    exe = tmp_path / "sp"
    subprocess.run([gxx, "-O2", "-std=c++17", f"-I{root / 'cufk_amd' / 'csrc'}", str(src), "-o", str(exe)], check=True)
    rng = np.random.default_rng(11)
    cases = []
    for n in (4, 5, 64, 400):
        x = rng.normal(size=(n, 3)) * [3.0, 2.0, 1.0] + 4.0
        cases.append((x, x @ _rot(rng).T + 0.2 * rng.normal(size=x.shape) - 6.0, True))
    x = rng.normal(size=(50, 3))
    cases.append((x, x @ _rot(rng).T + 1e-5 * rng.normal(size=x.shape), True))  # well fitted
    cases.append((x, x * [1.0, -1.0, 1.0], True))  # mirrored
    line = np.outer(np.arange(6.0), [1.0, 2.0, 0.5])
    cases.append((line, rng.normal(size=(6, 3)), False))  # collinear chain: R is not unique
    cases.append((x, x.copy(), True))  # identical: the identity, msd 0
    cases.append((x, np.full_like(x, 1.5), False))  # target at one point: the key matrix is 0
    square = np.array([[1.0, 1, 0], [-1, 1, 0], [-1, -1, 0], [1, -1, 0], [0.5, 0.2, 0]])
    cases.append((square, -square, True))  # inversion of a planar set: a half turn about its normal
    for k in range(200):  # fits from near-exact to pure noise
        n = int(rng.integers(4, 80))
        x = rng.normal(size=(n, 3)) * rng.uniform(0.5, 5.0, 3)
        noise = 10.0 ** rng.uniform(-7, 1)
        cases.append((x, x @ _rot(rng).T + noise * rng.normal(size=x.shape) + rng.normal(size=3) * 10, True))
    text = ""
    for x, t, _ in cases:
        text += f"{len(x)} " + " ".join(repr(float(v)) for v in (*x[2], *t[2])) + "\n"
        text += "\n".join(" ".join(repr(float(v)) for v in (*a, *b)) for a, b in zip(x, t)) + "\n"
    out = subprocess.run([str(exe)], input=text, capture_output=True, text=True, check=True).stdout.split("\n")
    for (x, t, unique), line_out in zip(cases, out):
        got = np.array([float(v) for v in line_out.split()])
        R, xb, tb, msd = o.superpose(x[None], t[None])
        # msd = (sum |x'|^2 + sum |t'|^2 - 2 lambda) / N cancels to about 1e-15 of its terms.
        size = (np.sum((x - xb) ** 2) + np.sum((t - tb) ** 2)) / len(x)
        assert abs(got[12] - msd[0]) <= 1e-10 * msd[0] + 1e-14 * size
        if unique and msd[0] > 1e-10 * size:
            M = got[:9].reshape(3, 3)
            assert np.abs(M - R[0].T).max() <= 1e-9
            assert np.abs(got[9:12] - (xb[0] - R[0].T @ tb[0])).max() <= 1e-9 * max(1.0, np.abs(xb).max())


def _superpose_move_exe(tmp_path):
    """superpose_move of cufk_amd/csrc/superpose.h built for the host: reads m, e, f, s1, s2
    and prints the 17 moved sums."""
    import shutil
    import subprocess

    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no host C++ compiler")
    root = Path(__file__).resolve().parent.parent
    src = tmp_path / "mv.cpp"
    src.write_text(
        '#include "superpose.h"\n#include <cstdio>\nusing namespace cufk_amd;\n'
        "int main() { double m, e[3], f[3], s1[6], s2[11];\n"
        '  while (scanf("%lf", &m) == 1) {\n'
        '    for (int k = 0; k < 3; ++k) if (scanf("%lf", e + k) != 1) return 1;\n'
        '    for (int k = 0; k < 3; ++k) if (scanf("%lf", f + k) != 1) return 1;\n'
        '    for (int k = 0; k < 6; ++k) if (scanf("%lf", s1 + k) != 1) return 1;\n'
        '    for (int k = 0; k < 11; ++k) if (scanf("%lf", s2 + k) != 1) return 1;\n'
        "    double out[kSuperposeSums]; superpose_move(s1, s2, m, e, f, out);\n"
        '    for (int k = 0; k < kSuperposeSums; ++k) printf("%.17g ", out[k]); printf("\\n"); }\n  return 0; }\n'
    )
    exe = tmp_path / "mv"
    subprocess.run([gxx, "-O2", "-std=c++17", f"-I{root / 'cufk_amd' / 'csrc'}", str(src), "-o", str(exe)], check=True)
    return exe


def _direct_sums(x, t, cx, ct):
    """The 17 superposition sums of the points about (cx, ct), straight from their definition."""
    a, b = x - cx, t - ct
    return np.concatenate([a.sum(0), b.sum(0), (a[:, :, None] * b[:, None, :]).sum(0).ravel(),
                           [np.sum(a * a), np.sum(b * b)]])


@pytest.mark.parametrize("plant", [None, "drop_cross", "swap_ef"])
def test_superpose_move_equals_the_direct_sums(tmp_path, plant):
    """The fused forwards sum each thread's points about that thread's own first point and
    target point, then move the sums to the chain's shift points with superpose_move: chains cut
    into runs of 1 to 15 points (as threads hold them), moved and added up, equal the sums taken
    directly about the chain's shift points (1e-12 relative).  Planted mistakes in the inputs
    (the cross term's first moments zeroed; e and f exchanged) fail the same comparison."""
    import subprocess

    exe = _superpose_move_exe(tmp_path)
    rng = np.random.default_rng(21)
    chains, text = [], ""
    for n in (4, 15, 16, 200, 2049):
        x = np.cumsum(rng.normal(size=(n, 3)) * 0.15, axis=0) + rng.normal(size=3) * 5.0
        t = x @ _rot(rng).T + rng.normal(size=3) * 4.0 + rng.normal(size=x.shape) * 0.3
        cx, ct = x[2], t[2]
        runs, i = [], 0
        while i < n:
            m = int(rng.integers(1, 16))
            runs.append((i, min(n, i + m)))
            i += m
        chains.append((x, t, cx, ct, len(runs)))
        for i0, i1 in runs:
            xl, tl = x[i0], t[i0]
            a, b = x[i0:i1] - xl, t[i0:i1] - tl
            s1 = np.concatenate([a.sum(0), b.sum(0)])
            if plant == "drop_cross":
                s1 = np.zeros(6)
            s2 = np.concatenate([(a[:, :, None] * b[:, None, :]).sum(0).ravel(), [np.sum(a * a), np.sum(b * b)]])
            e, f = xl - cx, tl - ct
            if plant == "swap_ef":
                e, f = f, e
            text += " ".join(repr(float(v)) for v in (i1 - i0, *e, *f, *s1, *s2)) + "\n"
    out = subprocess.run([str(exe)], input=text, capture_output=True, text=True, check=True).stdout.split("\n")
    row = 0
    worst = 0.0
    for x, t, cx, ct, nruns in chains:
        moved = np.sum([[float(v) for v in out[row + r].split()] for r in range(nruns)], axis=0)
        row += nruns
        want = _direct_sums(x, t, cx, ct)
        scale = np.abs(want).max()
        worst = max(worst, np.abs(moved - want).max() / scale)
    if plant is None:
        assert worst <= 1e-12, worst
    else:
        assert worst > 1e-6, (plant, worst)


def test_checks_catch_a_transposed_superposition(monkeypatch):
    """Planted mistake: the rotation transposed in superposed_grad_xyz's superposition.  The
    finite-difference pin above fails on it."""
    real = o.superpose

    def transposed(x, t):
        R, xb, tb, msd = real(x, t)
        return np.swapaxes(R, 1, 2), xb, tb, msd

    rng = np.random.default_rng(6)
    x = rng.normal(size=(1, 15, 3))
    t = rng.normal(size=(1, 15, 3))
    monkeypatch.setattr(o, "superpose", transposed)
    g = o.superposed_grad_xyz(x, t, None, True)
    monkeypatch.setattr(o, "superpose", real)
    h = 1e-6
    xp, xm = x.copy(), x.copy()
    xp[0, 7, 2] += h
    xm[0, 7, 2] -= h
    fd = (o.superposed_loss(xp, t, True)[0] - o.superposed_loss(xm, t, True)[0]) / (2 * h)
    assert abs(fd - g[0, 7, 2]) > 1e-4 * max(1.0, abs(fd))

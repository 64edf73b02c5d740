"""Long chains (reconstruct_long): the segmented path against the float64 oracle.

Segments are forced short (segment_steps) so that small chains, which the oracle handles in
seconds, cross many segment boundaries; a few cases run past the 2051-point cap of
reconstruct with the default segment length.  Bars: float64 as the single-workgroup path
(1e-12 relative forward, 1e-10 relative gradients); float32 error bounds printed and held
to the same per-length scale as the single-workgroup path; float16/bfloat16 reported with
sanity bounds.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import nerf64 as o

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cufk(device):
    import cufk_amd

    return cufk_amd


def _dev(x, dtype, device, requires_grad=False):
    t = torch.as_tensor(np.asarray(x), dtype=torch.float64).to(device=device, dtype=dtype)
    return t.requires_grad_(requires_grad)


def _round(x, dtype):
    return torch.as_tensor(np.asarray(x), dtype=torch.float64).to(dtype).double().numpy()


def _inputs(B, N, seed, anchors, dtype=torch.float64):
    d = o.synthetic_inputs(B, N, seed, anchors=anchors)
    return {k: _round(v, dtype) for k, v in d.items()}


def _anchors(d, dtype, device):
    if "p0" not in d:
        return {}
    return {k: _dev(d[k], dtype, device) for k in ("p0", "first_direction", "initial_normal")}


def _anchor_np(d):
    return {k: d.get(k) for k in ("p0", "first_direction", "initial_normal")}


def _run_long(cufk, d, dtype, device, segment_steps, grad=True):
    L = _dev(d["lengths"], dtype, device, grad)
    A = _dev(d["angles"], dtype, device, grad)
    D = _dev(d["dihedrals"], dtype, device, grad)
    xyz = cufk.reconstruct_long(L, A, D, **_anchors(d, dtype, device), segment_steps=segment_steps)
    if not grad:
        return xyz, None
    grads = torch.autograd.grad(xyz, (L, A, D), _dev(d["grad"], dtype, device))
    return xyz, grads


def _ref(d):
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    g = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    return x, g


# (N, segment_steps): one-step tails, segments smaller than one lane's items, every plan
# (256 -> (1,4), 512 -> (1,8), 1024 -> (2,8), 2048 -> (4,8)), chains past the cap.
CASES = [(5, 1), (11, 3), (40, 8), (300, 64), (1000, 255), (1200, 512), (3000, 1024), (2052, 2048), (5000, None)]


@pytest.mark.parametrize("N,seg", CASES)
def test_long_fp64_matches_oracle(cufk, device, N, seg):
    d = _inputs(3, N, seed=100 + N, anchors=True)
    xyz, grads = _run_long(cufk, d, torch.float64, device, seg)
    ref_x, ref_g = _ref(d)
    err = np.abs(xyz.detach().cpu().numpy() - ref_x).max()
    print(f"fp64 long N={N} seg={seg}: forward max err {err:.3e}")
    assert err <= 1e-12 * max(1.0, np.abs(ref_x).max())
    for name, got, want in zip(("lengths", "angles", "dihedrals"), grads, ref_g):
        gerr = np.abs(got.cpu().numpy() - want).max() / np.abs(want).max()
        print(f"  grad {name}: rel max err {gerr:.3e}")
        assert gerr <= 1e-10


@pytest.mark.parametrize("N,seg", [(2049, 256), (2049, 1000), (6000, None)])
def test_long_fp32_tolerance(cufk, device, N, seg):
    """float32 at the cap length with several segments, and past the cap: the forward holds
    the single-workgroup bar at N = 2049 (1e-5 nm RMS, 1e-4 nm max) and its max error
    relative to the chain extent past it; gradients 5e-5 relative (the exact adjoint's
    single-workgroup bar)."""
    d = _inputs(8, N, seed=7, anchors=True, dtype=torch.float32)
    xyz, grads = _run_long(cufk, d, torch.float32, device, seg)
    ref_x, ref_g = _ref(d)
    diff = xyz.detach().double().cpu().numpy() - ref_x
    rms = math.sqrt(np.mean(np.sum(diff**2, axis=-1)))
    mx = np.abs(diff).max()
    extent = np.abs(ref_x).max()
    print(f"fp32 long N={N} seg={seg}: rms {rms:.3e} nm, max {mx:.3e} nm, extent {extent:.1f} nm")
    assert rms <= 1e-5 * max(1.0, N / 2049)
    assert mx <= 1e-4 * max(1.0, N / 2049)
    for name, got, want in zip(("lengths", "angles", "dihedrals"), grads, ref_g):
        gerr = np.abs(got.double().cpu().numpy() - want).max() / np.abs(want).max()
        print(f"  grad {name}: rel max err {gerr:.3e}")
        assert gerr <= 5e-5


def test_long_single_segment_equals_reconstruct(cufk, device):
    """One segment with the plan reconstruct picks (segment_steps = N-3) runs the same
    forward arithmetic: bit-identical positions."""
    for dtype in (torch.float32, torch.float64, torch.bfloat16):
        d = _inputs(5, 700, seed=3, anchors=True, dtype=dtype)
        L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
        an = _anchors(d, dtype, device)
        a = cufk.reconstruct(L, A, D, **an)
        b = cufk.reconstruct_long(L, A, D, **an, segment_steps=697)
        assert torch.equal(a, b), dtype


def test_long_default_segments_past_the_cap(cufk, device):
    """Without segment_steps: N <= 2051 is reconstruct itself; past it the default segments."""
    d = _inputs(2, 300, seed=5, anchors=False, dtype=torch.float32)
    L, A, D = (_dev(d[k], torch.float32, device) for k in ("lengths", "angles", "dihedrals"))
    assert torch.equal(cufk.reconstruct_long(L, A, D), cufk.reconstruct(L, A, D))
    with pytest.raises(RuntimeError, match="at most 2048 local transforms"):
        n = 2100
        cufk.reconstruct(torch.ones(1, n - 1, device=device), torch.ones(1, n - 2, device=device),
                         torch.ones(1, n - 3, device=device))


def test_long_fp64_gradcheck(cufk, device):
    d = _inputs(2, 23, seed=9, anchors=True)
    L, A, D = (_dev(d[k], torch.float64, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = _anchors(d, torch.float64, device)
    assert torch.autograd.gradcheck(lambda l, a, t: cufk.reconstruct_long(l, a, t, **an, segment_steps=4), (L, A, D),
                                    eps=1e-6, atol=1e-8, rtol=1e-6)


def test_long_irregular_chains(cufk, device):
    """Negative and zero bonds, bond angles near 0 and pi, inside non-head segments and at
    segment boundaries: the segments they touch take the exact adjoint, the others the
    position-based one (float32 bar 5e-5 relative)."""
    d = _inputs(4, 400, seed=11, anchors=True, dtype=torch.float32)
    d["lengths"][0, 130] *= -1  # inside segment 2 (steps 128..191 place points 131..)
    d["lengths"][1, 66] = 0.0  # first step of segment 1 uses L[66]
    d["angles"][2, 65] = 0.05  # step 64 uses A[65]: first step of segment 1
    d["angles"][3, 200] = math.pi - 0.05
    d = {k: _round(v, torch.float32) for k, v in d.items()}
    xyz, grads = _run_long(cufk, d, torch.float32, device, 64)
    ref_x, ref_g = _ref(d)
    mx = np.abs(xyz.detach().double().cpu().numpy() - ref_x).max()
    print(f"fp32 long irregular: forward max err {mx:.3e}")
    assert mx <= 1e-4
    for got, want in zip(grads, ref_g):
        err = np.abs(got.double().cpu().numpy() - want).max(axis=1) / np.abs(want).max(axis=1)
        print("  per-chain grad rel err", err)
        assert err.max() <= 5e-5


def test_long_position_adjoint_far_anchor_and_boundary_bonds(cufk, device):
    """The position-based adjoint of later segments runs over positions local to each
    segment, so an anchor 90 nm from the origin (which sends the head segment to the
    exact adjoint) leaves the later segments at the float32 bar; a zero bond x1-x2 of a later
    segment (a step of the segment before it) sends that segment to the exact adjoint too."""
    d = _inputs(4, 1500, seed=21, anchors=True, dtype=torch.float32)
    d["p0"] = np.array([60.0, -40.0, 50.0])
    d["lengths"][1, 129] = 0.0  # segment 2 (steps 128..) has x1-x2 = L[129], from step 127
    d["lengths"][2, 257] = 1.0e-7  # below the float32 minimum bond: segments 3 and 4 exact
    d = {k: _round(v, torch.float32) for k, v in d.items()}
    xyz, grads = _run_long(cufk, d, torch.float32, device, 128)
    ref_x, ref_g = _ref(d)
    for got, want in zip(grads, ref_g):
        err = np.abs(got.double().cpu().numpy() - want).max(axis=1) / np.abs(want).max(axis=1)
        print("  per-chain grad rel err", err)
        assert err.max() <= 5e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_long_angles_beyond_the_polynomial_range(cufk, device, dtype):
    """Angles with |x| > 65536 in non-head segments switch those segments to the library
    sin/cos; float32 bars as above, bfloat16 2e-2 relative to the chain extent."""
    d = _inputs(3, 300, seed=12, anchors=True, dtype=dtype)
    d["dihedrals"][0, 150] += 2 * math.pi * 20000.0
    d["angles"][1, 70] -= 2 * math.pi * 30000.0
    d["angles"][2, 299 - 2] = 1.0e6 if dtype == torch.float32 else -1.0e6
    d = {k: _round(v, dtype) for k, v in d.items()}
    xyz, grads = _run_long(cufk, d, dtype, device, 64)
    ref_x, ref_g = _ref(d)
    err = np.abs(xyz.detach().double().cpu().numpy() - ref_x).max() / np.abs(ref_x).max()
    print(f"{dtype} long wide angles: forward rel max err {err:.3e}")
    assert err <= (1e-5 if dtype == torch.float32 else 2e-2)
    for got, want in zip(grads, ref_g):
        gerr = np.abs(got.double().cpu().numpy() - want).max() / np.abs(want).max()
        print(f"  grad rel max err {gerr:.3e}")
        assert gerr <= (5e-5 if dtype == torch.float32 else 5e-2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_long_low_precision_reported(cufk, device, dtype):
    """Half types: local positions of non-head segments are rounded to the type before they
    are moved into place, so the forward error is up to about twice the single path's; the
    gradients use the saved (rounded) positions for the segment sums.  Sanity bounds as for
    the single-workgroup path."""
    d = _inputs(4, 3000, seed=13, anchors=False, dtype=dtype)
    xyz, grads = _run_long(cufk, d, dtype, device, 512)
    ref_x, ref_g = _ref(d)
    rel = np.abs(xyz.detach().double().cpu().numpy() - ref_x).max() / np.abs(ref_x).max()
    gerr = [float(np.abs(g.double().cpu().numpy() - r).max() / np.abs(r).max()) for g, r in zip(grads, ref_g)]
    print(f"{dtype} long N=3000: forward rel max {rel:.2e}, grads " + ", ".join(f"{e:.2e}" for e in gerr))
    assert torch.isfinite(xyz).all()
    assert rel <= 1e-2 and max(gerr) <= 3e-2


def test_long_modified_output_recomputes(cufk, device):
    """An output changed in place (version bump) is recomputed for the backward: shifting
    every position by 5 nm would change the segment moments if the saved values were used;
    the recompute repeats the same arithmetic, so the gradients are bit-identical."""
    d = _inputs(2, 500, seed=14, anchors=True, dtype=torch.float32)
    dtype = torch.float32
    g = _dev(d["grad"], dtype, device)
    outs = []
    for modify in (False, True):
        L, A, D = (_dev(d[k], dtype, device, True) for k in ("lengths", "angles", "dihedrals"))
        xyz = cufk.reconstruct_long(L, A, D, **_anchors(d, dtype, device), segment_steps=100)
        if modify:
            with torch.no_grad():
                xyz.add_(5.0)
        outs.append(torch.autograd.grad(xyz, (L, A, D), g))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_long_validation(cufk, device):
    L = torch.ones(1, 99, device=device)
    A = torch.ones(1, 98, device=device)
    D = torch.ones(1, 97, device=device)
    with pytest.raises(RuntimeError, match="segment_steps must be in"):
        cufk.reconstruct_long(L, A, D, segment_steps=4096)
    with pytest.raises(RuntimeError, match="bad angles shape"):
        cufk.reconstruct_long(L, A[:, :50], D, segment_steps=16)
    with pytest.raises(RuntimeError, match="gradients are not supported"):
        cufk.reconstruct_long(L, A, D, torch.zeros(3, device=device, requires_grad=True), segment_steps=16)
    empty = cufk.reconstruct_long(L[:0], A[:0], D[:0], segment_steps=16)
    assert empty.shape == (0, 100, 3)

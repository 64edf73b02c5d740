"""GPU parity of the HIP path (through cufk_amd._C -> libcufk_hip.so) against the float64 oracle.

Tolerances (stated per test):
* float64 coordinates: max |x - oracle| <= 1e-12 * max(1, |x|) (reference-convention scan, fp64).
* float32 coordinates at N = 2049: RMS <= 1e-5 nm and max-abs <= 1e-4 nm against float64
  evaluated on the same (float32-valued) inputs.
* float64 gradients: torch.autograd.gradcheck, and max |g - oracle| <= 1e-9 * max|oracle|.
* float32 gradients: max |g - oracle| <= 5e-5 * max|oracle| per output (normwise).
* float16 / bfloat16: errors are reported, not gated (finite outputs are required).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import nerf64 as o

pytestmark = pytest.mark.gpu

BOND_LENGTHS = (0.14685231, 0.15365194, 0.13405086)
BOND_ANGLES = (1.9676635, 2.062335, 2.164016)


@pytest.fixture(scope="module")
def cufk(device):
    import cufk_amd

    return cufk_amd


def _dev(x, dtype, device, requires_grad=False):
    t = torch.as_tensor(np.asarray(x), dtype=torch.float64).to(device=device, dtype=dtype)
    return t.requires_grad_(requires_grad)


def _round(x, dtype):
    """The values a `dtype` tensor holds, as float64 (the oracle consumes exactly these)."""
    return torch.as_tensor(np.asarray(x), dtype=torch.float64).to(dtype).double().numpy()


def _inputs(B, N, seed, anchors, dtype=torch.float64):
    d = o.synthetic_inputs(B, N, seed, anchors=anchors)
    return {k: _round(v, dtype) for k, v in d.items()}


def _anchor_tensors(d, dtype, device):
    if "p0" not in d:
        return {}
    return {k: _dev(d[k], dtype, device) for k in ("p0", "first_direction", "initial_normal")}


def _anchor_np(d):
    return {k: d.get(k) for k in ("p0", "first_direction", "initial_normal")}


def _run(cufk, d, dtype, device, grad=True):
    L = _dev(d["lengths"], dtype, device, grad)
    A = _dev(d["angles"], dtype, device, grad)
    D = _dev(d["dihedrals"], dtype, device, grad)
    xyz = cufk.reconstruct(L, A, D, **_anchor_tensors(d, dtype, device))
    if not grad:
        return xyz, None
    g = _dev(d["grad"], dtype, device)
    grads = torch.autograd.grad(xyz, (L, A, D), g)
    return xyz, grads


# ----------------------------------------------------------------- forward


@pytest.mark.parametrize("N", [4, 5, 6, 37, 64, 259, 260, 515, 516, 1027, 1028, 2051])
@pytest.mark.parametrize("anchors", [False, True])
def test_forward_fp64_matches_oracle(cufk, device, N, anchors):
    d = _inputs(3, N, seed=N, anchors=anchors)
    xyz, _ = _run(cufk, d, torch.float64, device, grad=False)
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    got = xyz.cpu().numpy()
    err = np.abs(got - ref).max()
    print(f"fp64 forward N={N} anchors={anchors}: max err {err:.3e}")
    assert err <= 1e-12 * max(1.0, np.abs(ref).max())


def test_forward_fp32_tolerance_at_cap(cufk, device):
    # Config 2 shape per chain (N = 2049) with explicit random anchors; 32 chains.
    d = _inputs(32, 2049, seed=2, anchors=True, dtype=torch.float32)
    xyz, _ = _run(cufk, d, torch.float32, device, grad=False)
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    diff = xyz.double().cpu().numpy() - ref
    rms = math.sqrt(np.mean(np.sum(diff**2, axis=-1)))
    mx = np.abs(diff).max()
    print(f"fp32 forward N=2049: rms {rms:.3e} nm, max {mx:.3e} nm")
    assert rms <= 1e-5
    assert mx <= 1e-4


def test_forward_golden_fixture(cufk, device, golden_c0):
    g = golden_c0
    for dtype, tol in ((torch.float64, 1e-13), (torch.float32, 2e-6)):
        L = _dev(g["lengths"], dtype, device)
        A = _dev(g["angles"], dtype, device)
        D = _dev(g["dihedrals"], dtype, device)
        xyz = cufk.reconstruct(L, A, D)
        assert xyz.shape == g["xyz"].shape
        err = np.abs(xyz.double().cpu().numpy() - g["xyz"]).max()
        print(f"golden C0 {dtype}: max err {err:.3e}")
        assert err <= tol


def test_single_chain_shapes(cufk, device):
    d = _inputs(1, 20, seed=5, anchors=False)
    L = _dev(d["lengths"][0], torch.float32, device, True)
    A = _dev(d["angles"][0], torch.float32, device, True)
    D = _dev(d["dihedrals"][0], torch.float32, device, True)
    xyz = cufk.reconstruct(L, A, D)
    assert xyz.shape == (20, 3) and xyz.dtype == torch.float32
    gl, ga, gd = torch.autograd.grad(xyz, (L, A, D), torch.ones_like(xyz))
    assert gl.shape == (19,) and ga.shape == (18,) and gd.shape == (17,)


def test_noncontiguous_inputs(cufk, device):
    d = _inputs(4, 50, seed=9, anchors=False)
    wide = {k: np.concatenate([d[k], d[k]], axis=1) for k in ("lengths", "angles", "dihedrals")}
    L = _dev(wide["lengths"], torch.float64, device)[:, : d["lengths"].shape[1]]
    A = _dev(wide["angles"], torch.float64, device)[:, : d["angles"].shape[1]]
    D = _dev(wide["dihedrals"], torch.float64, device)[:, : d["dihedrals"].shape[1]]
    assert not L.is_contiguous()
    xyz = cufk.reconstruct(L, A, D)
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"])
    assert np.abs(xyz.cpu().numpy() - ref).max() <= 1e-12


def test_empty_batch(cufk, device):
    L = torch.zeros(0, 9, device=device)
    xyz = cufk.reconstruct(L, torch.zeros(0, 8, device=device), torch.zeros(0, 7, device=device))
    assert xyz.shape == (0, 10, 3)


def _empty_rows(N, dtype, device):
    return [torch.zeros(0, N - k, device=device, dtype=dtype, requires_grad=True) for k in (1, 2, 3)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
@pytest.mark.parametrize("kind", ["reconstruct", "anchor_grads", "long", "loss", "rmsd"])
def test_empty_batch_every_entry_point(cufk, device, dtype, kind):
    """B = 0 through every reconstruct entry point, forward and backward: empty outputs and
    gradients of the inputs' shapes (anchor gradients zero), no launch of an empty grid."""
    N = 40
    L, A, D = _empty_rows(N, dtype, device)
    an = [torch.tensor(v, device=device, dtype=dtype, requires_grad=kind == "anchor_grads")
          for v in ((0.1, 0.2, 0.3), (1.0, 0.0, 0.0), (0.0, 1.0, 0.0))]
    target = torch.zeros(0, N, 3, device=device, dtype=dtype)
    if kind == "reconstruct":
        out = cufk.reconstruct(L, A, D, *an)
    elif kind == "anchor_grads":
        out = cufk.reconstruct(L, A, D, *an, anchor_grads=True)
    elif kind == "long":
        out = cufk.reconstruct_long(L, A, D, *an, segment_steps=16)
    elif kind == "loss":
        out = cufk.reconstruct_loss(L, A, D, target, *an)
    else:
        out = cufk.reconstruct_rmsd(L, A, D, target, *an)
    assert out.shape == ((0, N, 3) if kind in ("reconstruct", "anchor_grads", "long") else (0,))
    inputs = (L, A, D, *an) if kind == "anchor_grads" else (L, A, D)
    grads = torch.autograd.grad(out, inputs, torch.zeros_like(out))
    for g, x in zip(grads, inputs):
        assert g.shape == x.shape
    if kind == "anchor_grads":
        assert all(bool((g == 0).all()) for g in grads[3:])
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
def test_partial_requires_grad_and_no_grad_mode(cufk, device, dtype):
    """Every subset of (lengths, angles, dihedrals) requiring grad gets the gradients of the
    full run, bit for bit; the others get none.  Under torch.no_grad (and with no input
    requiring grad) the output needs no graph and equals the autograd forward's bit for bit
    (the flagged and plain forwards place points with the same arithmetic)."""
    d = _inputs(5, 300, seed=41, anchors=True, dtype=dtype)
    xyz_full, full = _run(cufk, d, dtype, device)
    an = _anchor_tensors(d, dtype, device)
    g = _dev(d["grad"], dtype, device)
    for mask in range(1, 8):
        wants = [bool(mask >> k & 1) for k in range(3)]
        L, A, D = (_dev(d[k], dtype, device, w) for k, w in zip(("lengths", "angles", "dihedrals"), wants))
        xyz = cufk.reconstruct(L, A, D, **an)
        picked = [t for t, w in zip((L, A, D), wants) if w]
        grads = torch.autograd.grad(xyz, picked, g)
        for got, want in zip(grads, [f for f, w in zip(full, wants) if w]):
            assert torch.equal(got, want), mask
    with torch.no_grad():
        L, A, D = (_dev(d[k], dtype, device, True) for k in ("lengths", "angles", "dihedrals"))
        plain = cufk.reconstruct(L, A, D, **an)
    assert not plain.requires_grad and torch.equal(plain, xyz_full.detach())
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    plain = cufk.reconstruct(L, A, D, **an)
    assert not plain.requires_grad and torch.equal(plain, xyz_full.detach())


@pytest.mark.parametrize("kind", ["apply", "loss", "rmsd"])
def test_empty_batch_torsion(cufk, device, kind):
    f = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    N = 40
    raw = torch.zeros(0, 2 * (N - 3), device=device, requires_grad=True)
    target = torch.zeros(0, N, 3, device=device)
    out = f(raw) if kind == "apply" else (f.loss(raw, target) if kind == "loss" else f.rmsd(raw, target))
    assert out.shape == ((0, N, 3) if kind == "apply" else (0,))
    (g,) = torch.autograd.grad(out, (raw,), torch.zeros_like(out))
    assert g.shape == raw.shape
    torch.cuda.synchronize()


# ----------------------------------------------------------------- backward


@pytest.mark.parametrize("N", [4, 5, 9, 64, 259, 515, 1028, 2051])
def test_backward_fp64_matches_oracle(cufk, device, N):
    d = _inputs(2, N, seed=100 + N, anchors=True)
    _, grads = _run(cufk, d, torch.float64, device)
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for name, got, want in zip(("lengths", "angles", "dihedrals"), grads, ref):
        err = np.abs(got.cpu().numpy() - want).max()
        scale = max(1.0, np.abs(want).max())
        print(f"fp64 backward N={N} d/d{name}: max err {err:.3e} (scale {scale:.3e})")
        assert err <= 1e-9 * scale


def test_backward_degenerate_geometry_fp64(cufk, device):
    # Negative lengths, angles outside (0, pi) and a first direction parallel to the normal:
    # the exact-frame adjoint has no sign or degeneracy cases.
    d = _inputs(2, 30, seed=11, anchors=False)
    d["lengths"][:, 3] *= -1.0
    d["angles"][:, 0] = -0.7
    d["angles"][:, 5] = 3.5
    d["p0"] = np.array([0.3, -0.2, 0.1])
    d["first_direction"] = np.array([0.0, 0.0, 2.0])
    d["initial_normal"] = np.array([0.0, 0.0, 1.0])
    xyz, grads = _run(cufk, d, torch.float64, device)
    ref_x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    assert np.abs(xyz.detach().cpu().numpy() - ref_x).max() <= 1e-12
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for got, want in zip(grads, ref):
        assert np.abs(got.cpu().numpy() - want).max() <= 1e-9 * max(1.0, np.abs(want).max())


def test_gradcheck_fp64(cufk, device):
    d = _inputs(2, 12, seed=3, anchors=True)
    L = _dev(d["lengths"], torch.float64, device, True)
    A = _dev(d["angles"], torch.float64, device, True)
    D = _dev(d["dihedrals"], torch.float64, device, True)
    an = _anchor_tensors(d, torch.float64, device)
    assert torch.autograd.gradcheck(lambda a, b, c: cufk.reconstruct(a, b, c, **an), (L, A, D), eps=1e-6, atol=1e-7)


@pytest.mark.parametrize("N", [384, 2049])
def test_backward_fp32_tolerance(cufk, device, N):
    d = _inputs(8, N, seed=N, anchors=True, dtype=torch.float32)
    _, grads = _run(cufk, d, torch.float32, device)
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for name, got, want in zip(("lengths", "angles", "dihedrals"), grads, ref):
        err = np.abs(got.double().cpu().numpy() - want).max()
        scale = np.abs(want).max()
        print(f"fp32 backward N={N} d/d{name}: max err {err:.3e}, rel {err / scale:.3e}")
        assert err <= 5e-5 * scale


# ----------------------------------------------------------------- torsion


@pytest.mark.parametrize("N", [4, 5, 6, 7, 100, 195, 196, 387, 388, 771, 772, 1539, 1540, 2051])
def test_torsion_fp64_matches_oracle(cufk, device, N):
    rng = np.random.default_rng(N)
    B = 3
    raw = rng.normal(size=(B, 2 * (N - 3)))
    g = rng.normal(size=(B, N, 3))
    f = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    consts = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    r = _dev(raw, torch.float64, device, True)
    xyz = f(r)
    ref = o.torsion_forward(raw, consts)
    err = np.abs(xyz.detach().cpu().numpy() - ref).max()
    (graw,) = torch.autograd.grad(xyz, (r,), _dev(g, torch.float64, device))
    ref_g = o.torsion_backward(raw, ref, g, consts)
    gerr = np.abs(graw.cpu().numpy() - ref_g).max()
    print(f"torsion fp64 N={N}: xyz err {err:.3e}, grad err {gerr:.3e}")
    assert err <= 1e-12 * max(1.0, np.abs(ref).max())
    assert gerr <= 1e-9 * max(1.0, np.abs(ref_g).max())


def test_torsion_matches_reconstruct_fp64(cufk, device):
    rng = np.random.default_rng(0)
    B, N = 2, 301
    raw = rng.normal(size=(B, 2 * (N - 3)))
    consts = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    xyz_t = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)(_dev(raw, torch.float64, device))
    Sn, Cn, _ = o._normalize_pairs(raw)
    L = np.array([consts.lengths[i % 3] for i in range(N - 1)])[None].repeat(B, 0)
    A = np.array([math.atan2(consts.sin[i % 3], consts.cos[i % 3]) for i in range(N - 2)])[None].repeat(B, 0)
    xyz_r = cufk.reconstruct(_dev(L, torch.float64, device), _dev(A, torch.float64, device), _dev(np.arctan2(Sn, Cn), torch.float64, device))
    assert torch.allclose(xyz_t, xyz_r, atol=1e-12, rtol=0)


def test_torsion_fp32_tolerance(cufk, device):
    rng = np.random.default_rng(771)
    B, N = 16, 771
    raw = _round(rng.normal(size=(B, 2 * (N - 3))), torch.float32)
    g = _round(rng.normal(size=(B, N, 3)), torch.float32)
    consts = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    f = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    r = _dev(raw, torch.float32, device, True)
    xyz = f(r)
    (graw,) = torch.autograd.grad(xyz, (r,), _dev(g, torch.float32, device))
    ref = o.torsion_forward(raw, consts)
    diff = xyz.detach().double().cpu().numpy() - ref
    rms = math.sqrt(np.mean(np.sum(diff**2, -1)))
    ref_g = o.torsion_backward(raw, ref, g, consts)
    gerr = np.abs(graw.double().cpu().numpy() - ref_g).max() / np.abs(ref_g).max()
    print(f"torsion fp32 N={N}: rms {rms:.3e}, max {np.abs(diff).max():.3e}, grad rel {gerr:.3e}")
    assert rms <= 1e-5 and np.abs(diff).max() <= 1e-4
    assert gerr <= 5e-5


@pytest.mark.parametrize("N", [4, 5, 100, 195, 196, 388, 772, 1540, 2051])
def test_torsion_fp32_gradients_across_plans(cufk, device, N):
    """fp32 raw-pair gradients at every backward plan size (3 steps per lane, 1-11 waves)."""
    rng = np.random.default_rng(900 + N)
    B = 3
    raw = _round(rng.normal(size=(B, 2 * (N - 3))), torch.float32)
    g = _round(rng.normal(size=(B, N, 3)), torch.float32)
    consts = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    r = _dev(raw, torch.float32, device, True)
    xyz = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)(r)
    (graw,) = torch.autograd.grad(xyz, (r,), _dev(g, torch.float32, device))
    ref_g = o.torsion_backward(raw, o.torsion_forward(raw, consts), g, consts)
    gerr = np.abs(graw.double().cpu().numpy() - ref_g).max() / np.abs(ref_g).max()
    print(f"torsion fp32 N={N}: grad rel {gerr:.3e}")
    assert gerr <= 5e-5


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_torsion_low_precision_reported(cufk, device, dtype):
    """Half-precision torsion: computed in float from the rounded inputs; errors against the
    float64 oracle on the same inputs are reported, with only a loose sanity bound.  The
    backward works from the saved half-precision positions (as the reference's does), whose
    rounding (about 0.02 nm at chain scale in bfloat16) dominates the gradient error."""
    rng = np.random.default_rng(31)
    B, N = 4, 300
    raw = _round(rng.normal(size=(B, 2 * (N - 3))), dtype)
    g = _round(rng.normal(size=(B, N, 3)), dtype)
    consts = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    r = _dev(raw, dtype, device, True)
    xyz = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)(r)
    (graw,) = torch.autograd.grad(xyz, (r,), _dev(g, dtype, device))
    ref = o.torsion_forward(raw, consts)
    ref_g = o.torsion_backward(raw, ref, g, consts)
    err = np.abs(xyz.detach().double().cpu().numpy() - ref).max() / np.abs(ref).max()
    gerr = np.abs(graw.double().cpu().numpy() - ref_g).max() / np.abs(ref_g).max()
    print(f"torsion {dtype} N={N}: xyz rel {err:.3e}, grad rel {gerr:.3e}")
    assert torch.isfinite(xyz).all() and torch.isfinite(graw).all()
    assert err <= 5e-2 and gerr <= 0.5


def test_torsion_strided_rows_keep_grad_strides(cufk, device):
    rng = np.random.default_rng(5)
    B, N = 4, 40
    wide = rng.normal(size=(B, 2 * (N - 3) + 6))
    base = _dev(wide, torch.float64, device)
    raw = base[:, 2 : 2 + 2 * (N - 3)].detach().requires_grad_(False)
    raw = base[:, 2 : 2 + 2 * (N - 3)]
    assert raw.stride(0) == wide.shape[1] and not raw.is_contiguous()
    leaf = raw.detach().clone().requires_grad_(True)
    f = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    consts = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    xyz = f(raw.detach())  # strided, no grad
    ref = o.torsion_forward(wide[:, 2 : 2 + 2 * (N - 3)], consts)
    assert np.abs(xyz.cpu().numpy() - ref).max() <= 1e-12
    # Gradient of a strided input: autograd hands back the kernel's stride-preserving tensor.
    strided = base.detach().clone()[:, 2 : 2 + 2 * (N - 3)].requires_grad_(True)
    out = f(strided)
    g = rng.normal(size=(B, N, 3))
    (gr,) = torch.autograd.grad(out, (strided,), _dev(g, torch.float64, device))
    ref_g = o.torsion_backward(wide[:, 2 : 2 + 2 * (N - 3)], ref, g, consts)
    assert np.abs(gr.cpu().numpy() - ref_g).max() <= 1e-9 * np.abs(ref_g).max()
    del leaf


def test_torsion_overlapping_rows_get_a_dense_gradient(cufk, device):
    """Raw rows that overlap (row stride shorter than the row, as an as_strided or unfold view
    gives) are read as they lie; their gradient cannot keep that layout (its rows would
    overlap), so it comes back dense, each row the gradient of its own chain."""
    rng = np.random.default_rng(6)
    B, N = 5, 40
    K = 2 * (N - 3)
    flat = torch.as_tensor(rng.normal(size=K + 6 * (B - 1)), dtype=torch.float64, device=device)
    raw = flat.as_strided((B, K), (6, 1))
    assert raw.stride(0) < K
    leaf = raw.detach().clone().requires_grad_(True)  # the same values, dense rows
    f = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    g = _dev(rng.normal(size=(B, N, 3)), torch.float64, device)
    view = flat.clone().requires_grad_(True)
    out = f(view.as_strided((B, K), (6, 1)))
    (gv,) = torch.autograd.grad(out, (view,), g, retain_graph=True)
    want_x = f(leaf)
    (want_g,) = torch.autograd.grad(want_x, (leaf,), g)
    assert torch.equal(out, want_x)
    # Autograd sums the rows' gradients back into the flat storage they share.
    summed = torch.zeros_like(flat)
    for b in range(B):
        summed[6 * b : 6 * b + K] += want_g[b]
    assert torch.allclose(gv, summed, rtol=0, atol=1e-12)


def test_max_steps_on_the_device(device):
    from cufk_amd._native import _C

    for dtype in range(4):
        for direction in range(2):
            assert _C.max_steps(dtype, direction, 0) == 2048
    assert _C.max_steps(0, 0, torch.cuda.device_count()) == -8


# ----------------------------------------------------------------- low precision (reported)


@pytest.mark.parametrize("N", [40, 300, 1026, 2051])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_low_precision_reported(cufk, device, dtype, N):
    """Half types compute in float from the rounded inputs; errors against the float64 oracle
    on the same inputs are reported and held to sanity bounds about 10x the observed errors
    of the type's rounding (bf16 at N=1026: 1.5e-3 forward, 3e-3 gradients), far below what a
    misplaced or garbled element produces (order 1).  The sizes cover every scan plan; rows of
    odd length start at every alignment within a 16-byte block."""
    d = _inputs(8, N, seed=4, anchors=False, dtype=dtype)
    xyz, grads = _run(cufk, d, dtype, device)
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"])
    diff = xyz.detach().double().cpu().numpy() - ref
    err_pos = np.sqrt(np.mean(np.sum(diff**2, -1), axis=0))
    rel = np.abs(diff).max() / np.abs(ref).max()
    print(f"{dtype} forward N={N}: rms {math.sqrt(np.mean(err_pos**2)):.3e}, max {np.abs(diff).max():.3e}, "
          f"rel max {rel:.2e}, rms at the last position {err_pos[-1]:.2e}")
    marks = sorted({round(i * (N - 1) / 10) for i in range(11)})
    print(f"{dtype} forward N={N}: rms by position " + ", ".join(f"{i}: {err_pos[i]:.1e}" for i in marks))
    ref_g = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"])
    gerr = [float(np.abs(gr.double().cpu().numpy() - rg).max() / np.abs(rg).max()) for gr, rg in zip(grads, ref_g)]
    print(f"{dtype} backward N={N}: rel max err (lengths, angles, dihedrals) " + ", ".join(f"{e:.2e}" for e in gerr))
    assert torch.isfinite(xyz).all()
    for gr in grads:
        assert torch.isfinite(gr).all()
    assert rel <= 1e-2
    assert max(gerr) <= 3e-2


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N", [301, 1100])
@pytest.mark.parametrize("shift", range(1, 8))
def test_low_precision_unaligned_storage(dtype, N, shift, device):
    """float16/bfloat16 rows move in 8- or 4-element windows at the rows' own 2-byte alignment.
    Every input and output here is a view `shift` elements into a buffer (storage 2*shift bytes
    past a 16-byte boundary), through the C ABI: the forward, the exact backward and the shadow
    forward and backward equal those of the same values in fresh, aligned buffers, bit for bit.
    N = 301 runs 4-step lanes (4-element windows), N = 1100 8-step lanes (8-element windows);
    both leave rows that end past their last whole window."""
    lib = _abi()
    B = 5
    d = _inputs(B, N, seed=41 + shift, anchors=True, dtype=dtype)
    an = _anchors3(d, dtype, device)
    aligned = lambda t, s: t  # noqa: E731

    def shifted(t, s):
        buf = torch.full((t.numel() + 8,), float("nan"), dtype=t.dtype, device=device)
        v = buf[s : s + t.numel()].view(t.shape)
        v.copy_(t)
        assert v.data_ptr() % 16 == (s * t.element_size()) % 16
        return v

    outs = []
    for make in (aligned, shifted):
        L, A, D, g = (make(_dev(d[k], dtype, device), shift) for k in ("lengths", "angles", "dihedrals", "grad"))
        blank = lambda t: make(torch.full_like(t, float("nan")), shift)  # noqa: E731
        xyz, xyz2 = blank(g), blank(g)
        gL, gA, gD, sL, sA, sD = (blank(t) for t in (L, A, D, L, A, D))
        pos = torch.empty(B, N, 3, dtype=torch.float32, device=device)
        reg = torch.empty(B, dtype=torch.uint8, device=device)
        p = lambda t: t.data_ptr()  # noqa: E731
        code, st = _CODES[dtype], torch.cuda.current_stream().cuda_stream
        assert lib.cufk_reconstruct_fwd(code, p(L), p(A), p(D), *map(p, an), p(xyz), B, N, st) == 0
        assert lib.cufk_reconstruct_bwd(code, p(L), p(A), p(D), *map(p, an), p(g), p(gL), p(gA), p(gD), B, N, st) == 0
        assert lib.cufk_reconstruct_fwd_shadow(code, p(L), p(A), p(D), *map(p, an), p(xyz2), p(pos), p(reg), B, N,
                                               st) == 0
        assert lib.cufk_reconstruct_bwd_shadow(code, p(L), p(A), p(D), *map(p, an), p(pos), p(reg), p(g), p(sL), p(sA),
                                               p(sD), B, N, st) == 0
        torch.cuda.synchronize()
        outs.append([t.clone() for t in (xyz, gL, gA, gD, xyz2, pos, reg, sL, sA, sD)])
    assert torch.equal(outs[0][0], outs[0][4])  # the shadow forward's xyz is the plain forward's
    assert bool(outs[0][6].all())  # every chain here takes the position-based backward
    for a, b in zip(*outs):
        assert not a.is_floating_point() or torch.isfinite(a).all()
        assert torch.equal(a, b)


# ----------------------------------------------------------------- runtime behaviour


def test_deterministic_and_stream(cufk, device):
    d = _inputs(64, 700, seed=8, anchors=True, dtype=torch.float32)
    x1, g1 = _run(cufk, d, torch.float32, device)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        x2, g2 = _run(cufk, d, torch.float32, device)
    s.synchronize()
    assert torch.equal(x1, x2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_concurrent_streams(cufk, device):
    """Four different workloads enqueued on four streams with no synchronisation between them
    (reconstruct with default anchors, torsion, long chains, the fused RMSD), forward and
    backward, three times over: each equals its sequential result bit for bit.  The library
    holds no state between calls that they could share, beyond read-only defaults."""
    head = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    rng = np.random.default_rng(19)
    d1 = _inputs(32, 900, seed=91, anchors=False, dtype=torch.float32)
    d2 = _inputs(8, 5000, seed=92, anchors=True, dtype=torch.float32)
    d3 = _inputs(48, 700, seed=93, anchors=True, dtype=torch.float32)
    raw = torch.as_tensor(rng.normal(size=(64, 2 * 400)), dtype=torch.float32, device=device)
    graw = torch.as_tensor(rng.normal(size=(64, 403, 3)), dtype=torch.float32, device=device)
    target = _dev(d3["grad"], torch.float32, device)

    def rows(d):
        return [_dev(d[k], torch.float32, device, True) for k in ("lengths", "angles", "dihedrals")]

    def w1():
        L, A, D = rows(d1)
        x = cufk.reconstruct(L, A, D)
        return (x, *torch.autograd.grad(x, (L, A, D), _dev(d1["grad"], torch.float32, device)))

    def w2():
        r = raw.clone().requires_grad_(True)
        x = head(r)
        return (x, *torch.autograd.grad(x, (r,), graw))

    def w3():
        L, A, D = rows(d2)
        x = cufk.reconstruct_long(L, A, D, **_anchor_tensors(d2, torch.float32, device), segment_steps=700)
        return (x, *torch.autograd.grad(x, (L, A, D), _dev(d2["grad"], torch.float32, device)))

    def w4():
        L, A, D = rows(d3)
        loss = cufk.reconstruct_rmsd(L, A, D, target, **_anchor_tensors(d3, torch.float32, device))
        return (loss, *torch.autograd.grad(loss.sum(), (L, A, D)))

    work = (w1, w2, w3, w4)
    want = [w() for w in work]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in work]
    for rep in range(3):
        got = []
        for s, w in zip(streams, work):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                got.append(w())
        torch.cuda.synchronize()
        for i, (g, ww) in enumerate(zip(got, want)):
            for a, b in zip(g, ww):
                assert torch.equal(a, b), (rep, i)


def test_full_size_config2_sampled(cufk, device):
    # B = 4096, N = 2049 fp32: compare 6 sampled chains with the float64 oracle.
    B, N = 4096, 2049
    d = _inputs(B, N, seed=2, anchors=True, dtype=torch.float32)
    xyz, grads = _run(cufk, d, torch.float32, device)
    torch.cuda.synchronize()
    idx = [0, 1, 1000, 2047, 4000, 4095]
    sub = {k: (v[idx] if k in ("lengths", "angles", "dihedrals", "grad") else v) for k, v in d.items()}
    ref = o.reconstruct_forward(sub["lengths"], sub["angles"], sub["dihedrals"], **_anchor_np(sub))
    diff = xyz.detach()[idx].double().cpu().numpy() - ref
    rms = math.sqrt(np.mean(np.sum(diff**2, -1)))
    assert rms <= 1e-5 and np.abs(diff).max() <= 1e-4
    ref_g = o.reconstruct_backward(sub["lengths"], sub["angles"], sub["dihedrals"], sub["grad"], **_anchor_np(sub))
    for got, want in zip(grads, ref_g):
        assert np.abs(got[idx].double().cpu().numpy() - want).max() <= 5e-5 * np.abs(want).max()


# ----------------------------------------------------------------- the two backward paths


def _abi():
    import ctypes

    import cufk_amd

    lib = ctypes.CDLL(str(cufk_amd._native.HIP_LIBRARY))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.cufk_reconstruct_fwd.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, i64, i64, vp]
    lib.cufk_reconstruct_fwd_flagged.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, vp]
    lib.cufk_reconstruct_bwd.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, vp]
    lib.cufk_reconstruct_bwd_saved.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, vp]
    lib.cufk_reconstruct_shadow_floats.argtypes = [i64, i64]
    lib.cufk_reconstruct_shadow_floats.restype = i64
    lib.cufk_reconstruct_fwd_shadow.argtypes = [ctypes.c_int] + [vp] * 9 + [i64, i64, vp]
    lib.cufk_reconstruct_bwd_shadow.argtypes = [ctypes.c_int] + [vp] * 12 + [i64, i64, vp]
    return lib


_CODES = {torch.float32: 0, torch.float64: 1, torch.float16: 2, torch.bfloat16: 3}


def _flagged_forward(lib, L, A, D, an):
    B, N = L.shape[0], L.shape[1] + 1
    xyz = torch.empty(B, N, 3, device=L.device, dtype=L.dtype)
    reg = torch.full((B,), 7, device=L.device, dtype=torch.uint8)
    p = lambda t: t.data_ptr()  # noqa: E731
    rc = lib.cufk_reconstruct_fwd_flagged(_CODES[L.dtype], p(L), p(A), p(D), p(an[0]), p(an[1]), p(an[2]), p(xyz), p(reg),
                                          B, N, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return xyz, reg


def _anchors3(d, dtype, device):
    if "p0" in d:
        return tuple(_dev(d[k], dtype, device) for k in ("p0", "first_direction", "initial_normal"))
    return (_dev([0.0, 0, 0], dtype, device), _dev([1.0, 0, 0], dtype, device), _dev([0.0, 0, 1], dtype, device))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16, torch.bfloat16])
def test_regularity_flags(cufk, device, dtype):
    lib = _abi()
    d = _inputs(6, 300, seed=21, anchors=True, dtype=dtype)
    d["lengths"][1, 7] = -d["lengths"][1, 7]  # negative bond
    small = 0.2 if dtype != torch.float64 else 0.005  # below the fast-path sine threshold
    d["angles"][2, 40] = small
    d["angles"][3, 0] = math.pi - small  # first-frame angle
    d["lengths"][4, 1] = 0.0  # zero bond
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    xyz, reg = _flagged_forward(lib, L, A, D, _anchors3(d, dtype, device))
    flags = reg.cpu().tolist()
    if dtype in (torch.float16, torch.bfloat16):
        assert flags == [0] * 6
    else:
        assert flags == [1, 0, 0, 0, 0, 1]
    ref = cufk.reconstruct(L, A, D, *_anchor_tensors(d, dtype, device).values())
    assert torch.equal(xyz, ref)


def _abi_fused():
    import ctypes

    lib = _abi()
    vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.cufk_reconstruct_loss_fwd.argtypes = [ci] + [vp] * 10 + [i64, i64, vp]
    lib.cufk_reconstruct_superposed_fwd.argtypes = [ci, ci] + [vp] * 11 + [i64, i64, vp]
    lib.cufk_torsion_fwd.argtypes = [ci, vp, i64, vp, vp, i64, i64, vp]
    lib.cufk_torsion_loss_fwd.argtypes = [ci, ci, vp, i64, vp, vp, vp, vp, vp, i64, i64, vp]
    return lib


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
@pytest.mark.parametrize("B,N", [(40, 300), (9, 2049), (4100, 64)])
def test_fused_forwards_store_the_flagged_forwards_positions(device, dtype, B, N):
    """The fused-loss forwards (squared distance, superposed) write xyz and the regularity flags
    as cufk_reconstruct_fwd_flagged does: bit for bit where that entry point runs one chain per
    workgroup, within float rounding where it packs short chains (at least 4096 chains of at most
    131 points; the fused forwards never pack).  The shadow forward's xyz is the plain forward's
    bit for bit wherever it keeps a float copy.  The full-size fused-loss tests hold the fused
    gradients to the adjoint over the plain forward's positions, so they rely on this."""
    lib = _abi_fused()
    code = _CODES[dtype]
    st = torch.cuda.current_stream().cuda_stream
    p = lambda t: t.data_ptr()  # noqa: E731
    d = _inputs(B, N, seed=N + B, anchors=True, dtype=dtype)
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    an = _anchors3(d, dtype, device)
    xyz, reg = _flagged_forward(lib, L, A, D, an)
    target = (xyz.double() + 0.3 * torch.randn(B, N, 3, device=device, dtype=torch.float64)).to(dtype)
    packed = B >= 4096 and N - 3 <= 128
    scale = max(1.0, float(xyz.double().abs().max()))
    tol = {torch.float32: 2e-6, torch.float64: 1e-12, torch.bfloat16: 2.0**-7}[dtype] * scale

    def same(got, got_reg, what):
        if packed:
            err = float((got.double() - xyz.double()).abs().max())
            assert err <= tol, (what, err, tol)
        else:
            assert torch.equal(got, xyz), what
        assert torch.equal(got_reg, reg), what

    fused = [("squared distance", None)] + [(f"superposed kind {k}", k) for k in (1, 2)]
    for what, kind in fused:
        x2 = torch.empty_like(xyz)
        r2 = torch.full((B,), 7, device=device, dtype=torch.uint8)
        loss = torch.empty(B, device=device, dtype=dtype)
        if kind is None:
            rc = lib.cufk_reconstruct_loss_fwd(code, p(L), p(A), p(D), *(p(t) for t in an), p(target), p(x2), p(r2),
                                               p(loss), B, N, st)
        else:
            rec = torch.empty(B, 24, device=device, dtype=torch.float64)
            rc = lib.cufk_reconstruct_superposed_fwd(code, kind, p(L), p(A), p(D), *(p(t) for t in an), p(target),
                                                     p(x2), p(r2), p(loss), p(rec), B, N, st)
        assert rc == 0, what
        same(x2, r2, what)
    if dtype == torch.bfloat16 and lib.cufk_reconstruct_shadow_floats(B, N) > 0:
        x3 = torch.empty_like(xyz)
        pos = torch.empty(B, N, 3, device=device, dtype=torch.float32)
        r3 = torch.full((B,), 7, device=device, dtype=torch.uint8)
        assert lib.cufk_reconstruct_fwd_shadow(code, p(L), p(A), p(D), *(p(t) for t in an), p(x3), p(pos), p(r3),
                                               B, N, st) == 0
        assert torch.equal(x3, xyz)
        # The float copy rounds to the stored output.
        assert torch.equal(pos.to(dtype), xyz)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N", [300, 1100])
@pytest.mark.parametrize("shift", [0, 1, 3, 6])
def test_torsion_low_precision_is_the_rounded_float32_forward(device, dtype, N, shift):
    """The float16/bfloat16 torsion forward computes in float from the widened pairs, so its
    output is the float32 forward's on the same values, rounded once, bit for bit.  Pairs and
    output here are views `shift` elements into their buffers: the point rows (12-step lanes)
    move in 4-element windows at the rows' own 2-byte alignment, the pairs element by element.
    N = 300 runs one wave per chain, N = 1100 two."""
    import ctypes

    class Consts(ctypes.Structure):
        _fields_ = [("length", ctypes.c_float * 3), ("sin", ctypes.c_double * 3), ("cos", ctypes.c_double * 3)]

    lib = _abi_fused()
    st = torch.cuda.current_stream().cuda_stream
    p = lambda t: t.data_ptr()  # noqa: E731
    c = Consts((ctypes.c_float * 3)(*BOND_LENGTHS), (ctypes.c_double * 3)(*(math.sin(a) for a in BOND_ANGLES)),
               (ctypes.c_double * 3)(*(math.cos(a) for a in BOND_ANGLES)))
    B = 7
    gen = torch.Generator(device=device).manual_seed(N + shift)
    raw = torch.randn(B, 2 * (N - 3), generator=gen, device=device).to(dtype)

    def view(shape, dt, fill):
        n = math.prod(shape)
        buf = torch.full((n + 8,), fill, dtype=dt, device=device)
        return buf[shift : shift + n].view(shape)

    raw_h = view(raw.shape, dtype, 0.0)
    raw_h.copy_(raw)
    xyz_h = view((B, N, 3), dtype, float("nan"))
    xyz_f = torch.full((B, N, 3), float("nan"), device=device)
    raw_f = raw.float()
    assert lib.cufk_torsion_fwd(_CODES[dtype], p(raw_h), raw_h.stride(0), ctypes.byref(c), p(xyz_h), B, N, st) == 0
    assert lib.cufk_torsion_fwd(0, p(raw_f), raw_f.stride(0), ctypes.byref(c), p(xyz_f), B, N, st) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(xyz_f).all()
    assert torch.equal(xyz_h, xyz_f.to(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
@pytest.mark.parametrize("N", [300, 771])
def test_torsion_loss_forward_stores_the_torsion_forwards_positions(device, dtype, N):
    """cufk_torsion_loss_fwd writes xyz bit for bit as cufk_torsion_fwd does (both kinds)."""
    import ctypes

    class Consts(ctypes.Structure):
        _fields_ = [("length", ctypes.c_float * 3), ("sin", ctypes.c_double * 3), ("cos", ctypes.c_double * 3)]

    lib = _abi_fused()
    code = _CODES[dtype]
    st = torch.cuda.current_stream().cuda_stream
    p = lambda t: t.data_ptr()  # noqa: E731
    c = Consts((ctypes.c_float * 3)(*BOND_LENGTHS), (ctypes.c_double * 3)(*(math.sin(a) for a in BOND_ANGLES)),
               (ctypes.c_double * 3)(*(math.cos(a) for a in BOND_ANGLES)))
    B = 40
    gen = torch.Generator(device=device).manual_seed(N)
    raw = torch.randn(B, 2 * (N - 3), generator=gen, device=device).to(dtype)
    xyz = torch.empty(B, N, 3, device=device, dtype=dtype)
    assert lib.cufk_torsion_fwd(code, p(raw), raw.stride(0), ctypes.byref(c), p(xyz), B, N, st) == 0
    target = (xyz.double() + 0.3 * torch.randn(B, N, 3, device=device, dtype=torch.float64, generator=gen)).to(dtype)
    for kind in (0, 1):
        x2 = torch.empty_like(xyz)
        loss = torch.empty(B, device=device, dtype=dtype)
        rec = torch.empty(B, 24, device=device, dtype=torch.float64)
        assert lib.cufk_torsion_loss_fwd(code, kind, p(raw), raw.stride(0), ctypes.byref(c), p(target), p(x2), p(loss),
                                         p(rec), B, N, st) == 0
        assert torch.equal(x2, xyz), kind


def test_far_chain_is_not_regular_in_fp32(cufk, device):
    lib = _abi()
    d = _inputs(2, 50, seed=22, anchors=True, dtype=torch.float32)
    an = list(_anchors3(d, torch.float32, device))
    L, A, D = (_dev(d[k], torch.float32, device) for k in ("lengths", "angles", "dihedrals"))
    an[0] = torch.tensor([100.0, 0.0, 0.0], device=device)  # 100 nm > 256 * 0.12 nm
    _, reg = _flagged_forward(lib, L, A, D, an)
    assert reg.cpu().tolist() == [0, 0]


def test_tiny_chain_is_not_regular_in_fp32(cufk, device):
    """Bonds below 2^-20 keep float32 chains off the position-based adjoint (whose bare
    reciprocal square roots need normal inputs); the exact path still matches the oracle."""
    lib = _abi()
    d = _inputs(3, 60, seed=28, anchors=False, dtype=torch.float32)
    d["lengths"][1] = _round(d["lengths"][1] * 4e-6, torch.float32)  # about 6e-7 < 2^-20
    L, A, D = (_dev(d[k], torch.float32, device) for k in ("lengths", "angles", "dihedrals"))
    an = _anchors3(d, torch.float32, device)
    _, reg = _flagged_forward(lib, L, A, D, an)
    assert reg.cpu().tolist() == [1, 0, 1]
    _, grads = _run(cufk, d, torch.float32, device)
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"])
    for got, want in zip(grads, ref):
        err = np.abs(got.double().cpu().numpy() - want).max(axis=1) / np.abs(want).max(axis=1)
        assert err.max() <= 5e-5, err


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("N", [4, 5, 70, 259, 1028, 2049, 2051])
def test_fast_and_exact_backward_agree(cufk, device, dtype, N):
    lib = _abi()
    d = _inputs(4, N, seed=300 + N, anchors=True, dtype=dtype)
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    g = _dev(d["grad"], dtype, device)
    an = _anchors3(d, dtype, device)
    xyz, reg = _flagged_forward(lib, L, A, D, an)
    assert reg.cpu().tolist() == [1] * 4
    p = lambda t: t.data_ptr()  # noqa: E731
    st = torch.cuda.current_stream().cuda_stream
    fast = [torch.empty_like(t) for t in (L, A, D)]
    exact = [torch.empty_like(t) for t in (L, A, D)]
    assert lib.cufk_reconstruct_bwd_saved(_CODES[dtype], p(L), p(A), p(D), *map(p, an), p(xyz), p(reg), p(g),
                                          *map(p, fast), 4, N, st) == 0
    assert lib.cufk_reconstruct_bwd(_CODES[dtype], p(L), p(A), p(D), *map(p, an), p(g), *map(p, exact), 4, N, st) == 0
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    tol = 1e-9 if dtype == torch.float64 else 5e-5
    for name, f, e, r in zip(("lengths", "angles", "dihedrals"), fast, exact, ref):
        scale = max(1e-30, np.abs(r).max())
        ef = np.abs(f.double().cpu().numpy() - r).max() / scale
        ee = np.abs(e.double().cpu().numpy() - r).max() / scale
        print(f"{dtype} N={N} d/d{name}: fast rel {ef:.2e}, exact rel {ee:.2e}")
        assert ef <= tol and ee <= tol


def test_inplace_modified_output_uses_exact_backward(cufk, device):
    d = _inputs(3, 200, seed=23, anchors=True, dtype=torch.float64)
    L, A, D = (_dev(d[k], torch.float64, device, True) for k in ("lengths", "angles", "dihedrals"))
    xyz = cufk.reconstruct(L, A, D, *_anchor_tensors(d, torch.float64, device).values())
    xyz.mul_(1.0)  # bumps the version counter; d(xyz)/d(xyz) is the identity
    grads = torch.autograd.grad(xyz, (L, A, D), _dev(d["grad"], torch.float64, device))
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for got, want in zip(grads, ref):
        assert np.abs(got.cpu().numpy() - want).max() <= 1e-9 * max(1.0, np.abs(want).max())


def test_mixed_regular_and_irregular_batch(cufk, device):
    d = _inputs(8, 600, seed=24, anchors=True, dtype=torch.float32)
    d["lengths"][2, 100] *= -1
    d["angles"][5, 300] = 0.1
    _, grads = _run(cufk, d, torch.float32, device)
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for got, want in zip(grads, ref):
        err = np.abs(got.double().cpu().numpy() - want).max(axis=1) / np.abs(want).max(axis=1)
        print("per-chain rel err", err)
        assert err.max() <= 5e-5


# ----------------------------------------------------------------- half types: float positions


def _shadow_forward(lib, L, A, D, an):
    """cufk_reconstruct_fwd_shadow; positions and flags are None where the library keeps none."""
    B, N = L.shape[0], L.shape[1] + 1
    xyz = torch.empty(B, N, 3, device=L.device, dtype=L.dtype)
    n = lib.cufk_reconstruct_shadow_floats(B, N)
    assert n in (0, B * N * 3)
    pos = torch.full((B, N, 3), float("nan"), device=L.device) if n else None
    reg = torch.full((B,), 7, device=L.device, dtype=torch.uint8) if n else None
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = lib.cufk_reconstruct_fwd_shadow(_CODES[L.dtype], p(L), p(A), p(D), *map(p, an), p(xyz), p(pos), p(reg), B, N,
                                         torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return xyz, pos, reg


def _shadow_backward(lib, L, A, D, an, pos, reg, g):
    B, N = L.shape[0], L.shape[1] + 1
    out = [torch.empty_like(t) for t in (L, A, D)]
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = lib.cufk_reconstruct_bwd_shadow(_CODES[L.dtype], p(L), p(A), p(D), *map(p, an), p(pos), p(reg), p(g),
                                         *map(p, out), B, N, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_shadow_forward_positions_and_flags(cufk, device, dtype):
    """The half-type forward that keeps float positions: its output equals the plain forward's
    bit for bit, the kept positions round to exactly that output, they match the float64
    oracle to float32 accuracy, and the flags follow the float32 regularity test (the cases of
    test_regularity_flags: negative bond, small angle inside and at the first frame, zero bond)."""
    lib = _abi()
    d = _inputs(6, 300, seed=21, anchors=True, dtype=dtype)
    d["lengths"][1, 7] = -d["lengths"][1, 7]
    d["angles"][2, 40] = _round(0.2, dtype)
    d["angles"][3, 0] = _round(math.pi - 0.2, dtype)
    d["lengths"][4, 1] = 0.0
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    an = _anchors3(d, dtype, device)
    xyz, pos, reg = _shadow_forward(lib, L, A, D, an)
    plain, _ = _flagged_forward(lib, L, A, D, an)
    torch.cuda.synchronize()
    assert torch.equal(xyz, plain)
    assert torch.equal(pos.to(dtype), xyz)
    assert reg.cpu().tolist() == [1, 0, 0, 0, 0, 1]
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    err = np.abs(pos.double().cpu().numpy() - ref).max()
    print(f"{dtype} shadow positions: max abs err {err:.2e} nm against float64 on the same inputs")
    assert err <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N", [4, 5, 70, 259, 1028, 2049, 2051])
def test_shadow_backward_is_the_float32_adjoint(cufk, device, dtype, N):
    """Over the kept float positions the half-type backward runs the float32 position-based
    adjoint on the same values: it equals cufk_reconstruct_bwd_saved at float32 (positions as
    xyz, the gradient widened exactly), rounded to the dtype, bit for bit.  Against the float64
    oracle on the rounded inputs it holds the low-precision sanity bound (3e-2 relative)."""
    lib = _abi()
    B = 4
    d = _inputs(B, N, seed=300 + N, anchors=True, dtype=dtype)
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    g = _dev(d["grad"], dtype, device)
    an = _anchors3(d, dtype, device)
    _, pos, reg = _shadow_forward(lib, L, A, D, an)
    assert reg.cpu().tolist() == [1] * B
    got = _shadow_backward(lib, L, A, D, an, pos, reg, g)
    f32 = [t.float() for t in (L, A, D)]
    an32 = [t.float() for t in an]
    want = [torch.empty_like(t) for t in f32]
    p = lambda t: t.data_ptr()  # noqa: E731
    assert lib.cufk_reconstruct_bwd_saved(0, *map(p, f32), *map(p, an32), p(pos), p(reg), p(g.float()), *map(p, want),
                                          B, N, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    for a, w in zip(got, want):
        assert torch.equal(a, w.to(dtype))
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for a, r in zip(got, ref):
        assert np.abs(a.double().cpu().numpy() - r).max() <= 3e-2 * max(1e-30, np.abs(r).max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_shadow_backward_irregular_chains_recompute(cufk, device, dtype):
    """Chains the forward flags irregular take the exact recompute inside the same launch: their
    gradients equal cufk_reconstruct_bwd's bit for bit; every chain stays within the
    low-precision bound of the oracle."""
    lib = _abi()
    B, N = 8, 600
    d = _inputs(B, N, seed=24, anchors=True, dtype=dtype)
    d["lengths"][2, 100] *= -1
    d["angles"][5, 300] = _round(0.1, dtype)
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    g = _dev(d["grad"], dtype, device)
    an = _anchors3(d, dtype, device)
    _, pos, reg = _shadow_forward(lib, L, A, D, an)
    assert reg.cpu().tolist() == [1, 1, 0, 1, 1, 0, 1, 1]
    got = _shadow_backward(lib, L, A, D, an, pos, reg, g)
    exact = [torch.empty_like(t) for t in (L, A, D)]
    p = lambda t: t.data_ptr()  # noqa: E731
    assert lib.cufk_reconstruct_bwd(_CODES[dtype], p(L), p(A), p(D), *map(p, an), p(g), *map(p, exact), B, N,
                                    torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    for a, e in zip(got, exact):
        assert torch.equal(a[[2, 5]], e[[2, 5]])
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for a, r in zip(got, ref):
        err = np.abs(a.double().cpu().numpy() - r).max(axis=1) / np.abs(r).max(axis=1)
        print(f"{dtype} per-chain rel err", err)
        assert err.max() <= 3e-2


def test_shadow_short_chains_in_large_batches_recompute(cufk, device):
    """Where the forward packs short chains (4096 chains of 100 points) the library keeps no
    float positions: the shadow forward writes the plain forward's output and the shadow
    backward, given NULL positions and flags, equals cufk_reconstruct_bwd bit for bit."""
    lib = _abi()
    dtype, B, N = torch.bfloat16, 4096, 100
    d = _inputs(B, N, seed=26, anchors=True, dtype=dtype)
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    g = _dev(d["grad"], dtype, device)
    an = _anchors3(d, dtype, device)
    xyz, pos, reg = _shadow_forward(lib, L, A, D, an)
    assert pos is None and reg is None
    plain, _ = _flagged_forward(lib, L, A, D, an)
    got = _shadow_backward(lib, L, A, D, an, None, None, g)
    exact = [torch.empty_like(t) for t in (L, A, D)]
    p = lambda t: t.data_ptr()  # noqa: E731
    assert lib.cufk_reconstruct_bwd(_CODES[dtype], p(L), p(A), p(D), *map(p, an), p(g), *map(p, exact), B, N,
                                    torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(xyz, plain)
    for a, e in zip(got, exact):
        assert torch.equal(a, e)


def test_half_autograd_takes_the_float_positions(cufk, device):
    """bfloat16 autograd: the step's gradients are those of the shadow entry points; without
    gradients the forward is the plain one."""
    lib = _abi()
    dtype, B, N = torch.bfloat16, 16, 1026
    d = _inputs(B, N, seed=27, anchors=True, dtype=dtype)
    xyz, grads = _run(cufk, d, dtype, device)
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    g = _dev(d["grad"], dtype, device)
    an = _anchors3(d, dtype, device)
    sx, pos, reg = _shadow_forward(lib, L, A, D, an)
    want = _shadow_backward(lib, L, A, D, an, pos, reg, g)
    nograd, _ = _run(cufk, d, dtype, device, grad=False)
    torch.cuda.synchronize()
    assert torch.equal(xyz, sx) and torch.equal(nograd, sx)
    for a, w in zip(grads, want):
        assert torch.equal(a, w)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_angles_beyond_the_polynomial_range(cufk, device, dtype):
    """Angles with |x| > 65536 take the library sin/cos (the kernels switch the whole chain to
    the checked loop).  Chain 0 is ordinary, chain 1 regular with one huge dihedral, chain 2
    irregular (negative bond) with a huge dihedral and a huge bond angle, chain 3 a huge
    angle near a lane boundary.  Forward, the one-launch backward and the exact backward
    against the oracle on the same (dtype-rounded) inputs; fp32 tolerances as above, bf16
    compared with a loose 2e-2 relative bound (it computes in float from rounded inputs)."""
    lib = _abi()
    B, N = 4, 300
    d = _inputs(B, N, seed=25, anchors=True, dtype=dtype)
    d["dihedrals"][1, 50] += 2 * math.pi * 20000.0
    d["lengths"][2, 10] *= -1
    d["dihedrals"][2, 123] -= 2 * math.pi * 30000.0
    d["angles"][2, 200] += 2 * math.pi * 15000.0
    d["angles"][3, 8] = -1.0e6
    d = {k: _round(v, dtype) for k, v in d.items()}
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    g = _dev(d["grad"], dtype, device)
    an = _anchors3(d, dtype, device)
    xyz, reg = _flagged_forward(lib, L, A, D, an)
    ref_x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    tol_x = 1e-4 if dtype == torch.float32 else 2e-2
    err_x = np.abs(xyz.double().cpu().numpy() - ref_x).max() / max(1.0, np.abs(ref_x).max())
    print(f"{dtype} wide-range forward: rel max err {err_x:.2e}, flags {reg.cpu().tolist()}")
    assert err_x <= tol_x
    if dtype == torch.float32:
        assert reg.cpu().tolist()[:3] == [1, 1, 0]
    p = lambda t: t.data_ptr()  # noqa: E731
    st = torch.cuda.current_stream().cuda_stream
    saved = [torch.empty_like(t) for t in (L, A, D)]
    exact = [torch.empty_like(t) for t in (L, A, D)]
    code = _CODES[dtype]
    assert lib.cufk_reconstruct_bwd_saved(code, p(L), p(A), p(D), *map(p, an), p(xyz), p(reg), p(g), *map(p, saved), B,
                                          N, st) == 0
    assert lib.cufk_reconstruct_bwd(code, p(L), p(A), p(D), *map(p, an), p(g), *map(p, exact), B, N, st) == 0
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    tol = 5e-5 if dtype == torch.float32 else 5e-2
    for name, s_, e_, r in zip(("lengths", "angles", "dihedrals"), saved, exact, ref):
        scale = np.abs(r).max(axis=1, keepdims=True)
        es = (np.abs(s_.double().cpu().numpy() - r) / scale).max()
        ee = (np.abs(e_.double().cpu().numpy() - r) / scale).max()
        print(f"{dtype} wide-range d/d{name}: saved rel {es:.2e}, exact rel {ee:.2e}")
        assert es <= tol and ee <= tol


def test_huge_chain_is_not_regular_in_fp32(cufk, device):
    """Coordinates beyond 2^29 keep float32 chains off the position-based adjoint (whose squared
    bond normals would overflow float); the exact path still matches the oracle."""
    lib = _abi()
    d = _inputs(3, 60, seed=29, anchors=False, dtype=torch.float32)
    d["lengths"][1] = _round(d["lengths"][1] * 7.0e10, torch.float32)  # bonds of about 1e10: |b1 x b2|^2 > FLT_MAX
    L, A, D = (_dev(d[k], torch.float32, device) for k in ("lengths", "angles", "dihedrals"))
    _, reg = _flagged_forward(lib, L, A, D, _anchors3(d, torch.float32, device))
    assert reg.cpu().tolist() == [1, 0, 1]
    _, grads = _run(cufk, d, torch.float32, device)
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"])
    for got, want in zip(grads, ref):
        assert torch.isfinite(got).all()
        err = np.abs(got.double().cpu().numpy() - want).max(axis=1) / np.abs(want).max(axis=1)
        assert err.max() <= 5e-5, err

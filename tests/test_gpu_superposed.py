"""Fused superposed losses (reconstruct_rmsd; compile_torsion(...).rmsd) and the fused torsion
coordinate loss (compile_torsion(...).loss) against the float64 oracle.

The oracle composes its forward with the SVD Kabsch superposition (oracle/nerf64.py superpose,
an independent route from the kernels' quaternion eigenproblem) and its reference backward
with superposed_grad_xyz.  Bars: float64 loss 1e-12 relative, gradients 1e-10 relative;
float32 loss 1e-5 relative; float32 gradients 5e-5 relative (normwise per output) of the
oracle's adjoint fed with grad_xyz formed from the positions the kernels stored (the float64
values of the float32 output), which separates the adjoint from the forward's own position
error; float16/bfloat16 reported with sanity bounds.
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
    return torch.as_tensor(np.asarray(x), dtype=torch.float64).to(dtype).double().numpy()


def _case(B, N, seed, dtype, noise=0.3, rotate=True):
    """Inputs and a target: the true chain, rigidly moved (so the superposition matters), plus
    N(0, noise) nm per coordinate."""
    d = o.synthetic_inputs(B, N, seed, anchors=True)
    an = {k: d[k] for k in ("p0", "first_direction", "initial_normal")}
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **an)
    rng = np.random.default_rng(seed + 1)
    if rotate:
        q, _ = np.linalg.qr(rng.normal(size=(3, 3)))
        q *= np.sign(np.linalg.det(q))
        x = x @ q.T + rng.normal(size=3) * 4.0
    d["target"] = x + rng.normal(0.0, noise, x.shape)
    return {k: _round(v, dtype) for k, v in d.items()}


def _anchors(d):
    return {k: d[k] for k in ("p0", "first_direction", "initial_normal")}


def _ref(d, squared, w=None, x_used=None):
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchors(d))
    loss = o.superposed_loss(x, d["target"], squared)
    gx = o.superposed_grad_xyz(x if x_used is None else x_used, d["target"], w, squared)
    return loss, o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], gx, **_anchors(d))


def _run(cufk, d, dtype, device, squared, w=None):
    L, A, D = (_dev(d[k], dtype, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = {k: _dev(v, dtype, device) for k, v in _anchors(d).items()}
    loss = cufk.reconstruct_rmsd(L, A, D, _dev(d["target"], dtype, device), **an, squared=squared)
    weights = torch.ones_like(loss) if w is None else _dev(w, dtype, device)
    return loss, torch.autograd.grad(loss, (L, A, D), weights)


def _stored(cufk, d, dtype, device):
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    an = {k: _dev(v, dtype, device) for k, v in _anchors(d).items()}
    return cufk.reconstruct(L, A, D, **an).double().cpu().numpy()


@pytest.mark.parametrize("squared", [False, True])
@pytest.mark.parametrize("N", [4, 5, 37, 260, 1027, 2051])
def test_rmsd_fp64_matches_oracle(cufk, device, N, squared):
    d = _case(3, N, seed=700 + N, dtype=torch.float64)
    w = np.array([1.0, -0.5, 2.5])
    loss, grads = _run(cufk, d, torch.float64, device, squared, w)
    ref_loss, ref_g = _ref(d, squared, w)
    lerr = np.abs(loss.detach().cpu().numpy() - ref_loss).max() / np.abs(ref_loss).max()
    gerr = [np.abs(g.cpu().numpy() - r).max() / np.abs(r).max() for g, r in zip(grads, ref_g)]
    print(f"fp64 superposed N={N} squared={squared}: loss {lerr:.2e}, grads " + ", ".join(f"{e:.2e}" for e in gerr))
    assert lerr <= 1e-12
    assert max(gerr) <= 1e-10


def _unfused(cufk, d, dtype, device, squared):
    """reconstruct, then the superposed loss in torch (the rotation solved on the host by SVD and
    held fixed: its own dependence drops out at the optimum), then autograd."""
    L, A, D = (_dev(d[k], dtype, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = {k: _dev(v, dtype, device) for k, v in _anchors(d).items()}
    x = cufk.reconstruct(L, A, D, **an)
    t = _dev(d["target"], dtype, device)
    xc, tc = x - x.mean(1, keepdim=True), t - t.mean(1, keepdim=True)
    R, _, _, _ = o.superpose(x.detach().double().cpu().numpy(), d["target"])
    Rt = torch.as_tensor(R).to(device=device, dtype=dtype).transpose(1, 2).contiguous()
    msd = ((xc @ Rt - tc) ** 2).sum(-1).mean(-1)
    loss = msd if squared else msd.sqrt()
    return loss, torch.autograd.grad(loss.sum(), (L, A, D))


@pytest.mark.parametrize("squared", [False, True])
@pytest.mark.parametrize("N", [64, 2049])
def test_rmsd_fp32(cufk, device, N, squared):
    """float32: the loss within 1e-5 relative.  Gradients against the oracle's adjoint over the
    stored positions: within 5e-5 relative, or within the unfused composition's own error where
    that is larger.  A superposed loss is invariant under rigid motions, so its grad_xyz has zero
    net force and torque: the adjoint's float32 suffix sums end in a small remainder of a long
    cancelling sum, which amplifies their relative error at long chains (6.6e-5 at N = 2049);
    the unfused composition, reconstruct's own backward, carries the same."""
    d = _case(16, N, seed=5, dtype=torch.float32)
    loss, grads = _run(cufk, d, torch.float32, device, squared)
    ref_loss, _ = _ref(d, squared)
    _, adj = _ref(d, squared, x_used=_stored(cufk, d, torch.float32, device))
    _, ug = _unfused(cufk, d, torch.float32, device, squared)
    lerr = np.abs(loss.detach().double().cpu().numpy() - ref_loss).max() / np.abs(ref_loss).max()
    gerr = [np.abs(g.double().cpu().numpy() - r).max() / np.abs(r).max() for g, r in zip(grads, adj)]
    uerr = [np.abs(g.double().cpu().numpy() - r).max() / np.abs(r).max() for g, r in zip(ug, adj)]
    print(f"fp32 superposed N={N} squared={squared}: loss {lerr:.2e}, adjoint grads fused "
          + ", ".join(f"{e:.2e}" for e in gerr) + ", unfused " + ", ".join(f"{e:.2e}" for e in uerr))
    assert lerr <= 1e-5
    for f, u in zip(gerr, uerr):
        assert f <= max(5e-5, 1.5 * u)


@pytest.mark.parametrize("squared", [True, False])
def test_rmsd_fp32_small_deviation(cufk, device, squared):
    """Well-fitted chains, where training drives the loss: N = 2049 and 1e-3 nm of noise (mean
    squared deviation about 3e-6 nm^2).  The fused MSD is (sum |x'|^2 + sum |t'|^2 - 2 lambda) / N,
    a small difference of sums near 1e5 nm^2, so its float32 error has an absolute floor; the
    bounds below are stated against the oracle's SVD superposition of the positions the kernel
    stored, for the MSD (absolute, nm^2) and the gradients (normwise relative, per output).
    Measured: MSD within 2e-9 nm^2 (7e-4 relative); gradients of the MSD within 1.5e-5, of the
    RMSD within 2.5e-4 (its gradient scale 1 / (2 rmsd) carries half the MSD's relative error)."""
    d = _case(16, 2049, seed=9, dtype=torch.float32, noise=1e-3)
    stored = _stored(cufk, d, torch.float32, device)
    loss, grads = _run(cufk, d, torch.float32, device, squared)
    got = loss.detach().double().cpu().numpy()
    msd = got if squared else got**2
    ref_msd = o.superposed_loss(stored, d["target"], squared=True)
    _, adj = _ref(d, squared, x_used=stored)
    merr = np.abs(msd - ref_msd).max()
    gerr = [np.abs(g.double().cpu().numpy() - r).max() / np.abs(r).max() for g, r in zip(grads, adj)]
    print(f"fp32 small deviation squared={squared}: msd {ref_msd.mean():.3e} nm^2, abs error {merr:.2e} nm^2 "
          f"({merr / ref_msd.min():.2e} relative), grads " + ", ".join(f"{e:.2e}" for e in gerr))
    assert merr <= 6e-9
    assert max(gerr) <= (5e-5 if squared else 1e-3)


def test_rmsd_matches_the_unfused_composition(cufk, device):
    """float64: the fused loss and gradients equal the unfused composition's within 1e-12 / 1e-10."""
    d = _case(4, 300, seed=21, dtype=torch.float64)
    loss, grads = _run(cufk, d, torch.float64, device, False)
    unfused, ug = _unfused(cufk, d, torch.float64, device, False)
    assert torch.allclose(loss.detach(), unfused.detach(), rtol=1e-12, atol=0)
    for a, b in zip(grads, ug):
        assert (a - b).abs().max() <= 1e-10 * b.abs().max()


def test_rmsd_of_a_rigid_copy_is_zero(cufk, device):
    """A target that is the chain itself, rigidly moved: the mean squared deviation vanishes to
    rounding (the kernel forms it as sum |x'|^2 + sum |t'|^2 - 2 lambda, about 1e3 nm^2 here,
    so to about 1e-12 nm^2), and so does its gradient."""
    d = _case(3, 200, seed=31, dtype=torch.float64, noise=0.0)
    loss, grads = _run(cufk, d, torch.float64, device, True)
    assert loss.abs().max() <= 1e-12
    for g in grads:
        assert g.abs().max() <= 1e-9


def test_rmsd_to_a_single_point_is_the_radius_of_gyration(cufk, device):
    """A target collapsed to one point makes the key matrix zero (every rotation is optimal; the
    solver's fallback branch): the RMSD is the chain's radius of gyration, whose gradient
    (x - xbar) / (N rg) the oracle's adjoint turns into the internal-coordinate gradients."""
    d = _case(3, 150, seed=35, dtype=torch.float64)
    d["target"] = np.zeros_like(d["target"]) + 1.5
    loss, grads = _run(cufk, d, torch.float64, device, False)
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchors(d))
    xc = x - x.mean(axis=1, keepdims=True)
    rg = np.sqrt(np.mean(np.sum(xc**2, -1), axis=1))
    assert np.abs(loss.detach().cpu().numpy() - rg).max() <= 1e-12 * rg.max()
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], xc / (x.shape[1] * rg[:, None, None]),
                                 **_anchors(d))
    for g, r in zip(grads, ref):
        assert np.abs(g.cpu().numpy() - r).max() <= 1e-10 * np.abs(r).max()


def test_rmsd_irregular_chains_take_the_exact_adjoint(cufk, device):
    d = _case(4, 300, seed=33, dtype=torch.float32)
    d["lengths"][1, 50] *= -1
    d["angles"][2, 80] = _round(0.05, torch.float32)
    loss, grads = _run(cufk, d, torch.float32, device, False)
    _, adj = _ref(d, False, x_used=_stored(cufk, d, torch.float32, device))
    for g, r in zip(grads, adj):
        err = np.abs(g.double().cpu().numpy() - r).max(axis=1) / np.abs(r).max(axis=1)
        print("per-chain grad rel err", err)
        assert err.max() <= 5e-5


def test_rmsd_single_chain_and_gradcheck(cufk, device):
    d = _case(1, 15, seed=41, dtype=torch.float64)
    L, A, D = (_dev(d[k][0], torch.float64, device, True) for k in ("lengths", "angles", "dihedrals"))
    t = _dev(d["target"][0], torch.float64, device)
    loss = cufk.reconstruct_rmsd(L, A, D, t)
    assert loss.dim() == 0
    for squared in (False, True):
        assert torch.autograd.gradcheck(lambda a, b, c: cufk.reconstruct_rmsd(a, b, c, t, squared=squared), (L, A, D),
                                        eps=1e-6, atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rmsd_low_precision_reported(cufk, device, dtype):
    d = _case(8, 300, seed=43, dtype=dtype, noise=1.0)
    loss, grads = _run(cufk, d, dtype, device, False)
    ref_loss, ref_g = _ref(d, False)
    lerr = np.abs(loss.detach().double().cpu().numpy() - ref_loss).max() / np.abs(ref_loss).max()
    gerr = [float(np.abs(g.double().cpu().numpy() - r).max() / np.abs(r).max()) for g, r in zip(grads, ref_g)]
    print(f"{dtype} rmsd: loss rel {lerr:.2e}, grads " + ", ".join(f"{e:.2e}" for e in gerr))
    assert torch.isfinite(loss).all() and lerr <= 2e-2 and max(gerr) <= 5e-2


def test_rmsd_validation(cufk, device):
    L, A, D = torch.ones(2, 9, device=device), torch.ones(2, 8, device=device), torch.ones(2, 7, device=device)
    with pytest.raises(RuntimeError, match="target must have shape"):
        cufk.reconstruct_rmsd(L, A, D, torch.zeros(2, 9, 3, device=device))
    with pytest.raises(RuntimeError, match="target gradients are not supported"):
        cufk.reconstruct_rmsd(L, A, D, torch.zeros(2, 10, 3, device=device, requires_grad=True))


# ----------------------------------------------------------------- torsion path


def _torsion_case(B, N, seed, dtype):
    rng = np.random.default_rng(seed)
    raw = rng.normal(size=(B, 2 * (N - 3)))
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    x = o.torsion_forward(raw, c)
    q, _ = np.linalg.qr(rng.normal(size=(3, 3)))
    q *= np.sign(np.linalg.det(q))
    t = x @ q.T + 2.0 + rng.normal(0.0, 0.3, x.shape)
    return _round(raw, dtype), _round(t, dtype), c


def _torsion_ref(raw, t, c, kind, x_used=None):
    x = o.torsion_forward(raw, c)
    xu = x if x_used is None else x_used
    if kind == 0:
        return ((x - t) ** 2).sum(axis=(1, 2)), o.torsion_backward(raw, xu, 2.0 * (xu - t), c)
    sq = kind == 1
    return o.superposed_loss(x, t, sq), o.torsion_backward(raw, xu, o.superposed_grad_xyz(xu, t, None, sq), c)


def _torsion_run(cufk, raw, t, dtype, device, kind):
    f = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    r = _dev(raw, dtype, device, True)
    tt = _dev(t, dtype, device)
    loss = f.loss(r, tt) if kind == 0 else f.rmsd(r, tt, squared=kind == 1)
    (g,) = torch.autograd.grad(loss, (r,), torch.ones_like(loss))
    return loss, g


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("N", [4, 5, 100, 388, 771, 2051])
def test_torsion_losses_fp64(cufk, device, N, kind):
    raw, t, c = _torsion_case(3, N, 800 + N, torch.float64)
    loss, g = _torsion_run(cufk, raw, t, torch.float64, device, kind)
    ref_loss, ref_g = _torsion_ref(raw, t, c, kind)
    lerr = np.abs(loss.detach().cpu().numpy() - ref_loss).max() / np.abs(ref_loss).max()
    gerr = np.abs(g.cpu().numpy() - ref_g).max() / np.abs(ref_g).max()
    print(f"torsion loss kind={kind} N={N}: loss {lerr:.2e}, grad {gerr:.2e}")
    assert lerr <= 1e-12 and gerr <= 1e-10


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_torsion_losses_fp32(cufk, device, kind):
    raw, t, c = _torsion_case(16, 771, 901, torch.float32)
    loss, g = _torsion_run(cufk, raw, t, torch.float32, device, kind)
    xs = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)(_dev(raw, torch.float32, device)).double().cpu().numpy()
    ref_loss, _ = _torsion_ref(raw, t, c, kind)
    _, adj = _torsion_ref(raw, t, c, kind, x_used=xs)
    lerr = np.abs(loss.detach().double().cpu().numpy() - ref_loss).max() / np.abs(ref_loss).max()
    gerr = np.abs(g.double().cpu().numpy() - adj).max(axis=1) / np.abs(adj).max(axis=1)
    print(f"torsion fp32 kind={kind}: loss {lerr:.2e}, worst per-chain adjoint grad {gerr.max():.2e}")
    assert lerr <= 1e-5 and gerr.max() <= 5e-5


def test_torsion_loss_equals_the_unfused_composition(cufk, device):
    """compile_torsion(...).loss is the torsion path followed by the coordinate loss in torch,
    with the strided raw-pair gradient layout kept."""
    raw, t, _ = _torsion_case(4, 200, 77, torch.float64)
    f = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    wide = torch.zeros(4, raw.shape[1] + 6, dtype=torch.float64, device=device)
    wide[:, 2 : 2 + raw.shape[1]] = _dev(raw, torch.float64, device)
    r1 = wide[:, 2 : 2 + raw.shape[1]].detach().clone().requires_grad_(True)
    tt = _dev(t, torch.float64, device)
    fused = f.loss(r1, tt)
    (g1,) = torch.autograd.grad(fused.sum(), (r1,))
    r2 = r1.detach().clone().requires_grad_(True)
    plain = ((f(r2) - tt) ** 2).sum((-2, -1))
    (g2,) = torch.autograd.grad(plain.sum(), (r2,))
    assert torch.allclose(fused, plain, rtol=1e-13, atol=0)
    assert (g1 - g2).abs().max() <= 1e-12 * g2.abs().max()
    strided = wide.detach().clone()[:, 2 : 2 + raw.shape[1]].requires_grad_(True)
    (g3,) = torch.autograd.grad(f.loss(strided, tt).sum(), (strided,))
    assert g3.stride() == strided.stride() and torch.allclose(g3, g1, rtol=0, atol=0)


def test_torsion_loss_gradcheck(cufk, device):
    raw, t, _ = _torsion_case(2, 12, 5, torch.float64)
    f = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    r = _dev(raw, torch.float64, device, True)
    tt = _dev(t, torch.float64, device)
    assert torch.autograd.gradcheck(lambda x: f.loss(x, tt), (r,), eps=1e-6, atol=1e-7, rtol=1e-6)
    assert torch.autograd.gradcheck(lambda x: f.rmsd(x, tt), (r,), eps=1e-6, atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_torsion_losses_low_precision_reported(cufk, device, dtype):
    raw, t, c = _torsion_case(4, 300, 31, dtype)
    for kind in (0, 2):
        loss, g = _torsion_run(cufk, raw, t, dtype, device, kind)
        ref_loss, ref_g = _torsion_ref(raw, t, c, kind)
        lerr = np.abs(loss.detach().double().cpu().numpy() - ref_loss).max() / np.abs(ref_loss).max()
        gerr = np.abs(g.double().cpu().numpy() - ref_g).max() / np.abs(ref_g).max()
        print(f"torsion {dtype} kind={kind}: loss rel {lerr:.2e}, grad rel {gerr:.2e}")
        assert torch.isfinite(loss).all() and torch.isfinite(g).all() and lerr <= 2e-2 and gerr <= 0.5

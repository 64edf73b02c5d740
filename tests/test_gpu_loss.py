"""Fused coordinate loss (reconstruct_loss): loss[b] = sum_i |x_bi - t_bi|^2 with the
reconstruction inside the kernels.

The oracle composes its forward with the loss, and its reference backward with
grad_xyz = 2 w_b (x - t); bars as for reconstruct (float64 1e-12 relative loss and 1e-10
relative gradients; float32 1e-5 relative loss).  float32 gradients are held to 5e-5 relative of
the oracle's backward fed grad_xyz = 2 w_b (x - t) with x the float32 positions the kernels
stored (the float64 values of reconstruct's float32 output): that isolates the adjoint from the
forward's own position error, which `2 (x - t)` would otherwise carry into every gradient.  The
unfused PyTorch composition, reconstruct followed by the same loss in torch, is checked
alongside.
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


def _case(B, N, seed, dtype, noise=0.3):
    """Inputs and a target near the true chain (the true positions plus N(0, noise) nm)."""
    d = o.synthetic_inputs(B, N, seed, anchors=True)
    an = {k: d[k] for k in ("p0", "first_direction", "initial_normal")}
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **an)
    d["target"] = x + np.random.default_rng(seed + 1).normal(0.0, noise, x.shape)
    return {k: _round(v, dtype) for k, v in d.items()}


def _ref(d, w=None, x_used=None):
    """Oracle loss and gradients; with x_used (the positions a kernel stored, as float64) the
    gradient grad_xyz = 2 w (x_used - t) is formed from those positions instead."""
    an = {k: d[k] for k in ("p0", "first_direction", "initial_normal")}
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **an)
    loss = ((x - d["target"]) ** 2).sum(axis=(1, 2))
    w = np.ones(len(loss)) if w is None else w
    g = 2.0 * w[:, None, None] * ((x if x_used is None else x_used) - d["target"])
    grads = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], g, **an)
    return loss, grads


def _run(cufk, d, dtype, device, w=None):
    L, A, D = (_dev(d[k], dtype, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = {k: _dev(d[k], dtype, device) for k in ("p0", "first_direction", "initial_normal")}
    loss = cufk.reconstruct_loss(L, A, D, _dev(d["target"], dtype, device), **an)
    weights = torch.ones_like(loss) if w is None else _dev(w, dtype, device)
    grads = torch.autograd.grad(loss, (L, A, D), weights)
    return loss, grads


@pytest.mark.parametrize("N", [4, 5, 37, 260, 1027, 2051])
def test_loss_fp64_matches_oracle(cufk, device, N):
    d = _case(3, N, seed=400 + N, dtype=torch.float64)
    w = np.array([1.0, -0.5, 2.5])
    loss, grads = _run(cufk, d, torch.float64, device, w)
    ref_loss, ref_g = _ref(d, w)
    assert np.abs(loss.detach().cpu().numpy() - ref_loss).max() <= 1e-12 * np.abs(ref_loss).max()
    for got, want in zip(grads, ref_g):
        gerr = np.abs(got.cpu().numpy() - want).max() / np.abs(want).max()
        assert gerr <= 1e-10, gerr


def _stored_positions(cufk, d, dtype, device):
    """The positions the fused forward stores: reconstruct's output (the same kernel arithmetic)."""
    L, A, D = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals"))
    an = {k: _dev(d[k], dtype, device) for k in ("p0", "first_direction", "initial_normal")}
    return cufk.reconstruct(L, A, D, **an).double().cpu().numpy()


@pytest.mark.parametrize("N", [64, 2049])
def test_loss_fp32_and_the_unfused_composition(cufk, device, N):
    """float32: the loss within 1e-5 relative of the oracle and of the unfused composition;
    gradients within 5e-5 relative of the oracle's adjoint over the stored positions, and
    within the unfused composition's own error against the oracle's (where 2 (x - t) carries
    the forward's position error: 1.6e-4 relative at N = 2049)."""
    d = _case(16, N, seed=5, dtype=torch.float32)
    loss, grads = _run(cufk, d, torch.float32, device)
    ref_loss, ref_g = _ref(d)
    _, adj_g = _ref(d, x_used=_stored_positions(cufk, d, torch.float32, device))
    lerr = np.abs(loss.detach().double().cpu().numpy() - ref_loss).max() / np.abs(ref_loss).max()
    L, A, D = (_dev(d[k], torch.float32, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = {k: _dev(d[k], torch.float32, device) for k in ("p0", "first_direction", "initial_normal")}
    x = cufk.reconstruct(L, A, D, **an)
    unfused = ((x - _dev(d["target"], torch.float32, device)) ** 2).sum((-2, -1))
    ug = torch.autograd.grad(unfused.sum(), (L, A, D))
    print(f"fp32 fused loss N={N}: loss rel err {lerr:.2e}")
    assert lerr <= 1e-5
    assert torch.allclose(unfused, loss.detach(), rtol=1e-5, atol=0)
    for got, alt, want, adj in zip(grads, ug, ref_g, adj_g):
        scale = np.abs(want).max()
        fused_err = np.abs(got.double().cpu().numpy() - want).max() / scale
        unfused_err = np.abs(alt.double().cpu().numpy() - want).max() / scale
        adj_err = np.abs(got.double().cpu().numpy() - adj).max() / np.abs(adj).max()
        print(f"  grad rel err: adjoint {adj_err:.2e}; against the float64 chain fused {fused_err:.2e}, "
              f"unfused {unfused_err:.2e}")
        assert adj_err <= 5e-5
        assert fused_err <= max(2 * unfused_err, 2e-5)


def test_loss_irregular_chains(cufk, device):
    d = _case(4, 300, seed=31, dtype=torch.float32)
    d["lengths"][1, 50] *= -1
    d["angles"][2, 80] = 0.05
    loss, grads = _run(cufk, d, torch.float32, device)
    ref_loss, _ = _ref(d)
    _, ref_g = _ref(d, x_used=_stored_positions(cufk, d, torch.float32, device))
    assert np.abs(loss.detach().double().cpu().numpy() - ref_loss).max() <= 1e-5 * np.abs(ref_loss).max()
    for got, want in zip(grads, ref_g):
        err = np.abs(got.double().cpu().numpy() - want).max(axis=1) / np.abs(want).max(axis=1)
        print("  per-chain grad rel err", err)
        assert err.max() <= 5e-5, err


def test_loss_single_chain_and_gradcheck(cufk, device):
    d = _case(1, 17, seed=41, dtype=torch.float64)
    L, A, D = (_dev(d[k][0], torch.float64, device, True) for k in ("lengths", "angles", "dihedrals"))
    t = _dev(d["target"][0], torch.float64, device)
    loss = cufk.reconstruct_loss(L, A, D, t)
    assert loss.dim() == 0
    assert torch.autograd.gradcheck(lambda l, a, dd: cufk.reconstruct_loss(l, a, dd, t), (L, A, D), eps=1e-6,
                                    atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_loss_low_precision_reported(cufk, device, dtype):
    d = _case(8, 300, seed=43, dtype=dtype, noise=1.0)
    loss, grads = _run(cufk, d, dtype, device)
    ref_loss, ref_g = _ref(d)
    lerr = np.abs(loss.detach().double().cpu().numpy() - ref_loss).max() / np.abs(ref_loss).max()
    gerr = [float(np.abs(g.double().cpu().numpy() - r).max() / np.abs(r).max()) for g, r in zip(grads, ref_g)]
    print(f"{dtype} fused loss: loss rel {lerr:.2e}, grads " + ", ".join(f"{e:.2e}" for e in gerr))
    assert torch.isfinite(loss).all() and lerr <= 2e-2 and max(gerr) <= 5e-2


def test_loss_validation(cufk, device):
    L = torch.ones(2, 9, device=device)
    A = torch.ones(2, 8, device=device)
    D = torch.ones(2, 7, device=device)
    with pytest.raises(RuntimeError, match="target must have shape"):
        cufk.reconstruct_loss(L, A, D, torch.zeros(2, 9, 3, device=device))
    with pytest.raises(RuntimeError, match="target gradients are not supported"):
        cufk.reconstruct_loss(L, A, D, torch.zeros(2, 10, 3, device=device, requires_grad=True))
    with pytest.raises(RuntimeError, match="target must have the same dtype"):
        cufk.reconstruct_loss(L, A, D, torch.zeros(2, 10, 3, device=device, dtype=torch.float64))
    n = 2100
    with pytest.raises(RuntimeError, match="at most 2048 local transforms"):
        cufk.reconstruct_loss(torch.ones(1, n - 1, device=device), torch.ones(1, n - 2, device=device),
                              torch.ones(1, n - 3, device=device), torch.zeros(1, n, 3, device=device))

"""Anchor gradients (reconstruct(..., anchor_grads=True)) against the float64 oracle's
anchor_gradients (pinned by finite differences and torch autograd in test_oracle.py).

Shapes cover the one-chain-per-workgroup kernels and the packed ones (at least 4096 chains
of at most 64 steps), the saved-output backward and the recompute after an in-place change,
and the degenerate normal (initial_normal parallel to first_direction).  Bars: float64
1e-10 relative; float32 5e-5 relative; float16/bfloat16 reported with sanity bounds.
"""

from __future__ import annotations

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


def _run(cufk, d, dtype, device, modify=False):
    L, A, D = (_dev(d[k], dtype, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = [_dev(d[k], dtype, device, True) for k in ("p0", "first_direction", "initial_normal")]
    xyz = cufk.reconstruct(L, A, D, *an, anchor_grads=True)
    if modify:
        xyz.mul_(1.0)  # in place (version bump): the backward recomputes the positions
    return torch.autograd.grad(xyz, (L, A, D, *an), _dev(d["grad"], dtype, device))


def _case(B, N, seed, dtype=torch.float64, fd=None, n0=None):
    d = o.synthetic_inputs(B, N, seed, anchors=True)
    if fd is not None:
        d["first_direction"], d["initial_normal"] = np.array(fd, float), np.array(n0, float)
    return {k: _round(v, dtype) for k, v in d.items()}


def _ref(d):
    an = {k: d[k] for k in ("p0", "first_direction", "initial_normal")}
    g = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **an)
    a = o.anchor_gradients(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **an)
    return list(g) + list(a)


@pytest.mark.parametrize("B,N", [(3, 5), (3, 300), (2, 2051), (4133, 20), (4133, 67)])
@pytest.mark.parametrize("modify", [False, True])
def test_anchor_gradients_fp64(cufk, device, B, N, modify):
    d = _case(B, N, seed=500 + N)
    got = _run(cufk, d, torch.float64, device, modify)
    for name, a, b in zip(("L", "A", "D", "p0", "fd", "n0"), got, _ref(d)):
        err = np.abs(a.cpu().numpy() - b).max() / max(np.abs(b).max(), 1e-300)
        assert err <= 1e-10, (name, err)


@pytest.mark.parametrize("fd,n0", [([0.0, 0.0, 2.0], [0.0, 0.0, -3.0]), ([1.5, 0.2, 0.0], [3.0, 0.4, 0.0])])
def test_anchor_gradients_degenerate_normal(cufk, device, fd, n0):
    d = _case(3, 40, seed=7, fd=fd, n0=n0)
    got = _run(cufk, d, torch.float64, device)
    ref = _ref(d)
    assert torch.all(got[5] == 0)  # the normal comes from the helper axis
    for a, b in zip(got, ref):
        assert np.abs(a.cpu().numpy() - b).max() <= 1e-10 * max(1.0, np.abs(b).max())


def test_anchor_gradients_fp32(cufk, device):
    d = _case(64, 2049, seed=9, dtype=torch.float32)
    got = _run(cufk, d, torch.float32, device)
    for name, a, b in zip(("L", "A", "D", "p0", "fd", "n0"), got, _ref(d)):
        err = np.abs(a.double().cpu().numpy() - b).max() / np.abs(b).max()
        print(f"fp32 {name}: rel err {err:.2e}")
        assert err <= 5e-5, name


def test_anchor_gradcheck(cufk, device):
    d = _case(2, 12, seed=11)
    L, A, D = (_dev(d[k], torch.float64, device) for k in ("lengths", "angles", "dihedrals"))
    an = tuple(_dev(d[k], torch.float64, device, True) for k in ("p0", "first_direction", "initial_normal"))
    assert torch.autograd.gradcheck(lambda p, f, n: cufk.reconstruct(L, A, D, p, f, n, anchor_grads=True), an,
                                    eps=1e-6, atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_anchor_gradients_low_precision_reported(cufk, device, dtype):
    d = _case(8, 300, seed=13, dtype=dtype)
    got = _run(cufk, d, dtype, device)
    errs = [float(np.abs(a.double().cpu().numpy() - b).max() / np.abs(b).max()) for a, b in zip(got[3:], _ref(d)[3:])]
    print(f"{dtype} anchor grads rel err (p0, fd, n0): " + ", ".join(f"{e:.2e}" for e in errs))
    assert max(errs) <= 5e-2


def test_plain_reconstruct_still_rejects_anchor_grads(cufk, device):
    L, A, D = torch.ones(1, 9, device=device), torch.ones(1, 8, device=device), torch.ones(1, 7, device=device)
    with pytest.raises(RuntimeError, match="p0 gradients are not supported"):
        cufk.reconstruct(L, A, D, torch.zeros(3, device=device, requires_grad=True))


# ----------------------------------------------------------------- fused coordinate loss, long chains


def _loss_case(B, N, seed, dtype=torch.float64):
    d = _case(B, N, seed, dtype)
    an = {k: d[k] for k in ("p0", "first_direction", "initial_normal")}
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **an)
    d["target"] = _round(x + np.random.default_rng(seed).normal(0.0, 0.3, x.shape), dtype)
    return d


@pytest.mark.parametrize("B,N", [(3, 5), (3, 300), (2, 2051)])
def test_anchor_gradients_fused_loss_fp64(cufk, device, B, N):
    """reconstruct_loss(..., anchor_grads=True): the oracle's anchor map applied to the loss's
    grad_xyz = 2 w (x - t), per-chain weights; every output within 1e-10."""
    d = _loss_case(B, N, seed=900 + N)
    w = np.linspace(0.5, 2.0, B)
    L, A, D = (_dev(d[k], torch.float64, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = [_dev(d[k], torch.float64, device, True) for k in ("p0", "first_direction", "initial_normal")]
    loss = cufk.reconstruct_loss(L, A, D, _dev(d["target"], torch.float64, device), *an, anchor_grads=True)
    got = torch.autograd.grad(loss, (L, A, D, *an), _dev(w, torch.float64, device))
    a = {k: d[k] for k in ("p0", "first_direction", "initial_normal")}
    x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **a)
    gx = 2.0 * w[:, None, None] * (x - d["target"])
    want = list(o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], gx, **a))
    want += list(o.anchor_gradients(d["lengths"], d["angles"], d["dihedrals"], gx, **a))
    for name, g, r in zip(("L", "A", "D", "p0", "fd", "n0"), got, want):
        err = np.abs(g.cpu().numpy() - r).max() / max(np.abs(r).max(), 1e-300)
        assert err <= 1e-10, (name, err)


def test_anchor_gradients_fused_loss_gradcheck(cufk, device):
    d = _loss_case(2, 12, seed=17)
    L, A, D = (_dev(d[k], torch.float64, device) for k in ("lengths", "angles", "dihedrals"))
    t = _dev(d["target"], torch.float64, device)
    an = tuple(_dev(d[k], torch.float64, device, True) for k in ("p0", "first_direction", "initial_normal"))
    assert torch.autograd.gradcheck(lambda p, f, n: cufk.reconstruct_loss(L, A, D, t, p, f, n, anchor_grads=True), an,
                                    eps=1e-6, atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("N,seg", [(300, 64), (700, 100), (2051, None)])
@pytest.mark.parametrize("modify", [False, True])
def test_anchor_gradients_long_chains_fp64(cufk, device, N, seg, modify):
    """reconstruct_long(..., anchor_grads=True) over several segments (the head segment writes
    the chain's sums), with the saved output and after an in-place change; within 1e-10."""
    d = _case(3, N, seed=950 + N)
    L, A, D = (_dev(d[k], torch.float64, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = [_dev(d[k], torch.float64, device, True) for k in ("p0", "first_direction", "initial_normal")]
    xyz = cufk.reconstruct_long(L, A, D, *an, segment_steps=seg, anchor_grads=True)
    if modify:
        xyz.mul_(1.0)
    got = torch.autograd.grad(xyz, (L, A, D, *an), _dev(d["grad"], torch.float64, device))
    for name, g, r in zip(("L", "A", "D", "p0", "fd", "n0"), got, _ref(d)):
        err = np.abs(g.cpu().numpy() - r).max() / max(np.abs(r).max(), 1e-300)
        assert err <= 1e-10, (name, err)


def test_anchor_gradients_long_chains_fp32_and_gradcheck(cufk, device):
    d = _case(4, 3000, seed=31, dtype=torch.float32)
    L, A, D = (_dev(d[k], torch.float32, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = [_dev(d[k], torch.float32, device, True) for k in ("p0", "first_direction", "initial_normal")]
    xyz = cufk.reconstruct_long(L, A, D, *an, segment_steps=512, anchor_grads=True)
    got = torch.autograd.grad(xyz, (L, A, D, *an), _dev(d["grad"], torch.float32, device))
    for name, g, r in list(zip(("L", "A", "D", "p0", "fd", "n0"), got, _ref(d)))[3:]:
        err = np.abs(g.double().cpu().numpy() - r).max() / np.abs(r).max()
        print(f"fp32 long anchor {name}: rel err {err:.2e}")
        assert err <= 5e-5, name
    e = _case(2, 23, seed=33)
    L, A, D = (_dev(e[k], torch.float64, device) for k in ("lengths", "angles", "dihedrals"))
    an = tuple(_dev(e[k], torch.float64, device, True) for k in ("p0", "first_direction", "initial_normal"))
    assert torch.autograd.gradcheck(
        lambda p, f, n: cufk.reconstruct_long(L, A, D, p, f, n, segment_steps=4, anchor_grads=True), an, eps=1e-6,
        atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("path", ["reconstruct", "loss", "long"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("B,N", [(3, 300), (5, 2051), (4133, 67)])
def test_anchored_backward_keeps_the_plain_gradients(cufk, device, path, dtype, B, N):
    """With anchor_grads=True the gradients of lengths, angles and dihedrals are those of the
    same call without it, bit for bit: the same kernels run, with a pointer for the anchor sums
    they then also write."""
    d = _case(B, N, seed=B + N, dtype=dtype)
    g = _dev(d["grad"], dtype, device)
    target = _dev(d["grad"], dtype, device)  # any (B, N, 3) row will do for the loss

    def grads(anchored):
        L, A, D = (_dev(d[k], dtype, device, True) for k in ("lengths", "angles", "dihedrals"))
        an = [_dev(d[k], dtype, device, anchored) for k in ("p0", "first_direction", "initial_normal")]
        if path == "reconstruct":
            out, w = cufk.reconstruct(L, A, D, *an, anchor_grads=anchored), g
        elif path == "loss":
            out, w = cufk.reconstruct_loss(L, A, D, target, *an, anchor_grads=anchored), None
        else:
            out, w = cufk.reconstruct_long(L, A, D, *an, segment_steps=96, anchor_grads=anchored), g
        if w is None:
            return torch.autograd.grad(out.sum(), (L, A, D))
        return torch.autograd.grad(out, (L, A, D), w)

    for a, b, name in zip(grads(True), grads(False), ("lengths", "angles", "dihedrals")):
        assert torch.equal(a, b), (path, name)

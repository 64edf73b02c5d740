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

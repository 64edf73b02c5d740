"""A first call under ``torch.inference_mode()`` must not break later calls that need gradients.

``reconstruct``, ``reconstruct_long``, ``reconstruct_loss`` and ``reconstruct_rmsd`` cache the
default anchor tensors per device and dtype, and every autograd Function saves the anchors
for the backward.  An anchor cached as an inference tensor would make every later
gradient-taking call raise 'Inference tensors cannot be saved for backward'.  Each case clears
the cache, makes the first call under inference mode, then takes gradients and checks them bit
for bit against the same call made with a cache built outside inference mode.
"""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import nerf64 as o

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cufk(device):
    import cufk_amd

    return cufk_amd


def _inputs(B, N, dtype, device):
    d = o.synthetic_inputs(B, N, 91, anchors=False)
    L, A, D = (torch.as_tensor(d[k]).to(device=device, dtype=dtype) for k in ("lengths", "angles", "dihedrals"))
    g = torch.as_tensor(d["grad"]).to(device=device, dtype=dtype)
    return L, A, D, g


def _call(cufk, kind, L, A, D, target):
    if kind == "reconstruct":
        return cufk.reconstruct(L, A, D)
    if kind == "long":
        return cufk.reconstruct_long(L, A, D, segment_steps=64)
    if kind == "loss":
        return cufk.reconstruct_loss(L, A, D, target)
    return cufk.reconstruct_rmsd(L, A, D, target)


def _grads(cufk, kind, L, A, D, g):
    params = [t.detach().clone().requires_grad_(True) for t in (L, A, D)]
    out = _call(cufk, kind, *params, g)
    weight = g if out.dim() == 3 else torch.ones_like(out)
    return torch.autograd.grad(out, params, weight)


@pytest.mark.parametrize("kind", ["reconstruct", "long", "loss", "rmsd"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_first_call_under_inference_mode(cufk, device, kind, dtype):
    module = sys.modules["cufk_amd.reconstruct"]  # the package's `reconstruct` is the function

    L, A, D, g = _inputs(5, 300, dtype, device)
    module._DEFAULT_ANCHORS.clear()
    want = _grads(cufk, kind, L, A, D, g)

    module._DEFAULT_ANCHORS.clear()
    with torch.inference_mode():
        first = _call(cufk, kind, L, A, D, g)
    assert first.is_inference()
    assert all(not t.is_inference() for t in module._DEFAULT_ANCHORS.values())
    got = _grads(cufk, kind, L, A, D, g)
    for a, b in zip(got, want):
        assert torch.equal(a, b)


BOND_LENGTHS = (0.14685231, 0.15365194, 0.13405086)
BOND_ANGLES = (1.9676635, 2.062335, 2.164016)


def _every_entry_point(cufk, dtype, device):
    L, A, D, g = _inputs(5, 300, dtype, device)
    raw = torch.as_tensor(o.synthetic_inputs(5, 300, 92)["grad"].reshape(5, -1)[:, : 2 * 297]).to(device, dtype)
    f = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    return {
        "reconstruct": lambda: cufk.reconstruct(L, A, D),
        "anchored": lambda: cufk.reconstruct(L, A, D, anchor_grads=True),
        "long": lambda: cufk.reconstruct_long(L, A, D, segment_steps=64),
        "long_anchored": lambda: cufk.reconstruct_long(L, A, D, segment_steps=64, anchor_grads=True),
        "loss": lambda: cufk.reconstruct_loss(L, A, D, g),
        "loss_anchored": lambda: cufk.reconstruct_loss(L, A, D, g, anchor_grads=True),
        "rmsd": lambda: cufk.reconstruct_rmsd(L, A, D, g),
        "torsion": lambda: f(raw),
        "torsion_loss": lambda: f.loss(raw, g),
        "torsion_rmsd": lambda: f.rmsd(raw, g),
    }


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
def test_every_entry_point_under_inference_mode(cufk, device, dtype):
    """Under inference mode every public call returns what it returns under no_grad."""
    calls = _every_entry_point(cufk, dtype, device)
    for name, call in calls.items():
        with torch.no_grad():
            want = call()
        with torch.inference_mode():
            got = call()
        assert got.is_inference(), name
        assert torch.equal(got, want), name

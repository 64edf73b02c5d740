"""Batches whose tensors pass 2^31 elements (about 37 GB per case, which a 288 GB MI355X holds):
every row offset in the kernels is 64-bit, so chains past element 2^31 of xyz must come out as
the first ones do.  Inputs are drawn on the device; the chains that straddle element 2^31 of
the (B, N, 3) output, the last chain and the first are checked against the float64 oracle
under the float32 bars (1e-5 nm RMS, 1e-4 nm max-abs; gradients 5e-5 relative per chain)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import nerf64 as o

pytestmark = pytest.mark.gpu


def _draw(B, N, device, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    L = (torch.randn(B, N - 1, generator=gen, device=device) * 0.01 + 0.145).clamp_(0.12, 0.17)
    A = torch.randn(B, N - 2, generator=gen, device=device) * 0.08 + 2.05
    D = (torch.rand(B, N - 3, generator=gen, device=device) * 2 - 1) * math.pi
    g = torch.randn(B, N, 3, generator=gen, device=device)
    return L, A, D, g


@pytest.mark.parametrize("B,N", [(1_500_000, 512), (12_000_000, 64)])
def test_batches_past_two_to_the_31_elements(device, B, N):
    import cufk_amd

    assert B * N * 3 > 2**31
    L, A, D, g = _draw(B, N, device, seed=B)
    an = {"p0": torch.tensor([0.3, -0.2, 0.1], device=device),
          "first_direction": torch.tensor([0.0, 0.6, 0.8], device=device),
          "initial_normal": torch.tensor([1.0, 0.0, 0.0], device=device)}
    Lr, Ar, Dr = (t.requires_grad_(True) for t in (L, A, D))
    xyz = cufk_amd.reconstruct(Lr, Ar, Dr, **an)
    grads = torch.autograd.grad(xyz, (Lr, Ar, Dr), g)
    torch.cuda.synchronize()
    edge = 2**31 // (3 * N)  # the chain holding element 2^31 of xyz
    rows = [0, edge - 1, edge, edge + 1, B - 1]
    anchors = {k: v.double().cpu().numpy() for k, v in an.items()}
    pick = lambda t: t.detach()[rows].double().cpu().numpy()  # noqa: E731
    ref = o.reconstruct_forward(pick(L), pick(A), pick(D), **anchors)
    ref_g = o.reconstruct_backward(pick(L), pick(A), pick(D), pick(g), **anchors)
    diff = pick(xyz) - ref
    rms = np.sqrt(np.mean(np.sum(diff**2, axis=-1), axis=1))
    mx = np.abs(diff).max(axis=(1, 2))
    print(f"B={B} N={N}: chains {rows}: RMS {rms}, max-abs {mx}")
    assert (rms <= 1e-5).all() and (mx <= 1e-4).all()
    for name, got, want in zip(("lengths", "angles", "dihedrals"), grads, ref_g):
        err = np.abs(pick(got) - want).max(axis=1) / np.abs(want).max(axis=1)
        print(f"  d/d{name}: per-chain rel err {err}")
        assert (err <= 5e-5).all()
    del xyz, grads, L, A, D, g, Lr, Ar, Dr
    torch.cuda.empty_cache()


def test_torsion_batch_past_two_to_the_31_elements(device):
    """The torsion path at 8M chains of 100 points (raw pairs with their row stride, xyz past
    2^31 elements; about 32 GB)."""
    import cufk_amd

    bond_lengths = (0.14685231, 0.15365194, 0.13405086)
    bond_angles = (1.9676635, 2.062335, 2.164016)
    B, N = 8_000_000, 100
    assert B * N * 3 > 2**31
    gen = torch.Generator(device=device).manual_seed(7)
    raw = torch.randn(B, 2 * (N - 3), generator=gen, device=device).requires_grad_(True)
    g = torch.randn(B, N, 3, generator=gen, device=device)
    xyz = cufk_amd.compile_torsion(bond_lengths, bond_angles)(raw)
    (graw,) = torch.autograd.grad(xyz, (raw,), g)
    torch.cuda.synchronize()
    edge = 2**31 // (3 * N)
    rows = [0, edge - 1, edge, edge + 1, B - 1]
    c = o.torsion_constants(bond_lengths, bond_angles)
    pick = lambda t: t.detach()[rows].double().cpu().numpy()  # noqa: E731
    ref = o.torsion_forward(pick(raw), c)
    ref_g = o.torsion_backward(pick(raw), ref, pick(g), c)
    diff = pick(xyz) - ref
    rms = np.sqrt(np.mean(np.sum(diff**2, axis=-1), axis=1))
    err = np.abs(pick(graw) - ref_g).max(axis=1) / np.abs(ref_g).max(axis=1)
    print(f"torsion B={B} N={N}: chains {rows}: RMS {rms}, max-abs {np.abs(diff).max():.2e}, grad rel {err}")
    assert (rms <= 1e-5).all() and np.abs(diff).max() <= 1e-4 and (err <= 5e-5).all()
    del xyz, graw, raw, g
    torch.cuda.empty_cache()

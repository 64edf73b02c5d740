"""Validation and API contract on the host (no GPU): the RuntimeError messages of the
reference's checks (extension_utils.cuh:57-130, block.cu:367-378, torsion.cu:413-417),
reached through the extension's validators with the device-type check switched off, plus
the public Python surface (reconstruct.py, torsion.py, __init__.py)."""

from __future__ import annotations

import pytest
import torch

import cufk_amd
from cufk_amd import _C
import importlib

rmod = importlib.import_module("cufk_amd.reconstruct")
tmod = importlib.import_module("cufk_amd.torsion")

BL = (0.14685231, 0.15365194, 0.13405086)
BA = (1.9676635, 2.062335, 2.164016)


def geom(B=2, N=10, dtype=torch.float32):
    return torch.zeros(B, N - 1, dtype=dtype), torch.zeros(B, N - 2, dtype=dtype), torch.zeros(B, N - 3, dtype=dtype)


def anchors(dtype=torch.float32):
    return torch.zeros(3, dtype=dtype), torch.tensor([1.0, 0, 0], dtype=dtype), torch.tensor([0, 0, 1.0], dtype=dtype)


def validate(L, A, D, p0=None, fd=None, n0=None):
    a = anchors(L.dtype if L.dtype.is_floating_point else torch.float32)
    return _C.validate_reconstruct(L, A, D, p0 if p0 is not None else a[0], fd if fd is not None else a[1],
                                   n0 if n0 is not None else a[2], device=False)


def test_public_surface():
    assert cufk_amd.__all__ == ["BLOCK_SCAN_MAX_POINT_COUNT", "__version__", "compile_torsion", "reconstruct"]
    assert cufk_amd.BLOCK_SCAN_MAX_POINT_COUNT == 2051
    assert callable(cufk_amd.reconstruct_long)  # extension, outside the reference's __all__
    assert cufk_amd.__version__ == "0.1.0"
    assert _C.library_version() == "0.1.0"


def test_valid_shapes_pass():
    assert validate(*geom(3, 10)) == [3, 10]
    assert validate(*geom(1, 4)) == [1, 4]
    assert validate(*geom(2, 2051)) == [2, 2051]
    for dt in (torch.float64, torch.float16, torch.bfloat16):
        L, A, D = geom(2, 8, dt)
        assert validate(L, A, D, *anchors(dt)) == [2, 8]


def test_host_tensors_are_rejected_by_the_public_api():
    L, A, D = geom()
    with pytest.raises(RuntimeError, match="lengths must be CUDA"):
        cufk_amd.reconstruct(L, A, D)
    with pytest.raises(RuntimeError, match="raw_pairs must be CUDA"):
        cufk_amd.compile_torsion(BL, BA)(torch.zeros(2, 8))


@pytest.mark.parametrize(
    "mutate, message",
    [
        (lambda L, A, D: (L.long(), A, D), "lengths must be float32, float64, float16, or bfloat16"),
        (lambda L, A, D: (L.t().contiguous().t() if L.shape[0] > 1 else L, A, D), "lengths must be contiguous"),
        (lambda L, A, D: (L, A.double(), D), "angles must have the same dtype as reference"),
        (lambda L, A, D: (L, A, D.double()), "dihedrals must have the same dtype as reference"),
        (lambda L, A, D: (L, A[:, ::2], D), "angles must be contiguous"),
        (lambda L, A, D: (L[0], A, D), r"lengths must have shape \(B, N-1\)"),
        (lambda L, A, D: (L, A[0], D), r"angles must have shape \(B, N-2\)"),
        (lambda L, A, D: (L, A, D[0]), r"dihedrals must have shape \(B, N-3\)"),
        (lambda L, A, D: (L, A[:, :-1].contiguous(), D), "bad angles shape"),
        (lambda L, A, D: (L, A, D[:1].contiguous()), "bad dihedrals shape"),
        (lambda L, A, D: (L[:, :2].contiguous(), A[:, :1].contiguous(), D[:, :0].contiguous()), "point_count must be >= 4"),
    ],
)
def test_geometry_messages(mutate, message):
    L, A, D = geom(3, 10)
    L = torch.arange(27, dtype=torch.float32).reshape(3, 9) if "contiguous" in message and "lengths" in message else L
    with pytest.raises(RuntimeError, match=message):
        validate(*mutate(L, A, D))


def test_lengths_contiguity_message():
    L = torch.zeros(9, 3).t()
    assert not L.is_contiguous()
    with pytest.raises(RuntimeError, match="lengths must be contiguous"):
        validate(L, torch.zeros(3, 8), torch.zeros(3, 7))


def test_step_cap_message():
    with pytest.raises(RuntimeError, match="reconstruct supports at most 2048 local transforms"):
        validate(*geom(1, 2052))
    with pytest.raises(RuntimeError, match="torsion_pairs supports at most 2048 local transforms"):
        _C.validate_torsion(torch.zeros(1, 2 * 2049), device=False)


@pytest.mark.parametrize("name", ["p0", "first_direction", "initial_normal"])
def test_anchor_messages(name):
    L, A, D = geom()
    good = dict(zip(("p0", "fd", "n0"), anchors()))
    key = {"p0": "p0", "first_direction": "fd", "initial_normal": "n0"}[name]
    bad = dict(good)
    bad[key] = torch.zeros(4)
    with pytest.raises(RuntimeError, match=rf"{name} must have shape \(3,\)"):
        validate(L, A, D, **bad)
    bad[key] = torch.zeros(3, dtype=torch.float64)
    with pytest.raises(RuntimeError, match=f"{name} must have the same dtype as reference"):
        validate(L, A, D, **bad)
    bad[key] = torch.zeros(3, requires_grad=True)
    with pytest.raises(RuntimeError, match=f"{name} gradients are not supported"):
        validate(L, A, D, **bad)


def test_grad_points_messages():
    L, _, _ = geom()
    _C.validate_grad_points(torch.zeros(2, 10, 3), L, device=False)
    with pytest.raises(RuntimeError, match="grad_points must have the same dtype as reference"):
        _C.validate_grad_points(torch.zeros(2, 10, 3, dtype=torch.float64), L, device=False)
    with pytest.raises(RuntimeError, match="grad_points must be CUDA"):
        _C.validate_grad_points(torch.zeros(2, 10, 3), L, device=True)


def test_torsion_messages():
    assert _C.validate_torsion(torch.zeros(5, 8), device=False) == [5, 7]
    with pytest.raises(RuntimeError, match=r"raw_pairs must have shape \(B, K\)"):
        _C.validate_torsion(torch.zeros(8), device=False)
    with pytest.raises(RuntimeError, match=r"raw_pairs must have stride\(1\) == 1"):
        _C.validate_torsion(torch.zeros(8, 4).t(), device=False)
    with pytest.raises(RuntimeError, match="raw_pairs second dimension must be even"):
        _C.validate_torsion(torch.zeros(2, 7), device=False)
    with pytest.raises(RuntimeError, match="raw_pairs must be float32, float64, float16, or bfloat16"):
        _C.validate_torsion(torch.zeros(2, 8, dtype=torch.int32), device=False)
    with pytest.raises(RuntimeError, match="point_count must be >= 4"):
        _C.validate_torsion(torch.zeros(2, 0), device=False)
    # Row stride is free (only stride(1) == 1 is required): a column slice validates.
    assert _C.validate_torsion(torch.zeros(3, 20)[:, 2:12], device=False) == [3, 8]


def test_compile_torsion_cache_and_constants():
    f1 = cufk_amd.compile_torsion(BL, BA)
    f2 = cufk_amd.compile_torsion(tuple(BL), tuple(BA))
    assert f1 is f2
    assert cufk_amd.compile_torsion(BL, (1.9, 2.0, 2.1)) is not f1
    module = tmod._TORSION_MODULES[(BL, BA)]
    import math

    import numpy as np

    assert module.lengths == [float(np.float32(v)) for v in BL]
    assert module.sin == [math.sin(a) for a in BA]
    assert module.cos == [math.cos(a) for a in BA]
    with pytest.raises(AssertionError, match="bond_lengths must have 3 elements"):
        cufk_amd.compile_torsion((0.1, 0.2), BA)
    with pytest.raises(AssertionError, match="bond_angles must have 3 elements"):
        cufk_amd.compile_torsion(BL, (1.0, 2.0, 3.0, 4.0))


def test_batching_and_default_anchors():
    L, A, D = torch.zeros(9), torch.zeros(8), torch.zeros(7)
    bl, ba, bd, single = rmod._batched_inputs(L, A, D)
    assert single and bl.shape == (1, 9) and ba.shape == (1, 8) and bd.shape == (1, 7)
    *_, single = rmod._batched_inputs(L[None], A[None], D[None])
    assert not single
    ref = torch.zeros(2, 9, dtype=torch.float64)
    a = rmod._anchor(None, (1.0, 0.0, 0.0), ref)
    assert a.dtype == torch.float64 and a.tolist() == [1.0, 0.0, 0.0]
    given = torch.ones(3)
    assert rmod._anchor(given, (0.0, 0.0, 0.0), ref) is given
    # Defaults are built once per device, dtype and value, and keep their values.
    assert rmod._anchor(None, (1.0, 0.0, 0.0), ref) is a
    b = rmod._anchor(None, (0.0, 0.0, 1.0), ref)
    assert b is not a and b.tolist() == [0.0, 0.0, 1.0] and not b.requires_grad
    c = rmod._anchor(None, (1.0, 0.0, 0.0), ref.float())
    assert c.dtype == torch.float32 and c.tolist() == [1.0, 0.0, 0.0]


def test_default_anchor_made_under_inference_mode_is_a_normal_tensor():
    # The cached default is saved for backward by later calls that record one; an inference
    # tensor cannot be.
    ref = torch.zeros(2, 9, dtype=torch.float16)
    rmod._DEFAULT_ANCHORS.clear()
    with torch.inference_mode():
        a = rmod._anchor(None, (0.0, 1.0, 0.0), ref)
    assert not a.is_inference() and a.tolist() == [0.0, 1.0, 0.0]
    assert rmod._anchor(None, (0.0, 1.0, 0.0), ref) is a
    rmod._DEFAULT_ANCHORS.clear()


def test_max_steps():
    # 2048 on a present gfx950 device; this host may have none (then the device check fails).
    for dtype in range(4):
        for direction in range(2):
            assert _C.max_steps(dtype, direction, 0) in (2048, -8)
            assert _C.max_steps(dtype, direction, -1) == -8
    assert _C.max_steps(7, 0, 0) == -1
    assert _C.max_steps(0, 5, 0) == -12

"""Short chains packed several per wave (chains of at most 128 steps, batches of at least
4096 chains: forward; at most 64 steps: backward) against the float64 oracle.

Batch sizes leave the last workgroup partly empty; every lanes-per-chain plan (1, 2, 4, 8 and
16 lanes of 8 steps) is covered, with bars as for the single-chain kernels: float64 1e-12
relative forward and 1e-10 relative gradients; float32 1e-5 nm RMS and 1e-4 nm max forward
and 5e-5 relative gradients; float16/bfloat16 reported with sanity bounds.  Below the batch
threshold the same shapes take one workgroup per chain, so every comparison runs both.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import nerf64 as o

pytestmark = pytest.mark.gpu

BIG = 4096 + 37  # past the packing threshold; not a multiple of any workgroup's chain count


@pytest.fixture(scope="module")
def cufk(device):
    import cufk_amd

    return cufk_amd


@pytest.fixture(scope="module")
def lib(device):
    import cufk_amd

    lib = ctypes.CDLL(str(cufk_amd._native.HIP_LIBRARY))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.cufk_reconstruct_fwd.argtypes = [ctypes.c_int] + [vp] * 7 + [i64, i64, vp]
    lib.cufk_reconstruct_fwd_flagged.argtypes = [ctypes.c_int] + [vp] * 8 + [i64, i64, vp]
    lib.cufk_reconstruct_bwd.argtypes = [ctypes.c_int] + [vp] * 10 + [i64, i64, vp]
    lib.cufk_reconstruct_bwd_saved.argtypes = [ctypes.c_int] + [vp] * 12 + [i64, i64, vp]
    return lib


CODES = {torch.float32: 0, torch.float64: 1, torch.float16: 2, torch.bfloat16: 3}


def _dev(x, dtype, device, requires_grad=False):
    t = torch.as_tensor(np.asarray(x), dtype=torch.float64).to(device=device, dtype=dtype)
    return t.requires_grad_(requires_grad)


def _round(x, dtype):
    return torch.as_tensor(np.asarray(x), dtype=torch.float64).to(dtype).double().numpy()


def _inputs(B, N, seed, dtype=torch.float64):
    d = o.synthetic_inputs(B, N, seed, anchors=True)
    return {k: _round(v, dtype) for k, v in d.items()}


def _anchor_np(d):
    return {k: d[k] for k in ("p0", "first_direction", "initial_normal")}


def _abi_run(lib, d, dtype, device, recompute=False):
    """Forward (flagged) and backward through the C ABI: the saved-output backward, or the
    one that recomputes the positions."""
    L, A, D, g = (_dev(d[k], dtype, device) for k in ("lengths", "angles", "dihedrals", "grad"))
    an = [_dev(d[k], dtype, device) for k in ("p0", "first_direction", "initial_normal")]
    B, N = L.shape[0], L.shape[1] + 1
    xyz = torch.empty(B, N, 3, device=device, dtype=dtype)
    reg = torch.full((B,), 7, device=device, dtype=torch.uint8)
    gL, gA, gD = (torch.empty_like(t) for t in (L, A, D))
    p = lambda t: t.data_ptr()  # noqa: E731
    st = torch.cuda.current_stream().cuda_stream
    c = CODES[dtype]
    assert lib.cufk_reconstruct_fwd_flagged(c, p(L), p(A), p(D), *map(p, an), p(xyz), p(reg), B, N, st) == 0
    if recompute:
        assert lib.cufk_reconstruct_bwd(c, p(L), p(A), p(D), *map(p, an), p(g), p(gL), p(gA), p(gD), B, N, st) == 0
    else:
        assert lib.cufk_reconstruct_bwd_saved(c, p(L), p(A), p(D), *map(p, an), p(xyz), p(reg), p(g), p(gL), p(gA),
                                              p(gD), B, N, st) == 0
    torch.cuda.synchronize()
    return xyz, reg, (gL, gA, gD)


# points -> steps: 1, 2, 8, 9, 16, 17, 32, 33, 64, 65, 128 (every lanes-per-chain plan and its edges)
POINTS = [4, 5, 11, 12, 19, 20, 35, 36, 67, 68, 131]


@pytest.mark.parametrize("N", POINTS)
@pytest.mark.parametrize("recompute", [False, True])
def test_packed_fp64_matches_oracle(lib, device, N, recompute):
    d = _inputs(BIG, N, seed=200 + N)
    xyz, reg, grads = _abi_run(lib, d, torch.float64, device, recompute)
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    err = np.abs(xyz.cpu().numpy() - ref).max()
    assert err <= 1e-12 * max(1.0, np.abs(ref).max()), err
    assert reg.cpu().min() == 1  # every synthetic chain is regular
    ref_g = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for got, want in zip(grads, ref_g):
        gerr = np.abs(got.cpu().numpy() - want).max() / np.abs(want).max()
        assert gerr <= 1e-10, gerr


@pytest.mark.parametrize("N", [12, 36, 68, 131])
def test_packed_fp32_tolerance(cufk, device, N):
    d = _inputs(BIG, N, seed=300 + N, dtype=torch.float32)
    L, A, D = (_dev(d[k], torch.float32, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = {k: _dev(d[k], torch.float32, device) for k in ("p0", "first_direction", "initial_normal")}
    xyz = cufk.reconstruct(L, A, D, **an)
    grads = torch.autograd.grad(xyz, (L, A, D), _dev(d["grad"], torch.float32, device))
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    diff = xyz.detach().double().cpu().numpy() - ref
    rms = math.sqrt(np.mean(np.sum(diff**2, axis=-1)))
    print(f"fp32 packed N={N}: rms {rms:.3e} nm, max {np.abs(diff).max():.3e} nm")
    assert rms <= 1e-5 and np.abs(diff).max() <= 1e-4
    ref_g = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for got, want in zip(grads, ref_g):
        gerr = np.abs(got.double().cpu().numpy() - want).max(axis=1) / np.abs(want).max(axis=1)
        assert gerr.max() <= 5e-5, gerr.max()


def test_packed_chains_are_independent(cufk, device):
    """A chain's packed forward does not depend on its neighbours: shifting the batch by one
    chain moves every chain to another slot of its workgroup (or to the next workgroup) and
    leaves its coordinates bit-identical.  Reconstructed alone (one chain per workgroup, a
    different lane partition) it agrees within float rounding."""
    for N in (5, 20, 36, 131):
        d = _inputs(BIG, N, seed=7, dtype=torch.float32)
        L, A, D = (_dev(d[k], torch.float32, device) for k in ("lengths", "angles", "dihedrals"))
        an = {k: _dev(d[k], torch.float32, device) for k in ("p0", "first_direction", "initial_normal")}
        packed = cufk.reconstruct(L, A, D, **an)
        shifted = cufk.reconstruct(*(torch.roll(t, 1, dims=0) for t in (L, A, D)), **an)
        assert torch.equal(torch.roll(shifted, -1, dims=0), packed), N
        for b in (0, 1, 63, 64, 127, 128, BIG - 1):
            alone = cufk.reconstruct(L[b : b + 1], A[b : b + 1], D[b : b + 1], **an)
            assert torch.allclose(alone[0], packed[b], rtol=0, atol=2e-6), (N, b)


@pytest.mark.parametrize("recompute", [False, True])
def test_packed_irregular_chains_take_the_exact_adjoint(lib, device, recompute):
    """Irregular chains (negative bond, tiny bond angle, zero bond) send their workgroup to the
    exact adjoint; regular workgroups keep the position-based one.  Both agree with the oracle."""
    N = 36
    d = _inputs(BIG, N, seed=17, dtype=torch.float32)
    d["lengths"][5, 7] *= -1
    d["angles"][700, 12] = 0.05
    d["lengths"][2000, 1] = 0.0
    d = {k: _round(v, torch.float32) for k, v in d.items()}
    xyz, reg, grads = _abi_run(lib, d, torch.float32, device, recompute)
    flags = reg.cpu().numpy()
    assert flags[5] == 0 and flags[700] == 0 and flags[2000] == 0 and flags.sum() == BIG - 3
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    assert np.abs(xyz.double().cpu().numpy() - ref).max() <= 1e-4
    ref_g = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for got, want in zip(grads, ref_g):
        err = np.abs(got.double().cpu().numpy() - want).max(axis=1) / np.maximum(np.abs(want).max(axis=1), 1e-30)
        print("worst per-chain grad rel err", err.max(), "at", err.argmax())
        assert err.max() <= 5e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_packed_angles_beyond_the_polynomial_range(lib, device, dtype):
    N = 20
    d = _inputs(BIG, N, seed=19, dtype=dtype)
    d["dihedrals"][3, 5] += 2 * math.pi * 20000.0
    d["angles"][3000, 16] = -1.0e6
    d = {k: _round(v, dtype) for k, v in d.items()}
    xyz, _, grads = _abi_run(lib, d, dtype, device)
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    err = np.abs(xyz.double().cpu().numpy() - ref).max() / np.abs(ref).max()
    print(f"{dtype} packed wide angles: forward rel max err {err:.3e}")
    assert err <= (1e-5 if dtype == torch.float32 else 2e-2)
    ref_g = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for got, want in zip(grads, ref_g):
        gerr = np.abs(got.double().cpu().numpy() - want).max() / np.abs(want).max()
        assert gerr <= (5e-5 if dtype == torch.float32 else 5e-2), gerr


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N", [12, 68])
def test_packed_low_precision_reported(lib, device, dtype, N):
    d = _inputs(BIG, N, seed=23, dtype=dtype)
    xyz, reg, grads = _abi_run(lib, d, dtype, device)
    assert reg.cpu().max() == 0  # half types are never flagged regular
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    rel = np.abs(xyz.double().cpu().numpy() - ref).max() / np.abs(ref).max()
    ref_g = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    gerr = [float(np.abs(g.double().cpu().numpy() - r).max() / np.abs(r).max()) for g, r in zip(grads, ref_g)]
    print(f"{dtype} packed N={N}: forward rel max {rel:.2e}, grads " + ", ".join(f"{e:.2e}" for e in gerr))
    assert torch.isfinite(xyz).all() and rel <= 1e-2 and max(gerr) <= 3e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
def test_packed_unaligned_storage(lib, device, dtype):
    """Rows starting one element past a 16-byte boundary stream through the same windows:
    outputs bit-identical to those from aligned buffers."""
    N = 20
    d = _inputs(BIG, N, seed=29, dtype=dtype)

    def shifted(x):
        t = torch.as_tensor(np.asarray(x), dtype=torch.float64).to(dtype)
        buf = torch.zeros(t.numel() + 16, dtype=dtype, device=device)
        v = buf[1 : 1 + t.numel()].view(t.shape)
        v.copy_(t.to(device))
        assert v.data_ptr() % 16 != 0
        return v

    outs = []
    for make in (lambda x: _dev(x, dtype, device), shifted):
        L, A, D, g = (make(d[k]) for k in ("lengths", "angles", "dihedrals", "grad"))
        an = [_dev(d[k], dtype, device) for k in ("p0", "first_direction", "initial_normal")]
        B = L.shape[0]
        xyz = make(np.zeros((B, N, 3)))
        gL, gA, gD = (make(np.zeros(t.shape)) for t in (L, A, D))
        p = lambda t: t.data_ptr()  # noqa: E731
        st = torch.cuda.current_stream().cuda_stream
        c = CODES[dtype]
        assert lib.cufk_reconstruct_fwd(c, p(L), p(A), p(D), *map(p, an), p(xyz), B, N, st) == 0
        assert lib.cufk_reconstruct_bwd(c, p(L), p(A), p(D), *map(p, an), p(g), p(gL), p(gA), p(gD), B, N, st) == 0
        torch.cuda.synchronize()
        outs.append([t.clone() for t in (xyz, gL, gA, gD)])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


# ----------------------------------------------------------------- plans chosen by batch and length
#
# One chain per workgroup for 257..1024 steps takes two kinds of plan, picked by the grid's size:
# small grids (at most 4096 waves under the eight-item plan) take twice the waves at four items
# per lane, larger grids eight items per lane.  No plan leaves a wave without steps, so 513..768
# steps take three waves of four and 1025..1536 three waves of eight.  Each (batch, length) below
# sits on one side of one of those lines, at a plan edge.


_PLAN_CASES = {}


def _plan_case(B, N):
    """Inputs and the oracle's forward and gradients, computed once per shape."""
    if (B, N) not in _PLAN_CASES:
        d = _inputs(B, N, seed=600 + N + B)
        ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
        ref_g = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
        _PLAN_CASES.clear()
        _PLAN_CASES[(B, N)] = (d, ref, ref_g)
    return _PLAN_CASES[(B, N)]


@pytest.mark.parametrize("recompute", [False, True])
@pytest.mark.parametrize("B,N", [(1024, 260), (1024, 384), (1024, 515), (4097, 260), (4097, 515),
                                 (1024, 516), (1024, 700), (1024, 771), (1024, 772), (2048, 1027), (2049, 516),
                                 (2049, 1027), (512, 1028), (512, 1539), (512, 1540)])
def test_plans_by_batch_fp64(lib, device, B, N, recompute):
    """float64 forward within 1e-12 and gradients within 1e-10 of the oracle on every chain."""
    d, ref, ref_g = _plan_case(B, N)
    xyz, reg, grads = _abi_run(lib, d, torch.float64, device, recompute)
    assert np.abs(xyz.cpu().numpy() - ref).max() <= 1e-12 * max(1.0, np.abs(ref).max())
    assert reg.cpu().min() == 1
    for got, want in zip(grads, ref_g):
        assert np.abs(got.cpu().numpy() - want).max() <= 1e-10 * np.abs(want).max()


@pytest.mark.parametrize("B,N", [(1024, 384), (4097, 384), (1024, 700), (1024, 1027), (2049, 1027), (512, 1200)])
def test_plans_by_batch_fp32(cufk, device, B, N):
    """float32 through the autograd path: 1e-5 nm RMS and 1e-4 nm max forward, gradients 5e-5
    relative (normwise per chain)."""
    d = _inputs(B, N, seed=650 + N, dtype=torch.float32)
    L, A, D = (_dev(d[k], torch.float32, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = {k: _dev(d[k], torch.float32, device) for k in ("p0", "first_direction", "initial_normal")}
    xyz = cufk.reconstruct(L, A, D, **an)
    grads = torch.autograd.grad(xyz, (L, A, D), _dev(d["grad"], torch.float32, device))
    ref = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **_anchor_np(d))
    diff = xyz.detach().double().cpu().numpy() - ref
    rms = math.sqrt(np.mean(np.sum(diff**2, axis=-1)))
    print(f"fp32 B={B} N={N}: rms {rms:.3e} nm, max {np.abs(diff).max():.3e} nm")
    assert rms <= 1e-5 and np.abs(diff).max() <= 1e-4
    ref_g = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **_anchor_np(d))
    for got, want in zip(grads, ref_g):
        gerr = np.abs(got.double().cpu().numpy() - want).max(axis=1) / np.abs(want).max(axis=1)
        assert gerr.max() <= 5e-5, gerr.max()

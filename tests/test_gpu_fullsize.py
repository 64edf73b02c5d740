"""Every chain of the benchmark configurations at full size, and the committed fixtures, on the GPU.

The float64 checker for full batches is oracle/cpu_torch.py (the reference algorithm in
PyTorch float64, pinned to oracle/nerf64.py in tests/test_oracle.py) run on the device: a serial
NeRF forward and the explicit world-frame reverse adjoint.  Bars:
* float32 coordinates: RMS <= 1e-5 nm over the batch and max-abs <= 1e-4 nm on every chain
  against float64 on the same (float32-valued) inputs, at N = 2049 for C2 and N = 771 for C3;
* float32 gradients: per chain max |g - ref| <= 5e-5 * max|ref| (normwise per chain and output);
* the internal-coordinate round trip of every float32 chain, measured in float64 on the
  device: bond lengths, bond angles and dihedrals recovered from the stored coordinates agree
  with the inputs within what float32 rounding at the chain's extent allows (derived in
  `_check_roundtrip`);
* float64 at the C2 and C3 shapes: coordinates within 1e-12 nm and gradients within 1e-10
  relative on every chain;
* float16/bfloat16 (C4): reported, held to sanity bounds;
* the extension bench configurations, short chains (131072 x 64) and long chains (64 x 131075),
  every chain: coordinates, round trip and gradients (derived in the tests);
* the fused losses (coordinate loss, superposed RMSD and mean squared deviation) at the C2 and
  C3 shapes: loss per chain within 1e-5 relative, gradients per chain against the float64
  adjoint over the stored positions (derived in `_check_fused`).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import cpu_torch as ct
from oracle import nerf64 as o

pytestmark = pytest.mark.gpu

BOND_LENGTHS = (0.14685231, 0.15365194, 0.13405086)
BOND_ANGLES = (1.9676635, 2.062335, 2.164016)


@pytest.fixture(scope="module")
def cufk(device):
    import cufk_amd

    return cufk_amd


def _synthetic(B, N, seed, device):
    """The benchmark draws (float64 on the CPU, then moved): lengths ~N(0.145, 0.01) clipped to
    [0.12, 0.17], angles ~N(2.05, 0.08), dihedrals ~U(-pi, pi), grad ~N(0, 1), random anchors."""
    gen = torch.Generator().manual_seed(seed)
    L = (torch.randn(B, N - 1, generator=gen, dtype=torch.float64) * 0.01 + 0.145).clamp_(0.12, 0.17)
    A = torch.randn(B, N - 2, generator=gen, dtype=torch.float64) * 0.08 + 2.05
    D = (torch.rand(B, N - 3, generator=gen, dtype=torch.float64) * 2 - 1) * math.pi
    g = torch.randn(B, N, 3, generator=gen, dtype=torch.float64)
    p0 = torch.randn(3, generator=gen, dtype=torch.float64)
    q, _ = torch.linalg.qr(torch.randn(3, 3, generator=gen, dtype=torch.float64))
    return [t.to(device) for t in (L, A, D, g, p0, q[:, 0].contiguous(), q[:, 1].contiguous())]


def _internal(x):
    """Bond lengths, interior angles and IUPAC dihedrals of (B, N, 3) float64 positions
    (oracle/nerf64.py measure_internal, in torch)."""
    b = x[:, 1:] - x[:, :-1]
    L = b.norm(dim=-1)
    u, w = -b[:, :-1], b[:, 1:]
    A = torch.atan2(torch.linalg.cross(u, w).norm(dim=-1), (u * w).sum(-1))
    b1, b2, b3 = b[:, :-2], b[:, 1:-1], b[:, 2:]
    n1, n2 = torch.linalg.cross(b1, b2), torch.linalg.cross(b2, b3)
    D = torch.atan2(b2.norm(dim=-1) * (b1 * n2).sum(-1), (n1 * n2).sum(-1))
    return L, A, D


def _wrap(a):
    return torch.remainder(a + math.pi, 2 * math.pi) - math.pi


ROUNDTRIP_KAPPA = 32.0


def _check_roundtrip(xyz, L, A, D, label):
    """Internal coordinates recovered from the stored float32 positions, in float64.

    With h = 2^-24 * (the chain's largest |coordinate|), half an ulp of the chain's extent,
    a chain's bonds may move by kappa * h and its angles and dihedrals by kappa * h / (its
    shortest bond), kappa = 32.  Every stored coordinate is rounded once (h), and the float
    cross-lane scan rounds the running translation by up to about an ulp of the extent at each
    of its compositions (six DPP levels and the cross-wave carry), differently for adjacent
    lanes, so a bond across a lane boundary sees a few tens of h at most; points within a lane
    share one carry.  Angles and dihedrals turn a displacement into an angle over a bond
    length (sin theta >= 0.5 here).  A misplaced atom or a wrong carry moves them by orders
    of magnitude more (0.1 nm, a whole rotation)."""
    Lm, Am, Dm = _internal(xyz.double())
    h = 2.0**-24 * xyz.float().abs().amax(dim=(1, 2)).double()  # (B,)
    lmin = L.amin(dim=1)
    rL = (Lm - L).abs().amax(dim=1) / h
    rA = (Am - A).abs().amax(dim=1) * lmin / h
    rD = _wrap(Dm - D).abs().amax(dim=1) * lmin / h
    print(f"{label} round trip, worst chain in units of h (bonds) and h / shortest bond (angles): "
          f"bond {rL.max():.2f}, angle {rA.max():.2f}, dihedral {rD.max():.2f} (kappa {ROUNDTRIP_KAPPA})")
    assert float(rL.max()) <= ROUNDTRIP_KAPPA
    assert float(rA.max()) <= ROUNDTRIP_KAPPA
    assert float(rD.max()) <= ROUNDTRIP_KAPPA


def _check_coordinates(xyz, ref, label):
    """The float32 coordinate bar over the whole batch (1e-5 nm RMS) and on every chain
    (1e-4 nm max-abs); the worst chain's own RMS is reported and held to 2e-5 nm, which a
    garbled or misplaced chain exceeds by orders of magnitude."""
    diff = xyz.double() - ref
    rms_all = float(diff.pow(2).sum(-1).mean().sqrt())
    rms = diff.pow(2).sum(-1).mean(1).sqrt()
    mx = diff.abs().amax(dim=(1, 2))
    print(f"{label} every chain: RMS {rms_all:.2e} nm over the batch, worst chain RMS {rms.max():.2e} nm, "
          f"worst max-abs {mx.max():.2e} nm")
    assert rms_all <= 1e-5
    assert bool((mx <= 1e-4).all()) and bool((rms <= 2e-5).all())


def _per_chain_rel(got, want):
    """max |got - want| / max |want| for every chain (rows of a (B, ...) tensor)."""
    d = (got.double() - want).abs().flatten(1).amax(dim=1)
    return d / want.abs().flatten(1).amax(dim=1)


def test_config2_every_chain(cufk, device):
    """C2 (B = 4096, N = 2049, float32, random anchors), every chain: coordinates, the
    internal-coordinate round trip, and the three gradients of the autograd step."""
    B, N = 4096, 2049
    L, A, D, g, p0, fd, n0 = _synthetic(B, N, 2, device)
    f32 = [t.float() for t in (L, A, D, g, p0, fd, n0)]
    Lf, Af, Df = (t.clone().requires_grad_(True) for t in f32[:3])
    xyz = cufk.reconstruct(Lf, Af, Df, *f32[4:])
    grads = torch.autograd.grad(xyz, (Lf, Af, Df), f32[3])
    L64, A64, D64, g64 = (t.double() for t in f32[:4])  # float64 values of the float32 inputs
    an64 = [t.double() for t in f32[4:]]
    ref = ct.forward(L64, A64, D64, *an64)
    _check_coordinates(xyz.detach(), ref, "C2")
    _check_roundtrip(xyz.detach(), L64, A64, D64, "C2")
    want = ct.backward(ref, g64)
    for name, got, w in zip(("lengths", "angles", "dihedrals"), grads, want):
        err = _per_chain_rel(got, w)
        print(f"C2 every chain d/d{name}: worst per-chain rel err {err.max():.2e} (chain {int(err.argmax())})")
        assert bool((err <= 5e-5).all())


def test_config2_fp64_every_chain(cufk, device):
    """The C2 shape in float64 (B = 4096, N = 2049, random anchors), every chain: coordinates
    within 1e-12 nm of the serial float64 walk (the lane scans, wave scans and carries of the
    kernel associate the same products differently, about 1e-13 at this extent), gradients
    within 1e-10 relative per chain of the float64 adjoint."""
    B, N = 4096, 2049
    L, A, D, g, p0, fd, n0 = _synthetic(B, N, 22, device)
    Lr, Ar, Dr = (t.clone().requires_grad_(True) for t in (L, A, D))
    xyz = cufk.reconstruct(Lr, Ar, Dr, p0, fd, n0)
    grads = torch.autograd.grad(xyz, (Lr, Ar, Dr), g)
    ref = ct.forward(L, A, D, p0, fd, n0)
    err = (xyz.detach() - ref).abs().amax(dim=(1, 2))
    print(f"C2 fp64 every chain: worst max-abs {err.max():.2e} nm (chain {int(err.argmax())})")
    assert bool((err <= 1e-12).all())
    _check_gradients("C2 fp64", grads, ct.backward(ref, g), 1e-10)


def test_config3_fp64_every_chain(cufk, device):
    """The C3 torsion shape in float64 (B = 8192, N = 771), every chain: coordinates within
    1e-12 nm of the float64 torsion restatement, raw-pair gradients within 1e-10 relative per
    chain of its adjoint."""
    B, N = 8192, 771
    gen = torch.Generator().manual_seed(33)
    raw64 = torch.randn(B, 2 * (N - 3), generator=gen, dtype=torch.float64).to(device)
    g64 = torch.randn(B, N, 3, generator=gen, dtype=torch.float64).to(device)
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    raw = raw64.clone().requires_grad_(True)
    xyz = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)(raw)
    (graw,) = torch.autograd.grad(xyz, (raw,), g64)
    ref = ct.torsion_forward(raw64, c.lengths, c.sin, c.cos)
    err = (xyz.detach() - ref).abs().amax(dim=(1, 2))
    print(f"C3 fp64 every chain: worst max-abs {err.max():.2e} nm (chain {int(err.argmax())})")
    assert bool((err <= 1e-12).all())
    gerr = _per_chain_rel(graw, ct.torsion_backward(raw64, ref, g64, c.lengths))
    print(f"C3 fp64 every chain d/draw: worst per-chain rel err {gerr.max():.2e}")
    assert bool((gerr <= 1e-10).all())


def test_config3_every_chain(cufk, device):
    """C3 torsion (B = 8192, N = 771, float32), every chain: coordinates against the float64
    torsion restatement, the round trip of bond lengths and angles against the compiled
    constants and of dihedrals against atan2 of the pairs, and the raw-pair gradients."""
    B, N = 8192, 771
    gen = torch.Generator().manual_seed(3)
    raw64 = torch.randn(B, 2 * (N - 3), generator=gen, dtype=torch.float64).float().double().to(device)
    g64 = torch.randn(B, N, 3, generator=gen, dtype=torch.float64).float().double().to(device)
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    raw = raw64.float().requires_grad_(True)
    xyz = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)(raw)
    (graw,) = torch.autograd.grad(xyz, (raw,), g64.float())
    ref = ct.torsion_forward(raw64, c.lengths, c.sin, c.cos)
    _check_coordinates(xyz.detach(), ref, "C3")
    k = torch.arange(N - 1, device=device)
    L = torch.tensor(c.lengths, dtype=torch.float64, device=device)[k % 3].expand(B, N - 1)
    ang = torch.tensor([math.atan2(s, cc) for s, cc in zip(c.sin, c.cos)], dtype=torch.float64, device=device)
    A = ang[torch.arange(N - 2, device=device) % 3].expand(B, N - 2)
    D = torch.atan2(raw64[:, 0::2], raw64[:, 1::2])
    _check_roundtrip(xyz.detach(), L, A, D, "C3")
    # The torsion backward takes the saved forward output (torsion.cu:297-381 reads xyz), so its
    # parity is against the float64 adjoint over those stored positions; against the float64
    # chain it also carries the forward's position error, which the world-frame moments
    # multiply by the chain's extent (reported, 2e-4).
    kernel = _per_chain_rel(graw, ct.torsion_backward(raw64, xyz.detach().double(), g64, c.lengths))
    chain = _per_chain_rel(graw, ct.torsion_backward(raw64, ref, g64, c.lengths))
    print(f"C3 every chain d/draw: worst per-chain rel err {kernel.max():.2e} against the adjoint over the stored "
          f"positions (chain {int(kernel.argmax())}), {chain.max():.2e} against the float64 chain")
    assert bool((kernel <= 5e-5).all())
    assert bool((chain <= 2e-4).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_config4_every_chain_reported(cufk, device, dtype):
    """C4 (B = 16384, N = 1026), every chain: forward and gradients against float64 on the same
    rounded inputs.  Reported; held to the half-type sanity bounds (1e-2 relative forward,
    3e-2 relative gradients per chain), which a misplaced or garbled chain exceeds by orders
    of magnitude."""
    B, N = 16384, 1026
    L, A, D, g, p0, fd, n0 = _synthetic(B, N, 4, device)
    h = [t.to(dtype) for t in (L, A, D, g, p0, fd, n0)]
    Lh, Ah, Dh = (t.clone().requires_grad_(True) for t in h[:3])
    xyz = cufk.reconstruct(Lh, Ah, Dh, *h[4:])
    grads = torch.autograd.grad(xyz, (Lh, Ah, Dh), h[3])
    L64, A64, D64, g64 = (t.double() for t in h[:4])
    ref = ct.forward(L64, A64, D64, *(t.double() for t in h[4:]))
    rel = _per_chain_rel(xyz.detach(), ref)
    diff = xyz.detach().double() - ref
    rms_pos = diff.pow(2).sum(-1).mean(0).sqrt()
    marks = [round(i * (N - 1) / 10) for i in range(11)]
    print(f"C4 {dtype} every chain: worst rel max {rel.max():.2e}; RMS by position "
          + ", ".join(f"{i}: {float(rms_pos[i]):.1e}" for i in marks))
    assert bool(torch.isfinite(xyz).all()) and bool((rel <= 1e-2).all())
    want = ct.backward(ref, g64)
    for name, got, w in zip(("lengths", "angles", "dihedrals"), grads, want):
        err = _per_chain_rel(got, w)
        print(f"C4 {dtype} d/d{name}: worst per-chain rel err {err.max():.2e}")
        assert bool(torch.isfinite(got).all()) and bool((err <= 3e-2).all())


# ----------------------------------------------------------------- extension configurations


def _check_gradients(label, grads, want, bar):
    for name, got, w in zip(("lengths", "angles", "dihedrals"), grads, want):
        err = _per_chain_rel(got, w)
        print(f"{label} every chain d/d{name}: worst per-chain rel err {err.max():.2e} (chain {int(err.argmax())})")
        assert bool(torch.isfinite(got).all()) and bool((err <= bar).all())


def test_short_config_every_chain(cufk, device):
    """The short-chain bench configuration (B = 131072, N = 64, float32, random anchors: the
    packed kernels, several chains per wave), every chain: coordinates and round trip under the
    C2 bars, gradients within 5e-5 per chain."""
    B, N = 131072, 64
    L, A, D, g, p0, fd, n0 = _synthetic(B, N, 5, device)
    f32 = [t.float() for t in (L, A, D, g, p0, fd, n0)]
    Lf, Af, Df = (t.clone().requires_grad_(True) for t in f32[:3])
    xyz = cufk.reconstruct(Lf, Af, Df, *f32[4:])
    grads = torch.autograd.grad(xyz, (Lf, Af, Df), f32[3])
    L64, A64, D64, g64 = (t.double() for t in f32[:4])
    ref = ct.forward(L64, A64, D64, *(t.double() for t in f32[4:]))
    _check_coordinates(xyz.detach(), ref, "short")
    _check_roundtrip(xyz.detach(), L64, A64, D64, "short")
    _check_gradients("short", grads, ct.backward(ref, g64), 5e-5)


def test_long_config_every_chain(cufk, device):
    """The long-chain bench configuration (B = 64, N = 131075, float32, random anchors: 64
    segments of 2048 steps per chain), every chain.  Coordinates: the single-workgroup bars
    scaled with the chain length, as for every long chain (1e-5 nm RMS and 1e-4 nm max-abs per
    2049 points: 6.4e-4 and 6.4e-3 nm here; the float scan's rounding drifts along the chain).
    The internal-coordinate round trip holds at the chain's own rounding scale, which the drift
    does not enter: each bond, angle and dihedral is placed by one segment's float transform.
    Gradients: within 5e-5 per chain of the float64 adjoint over the float64 chain, the
    single-workgroup bar (the backward runs the position-based adjoint over each segment's
    local positions, which stay within the segment's extent of its origin)."""
    B, N = 64, 131075
    L, A, D, g, p0, fd, n0 = _synthetic(B, N, 6, device)
    f32 = [t.float() for t in (L, A, D, g, p0, fd, n0)]
    Lf, Af, Df = (t.clone().requires_grad_(True) for t in f32[:3])
    xyz = cufk.reconstruct_long(Lf, Af, Df, *f32[4:])
    grads = torch.autograd.grad(xyz, (Lf, Af, Df), f32[3])
    L64, A64, D64, g64 = (t.double() for t in f32[:4])
    ref = ct.forward(L64, A64, D64, *(t.double() for t in f32[4:]))
    diff = xyz.detach().double() - ref
    rms = float(diff.pow(2).sum(-1).mean().sqrt())
    mx = diff.abs().amax(dim=(1, 2))
    scale = N / 2049
    print(f"long every chain: RMS {rms:.2e} nm over the batch, worst max-abs {mx.max():.2e} nm "
          f"(bars {1e-5 * scale:.1e}, {1e-4 * scale:.1e}), extent {ref.abs().max():.0f} nm")
    assert rms <= 1e-5 * scale and bool((mx <= 1e-4 * scale).all())
    _check_roundtrip(xyz.detach(), L64, A64, D64, "long")
    _check_gradients("long", grads, ct.backward(ref, g64), 5e-5)


# ----------------------------------------------------------------- fused losses, every chain


def _target(xyz64, seed, rotate):
    """A target per chain: the float64 chain, rigidly moved when ``rotate`` (one proper rotation
    and a 4 nm shift for the batch, so the superposition has work to do), plus N(0, 0.3 nm)
    noise per coordinate; rounded to float32, whose float64 value is returned."""
    gen = torch.Generator().manual_seed(seed)
    dev = xyz64.device
    noise = (torch.randn(*xyz64.shape, generator=gen, dtype=torch.float64) * 0.3).to(dev)
    t = xyz64 + noise
    if rotate:
        q, _ = torch.linalg.qr(torch.randn(3, 3, generator=gen, dtype=torch.float64))
        q = q * torch.sign(torch.linalg.det(q))
        shift = torch.randn(3, generator=gen, dtype=torch.float64) * 4.0
        t = xyz64 @ q.T.contiguous().to(dev) + shift.to(dev) + noise
    return t.float().double()


def _loss_refs(kind, ref, xs, t64):
    """float64 loss of the float64 chain, and grad_xyz over the stored positions ``xs`` (the
    fused backward differentiates the loss of the positions it stored)."""
    if kind == "loss":
        return ((ref - t64) ** 2).sum((1, 2)), 2.0 * (xs - t64)
    sq = kind == "msd"
    tn = t64.cpu().numpy()
    loss = o.superposed_loss(ref.cpu().numpy(), tn, sq)
    gx = o.superposed_grad_xyz(xs.cpu().numpy(), tn, None, sq)
    return torch.as_tensor(loss).to(ref.device), torch.as_tensor(gx).to(ref.device)


def _unfused_loss(kind, x, t64):
    """The same loss in torch over the unfused output ``x``; for the superposed kinds the
    rotation is solved on the host (oracle/nerf64.py superpose, SVD) from x's values and held
    fixed, its own dependence dropping out at the optimum."""
    t = t64.to(x.dtype)
    if kind == "loss":
        return ((x - t) ** 2).sum((1, 2))
    R, _, _, _ = o.superpose(x.detach().double().cpu().numpy(), t64.cpu().numpy())
    Rt = torch.as_tensor(R).to(device=x.device, dtype=x.dtype).transpose(1, 2).contiguous()
    msd = ((x - x.mean(1, keepdim=True)) @ Rt - (t - t.mean(1, keepdim=True))).pow(2).sum(-1).mean(-1)
    return msd if kind == "msd" else msd.sqrt()


def _check_fused(kind, label, loss, unfused, want_loss, grads, ugrads, adj):
    """Loss per chain within 1e-5 relative of the float64 chain's and of the unfused composition;
    gradients per chain within 5e-5 relative of the float64 adjoint over the stored positions.
    A superposed loss is invariant under rigid motions, so its grad_xyz has zero net force and
    torque and the adjoint's float32 suffix sums end in the remainder of a cancelling sum; there
    the bar is the larger of 5e-5 and 1.5x the unfused composition's own error on that chain
    (reconstruct's backward over the same grad_xyz carries the same amplification)."""
    lerr = (loss.detach().double() - want_loss).abs() / want_loss.abs()
    uerr = (loss.detach() - unfused.detach()).abs() / unfused.detach().abs()
    print(f"{label} fused {kind}, every chain: worst loss rel err {lerr.max():.2e} against float64, "
          f"{uerr.max():.2e} against the unfused composition")
    assert bool((lerr <= 1e-5).all()) and bool((uerr <= 1e-5).all())
    for name, got, alt, w in zip(("lengths", "angles", "dihedrals", "raw pairs"), grads, ugrads, adj):
        f = _per_chain_rel(got, w)
        u = _per_chain_rel(alt, w)
        bar = torch.full_like(f, 5e-5) if kind == "loss" else torch.clamp(1.5 * u, min=5e-5)
        print(f"  d/d{name}: worst per-chain rel err fused {f.max():.2e} (chain {int(f.argmax())}), "
              f"unfused {u.max():.2e}; chains over 5e-5: fused {int((f > 5e-5).sum())}, unfused {int((u > 5e-5).sum())}")
        assert bool(torch.isfinite(got).all()) and bool((f <= bar).all())


@pytest.mark.parametrize("kind", ["loss", "rmsd", "msd"])
def test_config2_fused_losses_every_chain(cufk, device, kind):
    """reconstruct_loss and reconstruct_rmsd (root and squared) at the C2 shape (B = 4096,
    N = 2049, float32, random anchors), every chain, against float64 and the unfused
    composition (reconstruct, the loss in torch, autograd)."""
    B, N = 4096, 2049
    L, A, D, _, p0, fd, n0 = _synthetic(B, N, 12, device)
    f32 = [t.float() for t in (L, A, D, p0, fd, n0)]
    ref = ct.forward(*(t.double() for t in f32))
    t64 = _target(ref, 12, rotate=kind != "loss")
    t32 = t64.float()
    Lf, Af, Df = (x.clone().requires_grad_(True) for x in f32[:3])
    if kind == "loss":
        loss = cufk.reconstruct_loss(Lf, Af, Df, t32, *f32[3:])
    else:
        loss = cufk.reconstruct_rmsd(Lf, Af, Df, t32, *f32[3:], squared=kind == "msd")
    grads = torch.autograd.grad(loss.sum(), (Lf, Af, Df))
    Lu, Au, Du = (x.clone().requires_grad_(True) for x in f32[:3])
    x = cufk.reconstruct(Lu, Au, Du, *f32[3:])
    unfused = _unfused_loss(kind, x, t64)
    ugrads = torch.autograd.grad(unfused.sum(), (Lu, Au, Du))
    xs = x.detach().double()  # the positions the fused forward stores: the same kernel arithmetic
    want_loss, gx = _loss_refs(kind, ref, xs, t64)
    adj = ct.backward(xs, gx)
    _check_fused(kind, "C2", loss, unfused, want_loss, grads, ugrads, adj)


@pytest.mark.parametrize("kind", ["loss", "rmsd", "msd"])
def test_config3_fused_losses_every_chain(cufk, device, kind):
    """compile_torsion(...).loss and .rmsd (root and squared) at the C3 shape (B = 8192,
    N = 771, float32), every chain, against float64 and the unfused composition."""
    B, N = 8192, 771
    gen = torch.Generator().manual_seed(13)
    raw64 = torch.randn(B, 2 * (N - 3), generator=gen, dtype=torch.float64).float().double().to(device)
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    ref = ct.torsion_forward(raw64, c.lengths, c.sin, c.cos)
    t64 = _target(ref, 13, rotate=kind != "loss")
    f = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    raw = raw64.float().requires_grad_(True)
    loss = f.loss(raw, t64.float()) if kind == "loss" else f.rmsd(raw, t64.float(), squared=kind == "msd")
    (graw,) = torch.autograd.grad(loss.sum(), (raw,))
    raw_u = raw64.float().requires_grad_(True)
    x = f(raw_u)
    unfused = _unfused_loss(kind, x, t64)
    (ugraw,) = torch.autograd.grad(unfused.sum(), (raw_u,))
    xs = x.detach().double()
    want_loss, gx = _loss_refs(kind, ref, xs, t64)
    adj = ct.torsion_backward(raw64, xs, gx, c.lengths)
    _check_fused(kind, "C3", loss, unfused, want_loss, (graw,), (ugraw,), (adj,))


# ----------------------------------------------------------------- committed fixtures


def _t(x, dtype, device, grad=False):
    return torch.as_tensor(np.asarray(x), dtype=torch.float64).to(device=device, dtype=dtype).requires_grad_(grad)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_golden_reconstruct_fixtures_forward_and_backward(cufk, device, golden_c0, golden_anchored, dtype):
    """Both reconstruct fixtures (C0 with default anchors; three anchored chains), forward and
    gradients, through the autograd path.  float64 within 1e-13 / 1e-10 relative; float32 on
    the float32-rounded inputs within 2e-6 nm and 5e-5 relative (the fixtures hold float64
    inputs, so float32 adds the inputs' own rounding, a few 1e-8 relative)."""
    for g in (golden_c0, golden_anchored):
        L, A, D = (_t(g[k], dtype, device, True) for k in ("lengths", "angles", "dihedrals"))
        an = [_t(g[k], dtype, device) for k in ("p0", "first_direction", "initial_normal") if k in g]
        xyz = cufk.reconstruct(L, A, D, *an)
        grads = torch.autograd.grad(xyz, (L, A, D), _t(g["grad"], dtype, device))
        ex = np.abs(xyz.detach().double().cpu().numpy() - g["xyz"]).max()
        eg = [np.abs(a.double().cpu().numpy() - g[k]).max() / np.abs(g[k]).max()
              for a, k in zip(grads, ("grad_lengths", "grad_angles", "grad_dihedrals"))]
        print(f"fixture {g['xyz'].shape} {dtype}: xyz {ex:.2e}, grads " + ", ".join(f"{e:.2e}" for e in eg))
        assert ex <= (1e-13 if dtype == torch.float64 else 2e-6)
        assert max(eg) <= (1e-10 if dtype == torch.float64 else 5e-5)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_golden_torsion_fixture_forward_and_backward(cufk, device, golden_torsion, dtype):
    g = golden_torsion
    f = cufk.compile_torsion(tuple(g["bond_lengths"]), tuple(g["bond_angles"]))
    raw = _t(g["raw_pairs"], dtype, device, True)
    xyz = f(raw)
    (gr,) = torch.autograd.grad(xyz, (raw,), _t(g["grad"], dtype, device))
    ex = np.abs(xyz.detach().double().cpu().numpy() - g["xyz"]).max()
    eg = np.abs(gr.double().cpu().numpy() - g["grad_raw"]).max() / np.abs(g["grad_raw"]).max()
    print(f"torsion fixture {dtype}: xyz {ex:.2e}, grad {eg:.2e}")
    assert ex <= (1e-13 if dtype == torch.float64 else 2e-6)
    assert eg <= (1e-10 if dtype == torch.float64 else 5e-5)


# ----------------------------------------------------------------- torsion pair clamp


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_torsion_zero_and_tiny_pairs(cufk, device, dtype):
    """Raw pairs whose squared norm is below the 1e-16 clamp (torsion.cu:119-141): an exact
    zero pair, pairs of 1e-9 and 3e-9, and one just above the clamp (2e-8): forward and
    gradients against the oracle on the same values (float32: 1e-5 nm RMS, 5e-5 relative)."""
    rng = np.random.default_rng(77)
    B, N = 4, 200
    raw = rng.normal(size=(B, 2 * (N - 3)))
    raw[0, 10:12] = 0.0
    raw[1, 40:42] = (1e-9, 0.0)
    raw[2, 0:2] = (3e-9, -1e-9)  # the first step
    raw[3, 2 * (N - 4):] = (0.0, 2e-8)  # the last step, just above the clamp
    raw[3, 100:102] = (-4e-9, 5e-10)
    raw = torch.as_tensor(raw).to(dtype).double().numpy()
    g = rng.normal(size=(B, N, 3))
    c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
    r = _t(raw, dtype, device, True)
    xyz = cufk.compile_torsion(BOND_LENGTHS, BOND_ANGLES)(r)
    (gr,) = torch.autograd.grad(xyz, (r,), _t(g, dtype, device))
    ref = o.torsion_forward(raw, c)
    ref_g = o.torsion_backward(raw, ref, g, c)
    diff = xyz.detach().double().cpu().numpy() - ref
    eg = np.abs(gr.double().cpu().numpy() - ref_g).max(axis=1) / np.abs(ref_g).max(axis=1)
    print(f"torsion clamp {dtype}: xyz max {np.abs(diff).max():.2e}, grad rel per chain {eg}")
    assert torch.isfinite(xyz).all() and torch.isfinite(gr).all()
    if dtype == torch.float64:
        assert np.abs(diff).max() <= 1e-12 and eg.max() <= 1e-9
    else:
        assert math.sqrt(np.mean(np.sum(diff**2, -1))) <= 1e-5 and eg.max() <= 5e-5


# ----------------------------------------------------------------- multi-wave gradcheck


@pytest.mark.parametrize("modify", [False, True])
def test_gradcheck_fp64_multi_wave(cufk, device, modify):
    """torch.autograd.gradcheck at N = 600 (597 steps: the two-wave plan) through the backward
    over the saved output and, with the output changed in place, through the recompute."""
    d = o.synthetic_inputs(1, 600, seed=600, anchors=True)
    L, A, D = (_t(d[k], torch.float64, device, True) for k in ("lengths", "angles", "dihedrals"))
    an = [_t(d[k], torch.float64, device) for k in ("p0", "first_direction", "initial_normal")]

    def fn(a, b, c):
        x = cufk.reconstruct(a, b, c, *an)
        if modify:
            x.mul_(1.0)  # bumps the version counter: the backward recomputes
        return x

    assert torch.autograd.gradcheck(fn, (L, A, D), eps=1e-6, atol=1e-7, rtol=1e-6, fast_mode=False)

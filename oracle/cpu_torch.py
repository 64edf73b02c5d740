"""PyTorch-CPU float64 NeRF: the CPU baseline that bench.py times.  TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and the ``cpu_baseline`` leg of ``bench.py`` may import this module.  The
product (``cufk_amd``) never imports it.

The reference has no CPU path: every op requires a CUDA tensor (``extension_utils.cuh:57-61``
under the reference tree ``src/cufk/csrc/``).  This is the reference's algorithm restated for
the CPU in PyTorch float64, vectorised over the batch and serial over the chain's steps:

* ``forward``: the first frame of ``block.cu:113-148`` (Gram-Schmidt of the anchors with the
  helper-axis fallback of ``frame_utils.cuh:23-31``), then the running rigid transform of the
  reference's affine scan (``affine.cuh:24-58``, ``block.cu:190-201``) walked one step at a
  time: x_{k+3} = t_{k-1} + R_{k-1} v_k, R_k = R_{k-1} M_k, starting from R = F, t = x2.
* ``backward``: the explicit reverse adjoint in world-frame form (force and moment suffix sums
  F_i = sum_{j>=i} g_j, M_i = sum_{j>=i} x_j x g_j; the form ``torsion.cu:204-217`` uses for
  dihedrals), giving dL/d(lengths, angles, dihedrals).  Anchors get no gradient
  (``block.cu:427``).

Pinned in ``tests/test_oracle.py`` against ``oracle/nerf64.py`` (itself pinned against serial
Parsons NeRF, the internal-coordinate round trip, autograd and finite differences): forward
within 1e-12, gradients within 1e-10 relative, including the degenerate-normal branch.
"""

from __future__ import annotations

import torch

K_EPS = 9.999999960041972e-13  # float(1e-12f): block.cu:41, frame_utils.cuh:7


def _nrm(v):
    return v / torch.sqrt(torch.clamp((v * v).sum(-1, keepdim=True), min=K_EPS))


def first_frame(L0, L1, A0, p0, fd, n0):
    """block.cu:113-148.  L0, L1, A0: (B,); anchors (3,).  Returns x1, x2 (B, 3), F (B, 3, 3)."""
    B = L0.shape[0]
    d0 = _nrm(fd.expand(B, 3))
    x1 = p0 + L0[:, None] * d0
    n = n0.expand(B, 3) - (n0 * d0).sum(-1, keepdim=True) * d0
    degenerate = (n * n).sum(-1, keepdim=True) < K_EPS
    use_y = d0[:, :1].abs() >= 0.9
    helper = torch.cat([(~use_y).to(d0.dtype), use_y.to(d0.dtype), torch.zeros_like(d0[:, :1])], dim=1)
    n = torch.where(degenerate, _nrm(torch.linalg.cross(d0, helper)), _nrm(n))
    t0 = _nrm(torch.linalg.cross(n, d0))
    s, c = torch.sin(A0)[:, None], torch.cos(A0)[:, None]
    d1 = -c * d0 + s * t0
    x2 = x1 + L1[:, None] * d1
    nn = _nrm(torch.linalg.cross(d0, d1))
    frame = torch.stack([d1, torch.linalg.cross(nn, d1), nn], dim=-1)
    return x1, x2, frame


def _local(length, s, c, S, C):
    """affine.cuh:24-51: M_k as columns M[:, 0] = (-c, sC, sS), M[:, 1] = (-s, -cC, -cS),
    M[:, 2] = (0, -S, C), and v_k = l M[:, 0]; (B, K, 3, 3) and (B, K, 3)."""
    zero = torch.zeros_like(S)
    col0 = torch.stack([-c.expand_as(S), s * C, s * S], dim=-1)
    M = torch.stack([col0, torch.stack([-s.expand_as(S), -c * C, -c * S], dim=-1),
                     torch.stack([zero, -S, C], dim=-1)], dim=-1)
    return M, length[..., None] * col0


def _walk(xyz, x2, R, M, V):
    """The serial scan: x_{k+3} = t_{k-1} + R_{k-1} v_k, R_k = R_{k-1} M_k from R = F, t = x2.
    The per-step operands are laid out step-major first, so every product takes contiguous
    (B, 3, 3) / (B, 3, 1) operands (also when the tensors live on a GPU)."""
    M = M.transpose(0, 1).contiguous()
    V = V.transpose(0, 1).unsqueeze(-1).contiguous()
    R = R.contiguous()
    t = x2
    for k in range(M.shape[0]):  # one rigid compose per step
        t = t + torch.bmm(R, V[k])[..., 0]
        xyz[:, k + 3] = t
        R = torch.bmm(R, M[k])
    return xyz


def forward(L, A, D, p0, fd, n0):
    """(B, N-1), (B, N-2), (B, N-3) float64 CPU tensors and (3,) anchors -> xyz (B, N, 3)."""
    B, S = D.shape
    x1, x2, R = first_frame(L[:, 0], L[:, 1], A[:, 0], p0, fd, n0)
    M, V = _local(L[:, 2:], torch.sin(A[:, 1:]), torch.cos(A[:, 1:]), torch.sin(D), torch.cos(D))
    xyz = torch.empty(B, S + 3, 3, dtype=L.dtype, device=L.device)
    xyz[:, 0] = p0
    xyz[:, 1] = x1
    xyz[:, 2] = x2
    return _walk(xyz, x2, R, M, V)


K_NORM_EPS2 = 1.0000000168623835e-16  # float(1e-8f * 1e-8f) formed in float: torsion.cu:35,120-123


def _torsion_tables(S, lengths, sins, coss):
    """Phase maps of torsion.cu:67-73: step k uses l_{(k+2)%3} and angle (k+1)%3."""
    k = torch.arange(S)
    pick = lambda v, off: torch.tensor(v, dtype=torch.float64)[(k + off) % 3]  # noqa: E731
    return pick(lengths, 2), pick(sins, 1), pick(coss, 1)


def torsion_forward(raw, lengths, sins, coss):
    """torsion.cu:254-295: raw (B, 2(N-3)) interleaved (sin, cos) pairs; constants as torsion.cu:43-53
    (lengths float-rounded, bond-angle sin/cos float64).  Base frame torsion.cu:149-166."""
    B, K = raw.shape
    S = K // 2
    rs, rc = raw[:, 0::2], raw[:, 1::2]
    r = torch.rsqrt(torch.clamp(rs * rs + rc * rc, min=K_NORM_EPS2))
    dev = dict(dtype=torch.float64, device=raw.device)
    ell, s, c = (t.to(raw.device) for t in _torsion_tables(S, lengths, sins, coss))
    M, V = _local(ell.expand(B, S), s, c, rs * r, rc * r)
    l0, l1, s0, c0 = lengths[0], lengths[1], sins[0], coss[0]
    x2 = torch.tensor([l0 - l1 * c0, l1 * s0, 0.0], **dev).expand(B, 3)
    R = torch.tensor([[-c0, -s0, 0.0], [s0, -c0, 0.0], [0.0, 0.0, 1.0]], **dev).expand(B, 3, 3)
    xyz = torch.empty(B, S + 3, 3, **dev)
    xyz[:, 0] = 0.0
    xyz[:, 1] = torch.tensor([l0, 0.0, 0.0], **dev)
    xyz[:, 2] = x2
    return _walk(xyz, x2, R, M, V)


def torsion_backward(raw, xyz, g, lengths):
    """torsion.cu:297-381 with 173-182, 213-217: dphi_k = (1/l_{(k+1)%3}) (x_{k+2} - x_{k+1}) .
    (M_{k+3} - x_{k+2} x F_{k+3}), the reciprocal formed in float; raw grad = dphi (rc, -rs) / n2."""
    S = raw.shape[1] // 2
    F = torch.flip(torch.cumsum(torch.flip(g, [1]), 1), [1])
    Mo = torch.flip(torch.cumsum(torch.flip(torch.linalg.cross(xyz, g), [1]), 1), [1])
    f32 = lambda v: torch.tensor(v, dtype=torch.float32)  # noqa: E731
    inv = [float(f32(1.0) / f32(lengths[(p + 1) % 3])) for p in range(3)]
    inv = torch.tensor(inv, dtype=torch.float64, device=raw.device)[torch.arange(S, device=raw.device) % 3]
    pivot = xyz[:, 2:-1]
    tau = Mo[:, 3:] - torch.linalg.cross(pivot, F[:, 3:])
    dphi = inv * ((pivot - xyz[:, 1:-2]) * tau).sum(-1)
    rs, rc = raw[:, 0::2], raw[:, 1::2]
    scale = dphi / torch.clamp(rs * rs + rc * rc, min=K_NORM_EPS2)
    out = torch.empty_like(raw)
    out[:, 0::2] = rc * scale
    out[:, 1::2] = -rs * scale
    return out


def backward(xyz, g):
    """World-frame reverse adjoint: dL/d(lengths, angles, dihedrals) from xyz and grad_xyz."""
    centre = xyz[:, 2:3]  # moments about x2 keep the suffix sums well conditioned
    x = xyz - centre
    F = torch.flip(torch.cumsum(torch.flip(g, [1]), 1), [1])  # F_i = sum_{j>=i} g_j
    Mo = torch.flip(torch.cumsum(torch.flip(torch.linalg.cross(x, g), [1]), 1), [1])
    b = x[:, 1:] - x[:, :-1]  # b_i = x_{i+1} - x_i
    gL = (_unit(b) * F[:, 1:]).sum(-1)
    # tau_i(q) = M_i - q x F_i
    tau_a = Mo[:, 2:] - torch.linalg.cross(x[:, 1:-1], F[:, 2:])  # at x_{i+1}, i = 0..N-3
    gA = (_unit(torch.linalg.cross(-b[:, :-1], b[:, 1:])) * tau_a).sum(-1)
    tau_d = Mo[:, 3:] - torch.linalg.cross(x[:, 2:-1], F[:, 3:])  # at x_{i+2}, i = 0..N-4
    gD = (_unit(b[:, 1:-1]) * tau_d).sum(-1)
    return gL, gA, gD


def _unit(v):
    return v / torch.sqrt((v * v).sum(-1, keepdim=True))

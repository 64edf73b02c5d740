"""The backwards that choose per chain between the position-based adjoint and the exact one (the
saved-output backward and the fused-loss backward) start their grids with front workgroups: two
per group of 16 chains, the r-th taking the group's r-th refused chain (regular flag 0, counted
from a position that rotates with the group), whose own workgroup then does nothing.  Every chain must still be processed exactly once and by the right
path, whatever the refusal pattern (none, all, fewer or more than two per group, a partial last
group):

- float64: every gradient against the oracle, with the outputs filled with NaN beforehand so a
  chain that no workgroup takes shows up;
- float32: every sampled chain bit-identical to the same chain run alone (B = 1);
- the flags the forward wrote match the pattern the inputs were built for.

A chain is refused by giving it one bond angle of 3.135 rad (sin 0.0066, below both the float32
0.5 and the float64 0.01 thresholds).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import nerf64 as o

pytestmark = pytest.mark.gpu

B, N = 133, 40  # eight groups of 16 (every counting offset twice) and a partial ninth (chains 128..132)
PATTERNS = {
    "none": [],
    "all": list(range(B)),
    "group_heads": list(range(0, B, 16)),
    "two_per_group": [c for c in range(B) if c % 16 in (3, 4)],
    "six_per_group": [c for c in range(B) if c % 16 in (0, 2, 5, 7, 9, 15)],
    "last_only": [B - 1],
    "random": sorted(np.random.default_rng(5).choice(B, 40, replace=False).tolist()),
}
CODES = {torch.float32: 0, torch.float64: 1}


@pytest.fixture(scope="module")
def lib(device):
    import cufk_amd

    lib = ctypes.CDLL(str(cufk_amd._native.HIP_LIBRARY))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.cufk_reconstruct_fwd_flagged.argtypes = [ctypes.c_int] + [vp] * 8 + [i64, i64, vp]
    lib.cufk_reconstruct_bwd_saved.argtypes = [ctypes.c_int] + [vp] * 12 + [i64, i64, vp]
    lib.cufk_reconstruct_loss_fwd.argtypes = [ctypes.c_int] + [vp] * 10 + [i64, i64, vp]
    lib.cufk_reconstruct_loss_bwd.argtypes = [ctypes.c_int] + [vp] * 13 + [i64, i64, vp]
    return lib


def _case(refused):
    d = o.synthetic_inputs(B, N, 77, anchors=True)
    d["angles"][refused, 10] = 3.135
    d["target"] = o.synthetic_inputs(B, N, 78)["grad"] * 0.3
    return d


def _run(lib, d, dtype, device, rows, loss):
    """Flagged forward and the per-chain backward through the C ABI for chains `rows`;
    returns (flags, gL, gA, gD) with the outputs NaN-filled beforehand."""
    t = {k: torch.as_tensor(np.ascontiguousarray(v[rows] if np.ndim(v) > 1 else v)).to(device, dtype)
         for k, v in d.items()}
    b = len(rows)
    xyz = torch.empty(b, N, 3, device=device, dtype=dtype)
    flags = torch.full((b,), 7, device=device, dtype=torch.uint8)
    gL, gA, gD = (torch.full((b, N - k), float("nan"), device=device, dtype=dtype) for k in (1, 2, 3))
    p = lambda x: x.data_ptr()  # noqa: E731
    st = torch.cuda.current_stream().cuda_stream
    an = (p(t["p0"]), p(t["first_direction"]), p(t["initial_normal"]))
    c = CODES[dtype]
    if loss:
        out = torch.empty(b, device=device, dtype=dtype)
        assert lib.cufk_reconstruct_loss_fwd(c, p(t["lengths"]), p(t["angles"]), p(t["dihedrals"]), *an, p(t["target"]),
                                             p(xyz), p(flags), p(out), b, N, st) == 0
        assert lib.cufk_reconstruct_loss_bwd(c, p(t["lengths"]), p(t["angles"]), p(t["dihedrals"]), *an, p(xyz),
                                             p(flags), p(t["target"]), None, p(gL), p(gA), p(gD), b, N, st) == 0
    else:
        assert lib.cufk_reconstruct_fwd_flagged(c, p(t["lengths"]), p(t["angles"]), p(t["dihedrals"]), *an, p(xyz),
                                                p(flags), b, N, st) == 0
        assert lib.cufk_reconstruct_bwd_saved(c, p(t["lengths"]), p(t["angles"]), p(t["dihedrals"]), *an, p(xyz),
                                              p(flags), p(t["grad"]), p(gL), p(gA), p(gD), b, N, st) == 0
    torch.cuda.synchronize()
    return flags.cpu().numpy(), gL, gA, gD


@pytest.mark.parametrize("loss", [False, True])
@pytest.mark.parametrize("pattern", sorted(PATTERNS))
def test_every_chain_once_fp64(lib, device, pattern, loss):
    refused = PATTERNS[pattern]
    d = _case(refused)
    flags, *grads = _run(lib, d, torch.float64, device, list(range(B)), loss)
    assert flags.tolist() == [0 if c in refused else 1 for c in range(B)]
    an = {k: d[k] for k in ("p0", "first_direction", "initial_normal")}
    g = d["grad"]
    if loss:
        x = o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **an)
        g = 2.0 * (x - d["target"])
    ref = o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], g, **an)
    for got, want in zip(grads, ref):
        got = got.cpu().numpy()
        assert np.isfinite(got).all()
        assert np.abs(got - want).max() <= 1e-9 * np.abs(want).max()


@pytest.mark.parametrize("loss", [False, True])
@pytest.mark.parametrize("pattern", ["group_heads", "two_per_group", "six_per_group", "random", "last_only"])
def test_chains_match_alone_fp32(lib, device, pattern, loss):
    d = _case(PATTERNS[pattern])
    _, *batch = _run(lib, d, torch.float32, device, list(range(B)), loss)
    for c in sorted({0, 3, 4, 16, 19, 20, 31, 48, 127, 128, B - 1} | set(PATTERNS[pattern][:8])):
        _, *alone = _run(lib, d, torch.float32, device, [c], loss)
        for got, want in zip(batch, alone):
            assert torch.equal(got[c], want[0]), (pattern, c)

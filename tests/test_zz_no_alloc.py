"""The allocation-free anchored backward (cufk_reconstruct_bwd_anchored_noalloc) against
cufk_reconstruct_bwd_anchored with a caller-allocated workspace, through the C ABI.

Both run the same kernels on the same inputs, so every output is bit-identical.  Two calls in a
row, the second on a smaller batch, show that the static scratch keeps no state a call depends
on; both backward kinds (saved output and recompute) and float64/float32 are covered.  The entry
point is also captured in a HIP graph and replayed, and warm calls are checked to leave the
device's free memory unchanged.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import nerf64 as o

pytestmark = pytest.mark.gpu

CODES = {torch.float32: 0, torch.float64: 1}
ERR_SCRATCH = 10
MAX_CHAINS = 65536


@pytest.fixture(scope="module")
def lib(device):
    import cufk_amd

    lib = ctypes.CDLL(str(cufk_amd._native.HIP_LIBRARY))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.cufk_reconstruct_fwd_flagged.argtypes = [ctypes.c_int] + [vp] * 8 + [i64, i64, vp]
    lib.cufk_reconstruct_bwd_anchored.argtypes = [ctypes.c_int] + [vp] * 16 + [i64, i64, vp]
    lib.cufk_reconstruct_bwd_anchored_noalloc.argtypes = [ctypes.c_int] + [vp] * 15 + [i64, i64, vp]
    return lib


def _case(B, N, seed, dtype, device):
    d = o.synthetic_inputs(B, N, seed, anchors=True)
    t = {k: torch.as_tensor(v).to(device=device, dtype=dtype) for k, v in d.items()}
    return t


def _run(lib, t, B, N, dtype, saved, noalloc):
    p = lambda x: None if x is None else x.data_ptr()  # noqa: E731
    st = torch.cuda.current_stream().cuda_stream
    code = CODES[dtype]
    an = [t[k] for k in ("p0", "first_direction", "initial_normal")]
    L, A, D = t["lengths"], t["angles"], t["dihedrals"]
    xyz = reg = None
    if saved:
        xyz = torch.empty(B, N, 3, dtype=dtype, device=L.device)
        reg = torch.empty(B, dtype=torch.uint8, device=L.device)
        assert lib.cufk_reconstruct_fwd_flagged(code, p(L), p(A), p(D), *map(p, an), p(xyz), p(reg), B, N, st) == 0
    grads = [torch.full_like(x, float("nan")) for x in (L, A, D)]
    agrads = [torch.full((3,), float("nan"), dtype=dtype, device=L.device) for _ in range(3)]
    if noalloc:
        rc = lib.cufk_reconstruct_bwd_anchored_noalloc(code, p(L), p(A), p(D), *map(p, an), p(xyz), p(reg),
                                                       p(t["grad"]), *map(p, grads), *map(p, agrads), B, N, st)
    else:
        work = torch.full((6 * B,), float("nan"), dtype=torch.float64, device=L.device)
        rc = lib.cufk_reconstruct_bwd_anchored(code, p(L), p(A), p(D), *map(p, an), p(xyz), p(reg), p(t["grad"]),
                                               *map(p, grads), p(work), *map(p, agrads), B, N, st)
    assert rc == 0
    torch.cuda.synchronize()
    return grads + agrads


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("saved", [True, False])
def test_noalloc_equals_the_workspace_entry_point(lib, device, dtype, saved):
    # Two calls in a row on the allocation-free entry point, the second smaller: each must
    # equal the workspace entry point on the same inputs, bit for bit.
    for B, N, seed in ((3000, 300, 1), (700, 120, 2)):
        t = _case(B, N, seed, dtype, device)
        want = _run(lib, t, B, N, dtype, saved, noalloc=False)
        got = _run(lib, t, B, N, dtype, saved, noalloc=True)
        for a, b in zip(got, want):
            assert torch.isfinite(a).all()
            assert torch.equal(a, b)


def test_noalloc_full_scratch_and_packed_chains(lib, device):
    # The largest batch the scratch holds, with short chains (the packed kernels write the
    # per-chain sums), then a small batch with a chain count that is not a multiple of anything.
    for B, N, seed in ((MAX_CHAINS, 20, 3), (37, 64, 4)):
        t = _case(B, N, seed, torch.float32, device)
        want = _run(lib, t, B, N, torch.float32, True, noalloc=False)
        got = _run(lib, t, B, N, torch.float32, True, noalloc=True)
        for a, b in zip(got, want):
            assert torch.equal(a, b)


def test_noalloc_rejects_batches_beyond_the_scratch(lib, device):
    # Rejected before any device work: no pointer is touched.
    vp = [None] * 15
    rc = lib.cufk_reconstruct_bwd_anchored_noalloc(0, *vp, MAX_CHAINS + 1, 40, None)
    assert rc == ERR_SCRATCH
    rc = lib.cufk_reconstruct_bwd_anchored_noalloc(0, *vp, MAX_CHAINS, 3, None)
    assert rc == 2  # point_count must be >= 4, checked first


def test_noalloc_captured_in_a_graph_and_allocation_free(lib, device):
    """The entry point is for callers that cannot allocate, graph capture first among them.
    Captured in a HIP graph and replayed three times, with an eager call on other inputs (which
    overwrites the shared scratch) and a synchronisation between replays, every replay equals
    the eager call bit for bit.  Warm calls on fixed buffers leave the device's free memory as
    it was."""
    B, N, dtype = 2000, 300, torch.float32
    p = lambda x: None if x is None else x.data_ptr()  # noqa: E731

    def buffers(seed):
        t = _case(B, N, seed, dtype, device)
        xyz = torch.empty(B, N, 3, dtype=dtype, device=device)
        reg = torch.empty(B, dtype=torch.uint8, device=device)
        an = [p(t[k]) for k in ("p0", "first_direction", "initial_normal")]
        st = torch.cuda.current_stream().cuda_stream
        assert lib.cufk_reconstruct_fwd_flagged(0, p(t["lengths"]), p(t["angles"]), p(t["dihedrals"]), *an, p(xyz),
                                                p(reg), B, N, st) == 0
        outs = [torch.empty_like(t[k]) for k in ("lengths", "angles", "dihedrals")]
        outs += [torch.empty(3, dtype=dtype, device=device) for _ in range(3)]

        def call():
            s = torch.cuda.current_stream().cuda_stream  # the capture stream while capturing
            rc = lib.cufk_reconstruct_bwd_anchored_noalloc(0, p(t["lengths"]), p(t["angles"]), p(t["dihedrals"]), *an,
                                                           p(xyz), p(reg), p(t["grad"]), *map(p, outs), B, N, s)
            assert rc == 0

        return call, outs

    call, outs = buffers(11)
    other, _ = buffers(12)
    call()
    torch.cuda.synchronize()
    want = [o_.clone() for o_ in outs]

    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        call()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(3):
        for o_ in outs:
            o_.fill_(float("nan"))
        other()  # eager call on other inputs: the scratch now holds their sums
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, want):
            assert torch.equal(a, b)

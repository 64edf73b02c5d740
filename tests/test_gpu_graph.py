"""HIP-graph capture of the autograd step: forward + torch.autograd.grad captured once in a
torch CUDA graph (hipGraph on ROCm) and replayed.  The ops enqueue on the current stream,
allocate only through torch's allocator (the graph's private pool under capture), issue no
memset and never synchronise, so the step is capturable.  Each replay runs with new inputs
copied into the captured tensors, with eager work on the same stream between replays, and must
equal the eager step on the same inputs bit for bit (the same kernels run on the same data)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nerf64 as o

pytestmark = pytest.mark.gpu

BOND_LENGTHS = (0.14685231, 0.15365194, 0.13405086)
BOND_ANGLES = (1.9676635, 2.062335, 2.164016)


def _set(B, N, seed, dtype, device):
    d = o.synthetic_inputs(B, N, seed, anchors=True)
    return {k: torch.as_tensor(v, dtype=torch.float64).to(device=device, dtype=dtype) for k, v in d.items()}


def _capture(step, warmup_args):
    """Warm up on a side stream (as torch's capture recipe asks), then capture step()."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step(*warmup_args)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step(*warmup_args)
    return graph, out


@pytest.mark.parametrize("dtype,B,N", [(torch.float32, 64, 384), (torch.float64, 8, 300), (torch.bfloat16, 16, 1026),
                                       (torch.float32, 4096, 64)])
def test_reconstruct_step_replays(device, dtype, B, N):
    import cufk_amd

    s = _set(B, N, 11, dtype, device)
    L, A, D = (s[k].clone().requires_grad_(True) for k in ("lengths", "angles", "dihedrals"))
    p0, fd, n0, g = s["p0"], s["first_direction"], s["initial_normal"], s["grad"].clone()

    def step(L, A, D, g):
        xyz = cufk_amd.reconstruct(L, A, D, p0, fd, n0)
        return (xyz, *torch.autograd.grad(xyz, (L, A, D), g))

    graph, out = _capture(step, (L, A, D, g))
    for rep in range(4):
        t = _set(B, N, 100 + rep, dtype, device)
        with torch.no_grad():
            for dst, k in ((L, "lengths"), (A, "angles"), (D, "dihedrals"), (g, "grad")):
                dst.copy_(t[k])
        graph.replay()
        # eager work on the same stream between replays, then the eager reference
        ref = step(*(t[k].clone().requires_grad_(k != "grad") for k in ("lengths", "angles", "dihedrals", "grad")))
        torch.cuda.synchronize()
        for got, want in zip(out, ref):
            assert torch.equal(got, want), (rep, dtype)


def test_torsion_step_replays(device):
    import cufk_amd

    head = cufk_amd.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
    B, N = 256, 771
    rng = np.random.default_rng(3)

    def draw():
        raw = torch.as_tensor(rng.normal(size=(B, 2 * (N - 3))), dtype=torch.float32, device=device)
        g = torch.as_tensor(rng.normal(size=(B, N, 3)), dtype=torch.float32, device=device)
        return raw, g

    raw, g = draw()
    raw.requires_grad_(True)

    def step(raw, g):
        xyz = head(raw)
        return (xyz, *torch.autograd.grad(xyz, (raw,), g))

    graph, out = _capture(step, (raw, g))
    for rep in range(4):
        r2, g2 = draw()
        with torch.no_grad():
            raw.copy_(r2)
            g.copy_(g2)
        graph.replay()
        ref = step(r2.clone().requires_grad_(True), g2)
        torch.cuda.synchronize()
        for got, want in zip(out, ref):
            assert torch.equal(got, want), rep


@pytest.mark.parametrize("kind", ["loss", "rmsd", "long", "anchor_grads"])
def test_extension_steps_replay(device, kind):
    """The fused coordinate loss and RMSD, long chains (several segments, so every long-chain
    pass is in the graph) and anchor gradients: captured and replayed as the plain step."""
    import cufk_amd

    B, N = (6, 3000) if kind == "long" else (64, 700)
    s = _set(B, N, 12, torch.float32, device)
    names = ("lengths", "angles", "dihedrals", "p0", "first_direction", "initial_normal")
    grad_anchors = kind == "anchor_grads"
    ins = [s[k].clone().requires_grad_(i < 3 or grad_anchors) for i, k in enumerate(names)]
    extra = s["grad"].clone()  # the target of the losses, the upstream gradient otherwise

    def step(L, A, D, p0, fd, n0, extra):
        if kind == "loss":
            out = cufk_amd.reconstruct_loss(L, A, D, extra, p0, fd, n0)
        elif kind == "rmsd":
            out = cufk_amd.reconstruct_rmsd(L, A, D, extra, p0, fd, n0)
        elif kind == "long":
            out = cufk_amd.reconstruct_long(L, A, D, p0, fd, n0, segment_steps=512)
        else:
            out = cufk_amd.reconstruct(L, A, D, p0, fd, n0, anchor_grads=True)
        upstream = torch.ones_like(out) if kind in ("loss", "rmsd") else extra
        wrt = (L, A, D, p0, fd, n0) if grad_anchors else (L, A, D)
        return (out, *torch.autograd.grad(out, wrt, upstream))

    graph, out = _capture(step, (*ins, extra))
    for rep in range(4):
        t = _set(B, N, 200 + rep, torch.float32, device)
        with torch.no_grad():
            for dst, k in zip(ins, names):
                dst.copy_(t[k])
            extra.copy_(t["grad"])
        graph.replay()
        ref = step(*(t[k].clone().requires_grad_(i < 3 or grad_anchors) for i, k in enumerate(names)), t["grad"].clone())
        torch.cuda.synchronize()
        for got, want in zip(out, ref):
            assert torch.equal(got, want), (kind, rep)

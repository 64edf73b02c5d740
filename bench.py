"""Benchmark: fwd+bwd atoms/sec of cufk_amd.reconstruct at B=4096, N=2049 fp32 on one MI355X.

A step is one forward + backward pass of the reconstruction path over one batch of synthetic
chains (config 2 draws: lengths ~N(0.145, 0.01) clipped to [0.12, 0.17], angles ~N(2.05,
0.08), dihedrals ~U(-pi, pi), random anchors, upstream grad ~N(0, 1)), with every input
already resident in HBM.  The step runs through the public autograd API
(``reconstruct`` + ``torch.autograd.grad``).

The default 1000 warm-up steps (about 0.1 s of GPU work at config 2) bring the GPU to its
steady clocks: after only 10 warm-up steps the first 50 timed steps run about 20 % slower.
The timed steps rotate over ``--sets`` independent input batches (3 by default, about 1.2 GB
at config 2), so no step finds its inputs in the 256 MB last-level cache left behind by the
previous one.  HIP events recorded inside the timed region on the stream the kernels run on
(the current torch stream, which the extension launches on) bracket the K timed steps; a second
pass of K steps puts events around each step's forward call and around its backward node
(autograd pre- and post-hooks), which splits the step.  ``roofline`` is for the backward: its
algorithmic bytes per launch are 4*B*(9N-12) (read lengths, angles, dihedrals and grad_xyz,
write the three gradients), divided by the backward node's average duration over that second
pass (the kernel as the timed steps run it, which is what rocprofv3's kernel trace of the same
command averages), against MI355X's 8 TB/s HBM peak.  ``traffic`` is the HBM bytes per launch
the rocprofv3 FETCH_SIZE and WRITE_SIZE counters read for the same kernel, copied from the
committed summaries under profiles/ (MEASURED_TRAFFIC below).  ``abi_*_us`` time each C-ABI
entry point alone over back-to-back launches rotating over the input sets (an event pair per
launch); a backward launched after another backward, not after its forward, no longer finds the
forward's output in the last-level cache, so those run slower than in the step.

The CPU baseline is the float64 numpy oracle (oracle/nerf64.py) run on this host on a bounded
sample of chains of the same shape (chunks of about 128 x 2049 points until about 15 s of work),
scaled to atoms/s.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config c2|c1|c3|c4_bf16|c4_fp16|long|short|loss]
                    [--graph]

With --graph each input set's step is captured once in a HIP graph (torch.cuda.graph) and the
timed steps replay the graphs: the kernels are the same, the per-step Python, autograd-engine and
launch overhead is gone (which is what bounds small configs such as c1).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0

CONFIGS = {
    # name: (kind, dtype, B, N)
    "c1": ("reconstruct", "float32", 1024, 384),
    "c2": ("reconstruct", "float32", 4096, 2049),
    "c3": ("torsion", "float32", 8192, 771),
    "c4_bf16": ("reconstruct", "bfloat16", 16384, 1026),
    "c4_fp16": ("reconstruct", "float16", 16384, 1026),
    # Past the 2051-point cap (reconstruct_long): C2's atom count as 64 chains of 131075 points,
    # 64 segments of 2048 steps each.
    "long": ("long", "float32", 64, 131075),
    # Short chains packed several per wave: C2's atom count as 131072 chains of 64 points.
    "short": ("reconstruct", "float32", 131072, 64),
    # reconstruct_loss (reconstruction fused with a per-chain coordinate loss) at C2's shape; the
    # unfused composition (reconstruct, then the loss in torch) is timed beside it.
    "loss": ("loss", "float32", 4096, 2049),
}
BOND_LENGTHS = (0.14685231, 0.15365194, 0.13405086)
BOND_ANGLES = (1.9676635, 2.062335, 2.164016)
DTYPE_CODES = {"float32": 0, "float64": 1, "float16": 2, "bfloat16": 3}
ELEM_BYTES = {"float32": 4, "float64": 8, "float16": 2, "bfloat16": 2}

# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, each scaled by what the
# counter reads for a plain copy of known size; see profiles/reconstruct_c2_hbm_traffic.md.
# Keyed by (config, kernel); a missing entry reports traffic as null.
MEASURED_TRAFFIC = {
    ("c2", "reconstruct_backward"): 303494325,  # 202665849 read (xyz, grad_xyz) + 100828476 written
}


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=500)
    p.add_argument("--warmup", type=int, default=1000)
    p.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    p.add_argument("--kernel-reps", type=int, default=200)
    p.add_argument("--sets", type=int, default=3, help="independent input batches the steps rotate over")
    p.add_argument("--graph", action="store_true",
                   help="capture each input set's step (forward + torch.autograd.grad) in a HIP graph and time replays")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-sample", type=int, default=0, help="chains in the CPU sample (0 = about 15 s of work)")
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                   help="only run a plain device-to-device copy of MIB MiB (HBM counter calibration) and exit")
    return p.parse_args()


def copy_probe(mib):
    """A plain copy kernel of known size: reads and writes exactly mib MiB once per launch."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    ms = event_time_ms(torch, lambda i: dst.copy_(src), 10)
    print(json.dumps({"copy_probe_mib": mib, "avg_us": ms * 1e3, "GBs_read_plus_write": 2 * n * 4 / (ms * 1e-3) / 1e9}))
    return 0


def synthetic(B, N, seed, torch, device, dtype):
    gen = torch.Generator().manual_seed(seed)
    L = (torch.randn(B, N - 1, generator=gen, dtype=torch.float64) * 0.01 + 0.145).clamp_(0.12, 0.17)
    A = torch.randn(B, N - 2, generator=gen, dtype=torch.float64) * 0.08 + 2.05
    D = (torch.rand(B, N - 3, generator=gen, dtype=torch.float64) * 2 - 1) * np.pi
    g = torch.randn(B, N, 3, generator=gen, dtype=torch.float64)
    p0 = torch.randn(3, generator=gen, dtype=torch.float64)
    q, _ = torch.linalg.qr(torch.randn(3, 3, generator=gen, dtype=torch.float64))
    cast = lambda t: t.to(device=device, dtype=dtype).contiguous()  # noqa: E731
    return cast(L), cast(A), cast(D), cast(g), cast(p0), cast(q[:, 0]), cast(q[:, 1])


def event_time_ms(torch, fn, reps):
    """Average duration of fn(i) over reps back-to-back calls (i = 0..reps-1): a pair of HIP
    events on the current stream brackets each call, so the average is the launch's own
    duration (what rocprofv3's kernel trace reports), without the gaps between launches."""
    stream = torch.cuda.current_stream()
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    fn(0)
    torch.cuda.synchronize()
    for i in range(reps):
        marks[i][0].record(stream)
        fn(i)
        marks[i][1].record(stream)
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in marks) / reps


def coordinate_error_by_position(torch, cufk_amd, B, N, dtype, device, chains=64):
    """Coordinate error of `dtype` against the float64 path on the same (rounded) inputs, over
    `chains` chains drawn like the timed inputs (outside the timed region): RMS over chains and
    coordinates, and max-abs, at chain positions 0, N/10, ..., N-1, plus over the whole chain.
    The float64 path is the library's own (within 1e-12 of the CPU oracle in the GPU tests)."""
    n = min(B, chains)
    L, A, D, _, p0, fd, n0 = synthetic(n, N, 2, torch, device, dtype)
    with torch.no_grad():
        x = cufk_amd.reconstruct(L, A, D, p0, fd, n0).double()
        r = cufk_amd.reconstruct(*(t.double() for t in (L, A, D, p0, fd, n0)))
    d = x - r
    rms_pos = d.pow(2).sum(-1).mean(0).sqrt()  # (N,)
    max_pos = d.abs().amax(dim=(0, 2))
    marks = sorted({round(i * (N - 1) / 10) for i in range(11)})
    return {
        "reference": "float64 reconstruct on the same rounded inputs",
        "chains": n,
        "unit": "input length unit (nm)",
        "positions": marks,
        "rms": [float(rms_pos[i]) for i in marks],
        "max_abs": [float(max_pos[i]) for i in marks],
        "rms_all": float(d.pow(2).sum(-1).mean().sqrt()),
        "max_abs_all": float(d.abs().max()),
    }


def cpu_baseline(kind, B, N, sample, seconds):
    """Float64 oracle fwd + bwd on a bounded sample of chains, scaled to atoms/s.

    Chains are processed in chunks of at most 128 (bounding memory).  With sample == 0,
    chunks run until about `seconds` of work is done or B chains are covered; otherwise exactly
    `sample` chains.  A 4-chain warm-up (1 chain for chains past 65k points) is not counted.
    Returns (atoms/s, chains, wall seconds, cpu seconds)."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import nerf64 as o

    def chunk(n, seed):
        if kind == "torsion":
            rng = np.random.default_rng(seed)
            raw = rng.normal(size=(n, 2 * (N - 3)))
            g = rng.normal(size=(n, N, 3))
            c = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)
            t0, c0 = time.perf_counter(), time.process_time()
            x = o.torsion_forward(raw, c)
            o.torsion_backward(raw, x, g, c)
        else:
            d = o.synthetic_inputs(n, N, seed=seed, anchors=True)
            an = dict(p0=d["p0"], first_direction=d["first_direction"], initial_normal=d["initial_normal"])
            t0, c0 = time.perf_counter(), time.process_time()
            o.reconstruct_forward(d["lengths"], d["angles"], d["dihedrals"], **an)
            o.reconstruct_backward(d["lengths"], d["angles"], d["dihedrals"], d["grad"], **an)
        return time.perf_counter() - t0, time.process_time() - c0

    per_chunk = max(1, min(128, 128 * 2049 // N))  # about 128 x 2049 points per chunk
    chunk(4 if per_chunk >= 4 else 1, 1000)
    limit = sample if sample > 0 else B
    wall = cpu = 0.0
    done = 0
    while done < limit and (sample > 0 or wall < seconds):
        n = min(per_chunk, limit - done)
        w, c = chunk(n, 2 + done)
        wall += w
        cpu += c
        done += n
    return done * N / wall, done, wall, cpu


def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only; --gpus {args.gpus} is not supported (chains shard over the batch "
            "with no communication, so N GPUs run B/N chains each).",
            file=sys.stderr,
        )
        return 2

    if args.copy_probe:
        return copy_probe(args.copy_probe)

    import torch

    import cufk_amd

    kind, dtype_name, B, N = CONFIGS[args.config]
    dtype = getattr(torch, dtype_name)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    nsets = max(1, args.sets)
    s = ELEM_BYTES[dtype_name]
    code = DTYPE_CODES[dtype_name]
    lib = ctypes.CDLL(str(cufk_amd._native.HIP_LIBRARY))  # the library the extension links
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    i64 = ctypes.c_int64

    # One entry per input set: the autograd step and the two C-ABI calls it makes.
    steps, fwds, bwds, regular = [], [], [], []
    if kind == "long":
        # Algorithmic bytes as for reconstruct; the segment joins (placement, segment sums)
        # are extra traffic the roofline fraction is charged with.
        fwd_bytes = s * B * (6 * N - 6)
        bwd_bytes = s * B * (9 * N - 12)
        lib.cufk_long_segment_steps.restype = i64
        seg = lib.cufk_long_segment_steps(i64(B), i64(N))
        lib.cufk_long_state_doubles.restype = i64
        lib.cufk_long_work_doubles.restype = i64
        n_state = lib.cufk_long_state_doubles(i64(B), i64(N), i64(seg))
        n_work = lib.cufk_long_work_doubles(i64(B), i64(N), i64(seg))
        assert n_state > 0 and n_work > 0
        for k in range(nsets):
            L, A, D, g, p0, fd, n0 = synthetic(B, N, 2 + k, torch, device, dtype)
            for t in (L, A, D):
                t.requires_grad_(True)

            def step(L=L, A=A, D=D, g=g, p0=p0, fd=fd, n0=n0, mark=None):
                xyz = cufk_amd.reconstruct_long(L, A, D, p0, fd, n0)
                if mark is not None:
                    mark(xyz)
                return torch.autograd.grad(xyz, (L, A, D), g)

            xyz = torch.empty(B, N, 3, device=device, dtype=dtype)
            state = torch.empty(n_state, device=device, dtype=torch.float64)
            work = torch.empty(n_work, device=device, dtype=torch.float64)
            gL, gA, gD = torch.empty_like(L), torch.empty_like(A), torch.empty_like(D)

            def fwd(st, L=L, A=A, D=D, p0=p0, fd=fd, n0=n0, xyz=xyz, state=state):
                rc = lib.cufk_reconstruct_long_fwd(code, P(L), P(A), P(D), P(p0), P(fd), P(n0), P(xyz), P(state),
                                                   i64(B), i64(N), i64(seg), st)
                assert rc == 0, rc

            def bwd(st, L=L, A=A, D=D, p0=p0, fd=fd, n0=n0, xyz=xyz, state=state, g=g, work=work, gL=gL, gA=gA,
                    gD=gD):
                rc = lib.cufk_reconstruct_long_bwd(code, P(L), P(A), P(D), P(p0), P(fd), P(n0), P(xyz), P(state),
                                                   P(g), P(work), P(gL), P(gA), P(gD), i64(B), i64(N), i64(seg), st)
                assert rc == 0, rc

            fwd(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))  # state for the ABI backward
            steps.append(step)
            fwds.append(fwd)
            bwds.append(bwd)
    elif kind == "loss":
        # Forward reads the parameters and the target and writes xyz (s(9N-6)); backward reads
        # xyz and the target and writes the three gradient rows (s(9N-6)): grad_xyz never
        # exists, and the loss terms never leave the kernels.
        fwd_bytes = s * B * (9 * N - 6)
        bwd_bytes = s * B * (9 * N - 6)
        unfused = []
        for k in range(nsets):
            L, A, D, g, p0, fd, n0 = synthetic(B, N, 2 + k, torch, device, dtype)
            target = g * 0.3  # any (B, N, 3) tensor: the loss only shifts by a constant
            for t in (L, A, D):
                t.requires_grad_(True)

            def step(L=L, A=A, D=D, target=target, p0=p0, fd=fd, n0=n0, mark=None):
                loss = cufk_amd.reconstruct_loss(L, A, D, target, p0, fd, n0)
                if mark is not None:
                    mark(loss)
                return torch.autograd.grad(loss.sum(), (L, A, D))

            def plain(L=L, A=A, D=D, target=target, p0=p0, fd=fd, n0=n0):
                xyz = cufk_amd.reconstruct(L, A, D, p0, fd, n0)
                return torch.autograd.grad(((xyz - target) ** 2).sum(), (L, A, D))

            loss_out = torch.empty(B, device=device, dtype=dtype)
            xyz = torch.empty(B, N, 3, device=device, dtype=dtype)
            flags = torch.empty(B, device=device, dtype=torch.uint8)
            gL, gA, gD = torch.empty_like(L), torch.empty_like(A), torch.empty_like(D)

            def fwd(st, L=L, A=A, D=D, target=target, p0=p0, fd=fd, n0=n0, xyz=xyz, flags=flags, loss_out=loss_out):
                rc = lib.cufk_reconstruct_loss_fwd(code, P(L), P(A), P(D), P(p0), P(fd), P(n0), P(target), P(xyz),
                                                   P(flags), P(loss_out), i64(B), i64(N), st)
                assert rc == 0, rc

            def bwd(st, L=L, A=A, D=D, target=target, p0=p0, fd=fd, n0=n0, xyz=xyz, flags=flags, gL=gL, gA=gA, gD=gD):
                rc = lib.cufk_reconstruct_loss_bwd(code, P(L), P(A), P(D), P(p0), P(fd), P(n0), P(xyz), P(flags),
                                                   P(target), None, P(gL), P(gA), P(gD), i64(B), i64(N), st)
                assert rc == 0, rc

            steps.append(step)
            fwds.append(fwd)
            bwds.append(bwd)
            unfused.append(plain)
    elif kind == "reconstruct":
        fwd_bytes = s * B * (6 * N - 6)
        bwd_bytes = s * B * (9 * N - 12)
        for k in range(nsets):
            L, A, D, g, p0, fd, n0 = synthetic(B, N, 2 + k, torch, device, dtype)
            L.requires_grad_(True)
            A.requires_grad_(True)
            D.requires_grad_(True)

            def step(L=L, A=A, D=D, g=g, p0=p0, fd=fd, n0=n0, mark=None):
                xyz = cufk_amd.reconstruct(L, A, D, p0, fd, n0)
                if mark is not None:
                    mark(xyz)
                return torch.autograd.grad(xyz, (L, A, D), g)

            xyz = torch.empty(B, N, 3, device=device, dtype=dtype)
            flags = torch.empty(B, device=device, dtype=torch.uint8)
            gL, gA, gD = torch.empty_like(L), torch.empty_like(A), torch.empty_like(D)

            # The entry points the autograd path uses: the flagged forward and the backward
            # that takes the forward's output (position-based adjoint for regular chains);
            # float16/bfloat16 keep a float copy of the positions for it instead.
            lib.cufk_reconstruct_shadow_floats.restype = i64
            if s == 2 and lib.cufk_reconstruct_shadow_floats(i64(B), i64(N)) > 0:
                pos = torch.empty(B, N, 3, device=device, dtype=torch.float32)

                def fwd(st, L=L, A=A, D=D, p0=p0, fd=fd, n0=n0, xyz=xyz, pos=pos, flags=flags):
                    rc = lib.cufk_reconstruct_fwd_shadow(code, P(L), P(A), P(D), P(p0), P(fd), P(n0), P(xyz), P(pos),
                                                         P(flags), i64(B), i64(N), st)
                    assert rc == 0, rc

                def bwd(st, L=L, A=A, D=D, p0=p0, fd=fd, n0=n0, pos=pos, flags=flags, g=g, gL=gL, gA=gA, gD=gD):
                    rc = lib.cufk_reconstruct_bwd_shadow(code, P(L), P(A), P(D), P(p0), P(fd), P(n0), P(pos), P(flags),
                                                         P(g), P(gL), P(gA), P(gD), i64(B), i64(N), st)
                    assert rc == 0, rc
            else:

                def fwd(st, L=L, A=A, D=D, p0=p0, fd=fd, n0=n0, xyz=xyz, flags=flags):
                    rc = lib.cufk_reconstruct_fwd_flagged(code, P(L), P(A), P(D), P(p0), P(fd), P(n0), P(xyz),
                                                          P(flags), i64(B), i64(N), st)
                    assert rc == 0, rc

                def bwd(st, L=L, A=A, D=D, p0=p0, fd=fd, n0=n0, xyz=xyz, flags=flags, g=g, gL=gL, gA=gA, gD=gD):
                    rc = lib.cufk_reconstruct_bwd_saved(code, P(L), P(A), P(D), P(p0), P(fd), P(n0), P(xyz),
                                                        P(flags), P(g), P(gL), P(gA), P(gD), i64(B), i64(N), st)
                    assert rc == 0, rc

            steps.append(step)
            fwds.append(fwd)
            bwds.append(bwd)
            regular.append(flags)
    else:
        import math

        class Consts(ctypes.Structure):
            _fields_ = [("length", ctypes.c_float * 3), ("sin", ctypes.c_double * 3), ("cos", ctypes.c_double * 3)]

        c = Consts((ctypes.c_float * 3)(*BOND_LENGTHS), (ctypes.c_double * 3)(*[math.sin(a) for a in BOND_ANGLES]),
                   (ctypes.c_double * 3)(*[math.cos(a) for a in BOND_ANGLES]))
        f = cufk_amd.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
        fwd_bytes = s * B * (5 * N - 6)
        bwd_bytes = s * B * (10 * N - 12)
        for k in range(nsets):
            gen = torch.Generator().manual_seed(3 + k)
            raw = torch.randn(B, 2 * (N - 3), generator=gen, dtype=torch.float64).to(device=device, dtype=dtype)
            g = torch.randn(B, N, 3, generator=gen, dtype=torch.float64).to(device=device, dtype=dtype)
            raw.requires_grad_(True)

            def step(raw=raw, g=g, mark=None):
                xyz = f(raw)
                if mark is not None:
                    mark(xyz)
                return torch.autograd.grad(xyz, (raw,), g)

            xyz = torch.empty(B, N, 3, device=device, dtype=dtype)
            graw = torch.empty_like(raw)

            def fwd(st, raw=raw, xyz=xyz):
                rc = lib.cufk_torsion_fwd(code, P(raw), i64(raw.stride(0)), ctypes.byref(c), P(xyz), i64(B), i64(N), st)
                assert rc == 0, rc

            def bwd(st, raw=raw, xyz=xyz, g=g, graw=graw):
                rc = lib.cufk_torsion_bwd(code, P(raw), i64(raw.stride(0)), P(xyz), P(g), P(graw), i64(graw.stride(0)),
                                          ctypes.byref(c), i64(B), i64(N), st)
                assert rc == 0, rc

            steps.append(step)
            fwds.append(fwd)
            bwds.append(bwd)

    if args.graph:
        # One graph per input set: warm up on a side stream, capture, then the timed steps
        # replay (no per-step Python, autograd engine or launch overhead).
        graphs = []
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for k in range(nsets):
                for _ in range(3):
                    steps[k]()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for k in range(nsets):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                steps[k]()
            graphs.append(graph)
        steps = [graph.replay for graph in graphs]

    for i in range(args.warmup):
        steps[i % nsets]()
    torch.cuda.synchronize()

    # Timed region: K steps back to back on the stream the kernels run on.
    stream = torch.cuda.current_stream()
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    t_start, t_end = ev(), ev()
    torch.cuda.synchronize()
    t_start.record(stream)
    for i in range(args.steps):
        steps[i % nsets]()
    t_end.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t_start.elapsed_time(t_end) / args.steps

    # The same K steps again with events around each step's forward call and around its
    # backward node (autograd pre- and post-hooks on the output's grad_fn, run on the same
    # stream right before and after the node launches its kernel).  The extra event packets
    # cost a little per step, so this pass is reported apart from ms_per_step.
    marks = [(ev(), ev(), ev(), ev()) for _ in range(0 if args.graph else args.steps)]

    def marker(m):
        def mark(out):
            m[1].record(stream)
            out.grad_fn.register_prehook(lambda grad_out: m[2].record(stream))
            out.grad_fn.register_hook(lambda grad_in, grad_out: m[3].record(stream))

        return mark

    torch.cuda.synchronize()
    for i in range(len(marks)):
        marks[i][0].record(stream)
        steps[i % nsets](mark=marker(marks[i]))
    torch.cuda.synchronize()
    seg_fwd = sum(m[0].elapsed_time(m[1]) for m in marks) / len(marks) if marks else None
    seg_bwd = sum(m[2].elapsed_time(m[3]) for m in marks) / len(marks) if marks else None

    # Kernel-level timing straight through the C ABI, rotating over the same sets.
    st = ctypes.c_void_p(stream.cuda_stream)
    t_fwd = event_time_ms(torch, lambda i: fwds[i % nsets](st), args.kernel_reps)
    t_bwd = event_time_ms(torch, lambda i: bwds[i % nsets](st), args.kernel_reps)
    regular_frac = float(torch.stack(regular).float().mean()) if regular else None

    unfused_us = None
    if kind == "loss":  # the same step through reconstruct and a torch loss, same input sets
        for i in range(args.warmup // 4):
            unfused[i % nsets]()
        torch.cuda.synchronize()
        u0, u1 = ev(), ev()
        u0.record(stream)
        for i in range(args.steps):
            unfused[i % nsets]()
        u1.record(stream)
        torch.cuda.synchronize()
        unfused_us = u0.elapsed_time(u1) / args.steps * 1e3

    precision = None
    if kind == "reconstruct":
        precision = coordinate_error_by_position(torch, cufk_amd, B, N, dtype, device)

    atoms = B * N
    # The backward kernel as the timed steps run it; replayed graphs hold no events, so with
    # --graph the C-ABI launches stand in.
    bwd_ms = seg_bwd if seg_bwd is not None else t_bwd
    fwd_ms = seg_fwd if seg_fwd is not None else t_fwd
    bw_bwd = bwd_bytes / (bwd_ms * 1e-3) / 1e9
    bw_fwd = fwd_bytes / (fwd_ms * 1e-3) / 1e9
    traffic = MEASURED_TRAFFIC.get((args.config, f"{kind}_backward"))
    result = {
        "metric": "fwd+bwd atoms/sec @ B=4096 N=2049 fp32; % of HBM roofline",
        "value": atoms / (ms_per_step * 1e-3),
        "unit": "atoms/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"float32": "f32", "float64": "f64", "float16": "f16", "bfloat16": "bf16"}[dtype_name],
        "data": "synthetic",
        "config": {"workload": f"{kind} fwd+bwd" + (", replayed HIP graph" if args.graph else ""),
                   "config": args.config, "batch": B, "points": N, "dtype": dtype_name, "anchors": "random",
                   "input_sets": nsets},
        "roofline": {
            "bound": "hbm",
            "kernel": f"{kind}_backward",
            "achieved": bw_bwd,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": bw_bwd / HBM_PEAK_GBS,
            "traffic": traffic,
            "algorithmic_bytes": bwd_bytes,
            "avg_launch_us": bwd_ms * 1e3,
        },
        "kernels": {
            "step_forward_us": seg_fwd * 1e3 if seg_fwd is not None else None,
            "step_backward_us": seg_bwd * 1e3 if seg_bwd is not None else None,
            "step_forward_GBs": bw_fwd,
            "step_backward_GBs": bw_bwd,
            "abi_forward_us": t_fwd * 1e3,
            "abi_backward_us": t_bwd * 1e3,
            "step_frac_of_hbm_peak": (fwd_bytes + bwd_bytes) / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "regular_chain_fraction": regular_frac,
            "unfused_step_us": unfused_us,
        },
    }
    if precision is not None:
        result["precision"] = precision
    if not args.no_cpu_baseline:
        v, chains, wall, cpu = cpu_baseline(kind, B, N, args.cpu_sample, args.cpu_seconds)
        result["cpu_baseline"] = {
            "value": v,
            "unit": "atoms/s",
            "cores": max(1, round(cpu / wall)),
            "kind": "port",
            "sample": f"float64 numpy oracle, fwd+bwd of {chains} chains x N={N} ({wall:.1f} s wall, "
                      f"{cpu:.1f} s cpu), scaled to atoms/s",
        }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Benchmark: fwd+bwd atoms/sec of cufk_amd.reconstruct at B=4096, N=2049 fp32 on one MI355X.

A step is one forward + backward pass of the reconstruction path over one batch of synthetic
chains (config 2 draws: lengths ~N(0.145, 0.01) clipped to [0.12, 0.17], angles ~N(2.05,
0.08), dihedrals ~U(-pi, pi), random anchors, upstream grad ~N(0, 1)), with every input
already resident in HBM.  The step runs through the public autograd API
(``reconstruct`` + ``torch.autograd.grad``).

Order of work:
1. Clock ramp: steps are run for ``--ramp-s`` seconds (0.5 s by default) before the W warm-up
   steps, so a short ``--warmup`` still times the GPU at its steady clocks (after only a few
   warm-up steps the first 50 timed steps run about 20 % slower).  Reported as
   ``config.ramp_steps``; none of it is timed.
2. W warm-up steps, then the K timed steps back to back, bracketed by synchronize and a pair of
   HIP events on the stream the kernels run on: ``ms_per_step`` and ``value`` = B*N / step.
   The steps rotate over ``--sets`` independent input batches (3 by default, about 1.2 GB at
   config 2), so no step finds its inputs in the 256 MB last-level cache.
3. Forward only: K forward calls without autograd, timed the same way (``forward_atoms_per_s``).
4. Kernel split: K (or ``--abi-reps``) back-to-back launches of the step's forward C-ABI entry
   point, then of its backward entry point over each set's saved forward output, each under one
   event pair: ``kernels.forward_us``, ``backward_us``, and ``step_gap_us`` = the step minus both.
   ``--phases`` splits a rocprofv3 kernel trace of the same command into the kernels' in-step
   and back-to-back durations.
5. For reconstruct and torsion configs run eagerly, the same step replayed from one HIP graph
   per input set (``kernels.graph_step_us``; ``--no-graph-too`` skips it).
6. For c1 (or any reconstruct config with ``--host-breakdown``), the host time of the eager
   step's pieces (``host``): the public forward, ``_C.apply`` alone, the backward alone, the
   autograd engine's own hand-off for a one-op graph, the two C-ABI calls, the whole step.

``roofline`` is for the step, the metric's own quantity: (forward + backward algorithmic bytes)
/ ms_per_step against MI355X's 8 TB/s HBM peak.  Algorithmic bytes per chain: forward s(6N-6)
(read lengths, angles, dihedrals; write xyz), backward s(9N-12) (read the three parameter rows'
worth and grad_xyz; write the three gradients).  ``traffic`` is what rocprofv3's FETCH_SIZE and
WRITE_SIZE counters read for the step's kernels (MEASURED_TRAFFIC below, copied from the
committed summary under profiles/).  ``roofline_valu`` is the VALU roofline of the step's
forward launch: its VALU instructions (MEASURED_VALU) over its duration (pass 4) against the
1024 SIMDs' issue rate.  ``kernels`` splits the step: forward and backward
durations from pass 4 and each one's fraction of the HBM peak.

The CPU baseline is the reference algorithm on this host's cores: serial float64 NeRF
(forward, then the explicit reverse adjoint) in PyTorch CPU (oracle/cpu_torch.py), vectorised
over the chains with torch's intra-op threads, the median of 3 runs over the config's batch (or
a subset of it where one run would take longer than about 20 s), scaled to atoms/s.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config NAME] [--graph]

NAME is one of CONFIGS below: c1, c2 (the default, BASELINE.json's headline), c3, c4_bf16,
c4_fp16, the extensions long, short, loss, rmsd, torsion_loss, and c2_far / c2_mixed (C2 with
chains that take the exact backward).

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
    # reconstruct_rmsd (the reconstruction fused with the RMSD after optimal superposition) at
    # C2's shape, against reconstruct followed by the Kabsch superposition in torch.
    "rmsd": ("rmsd", "float32", 4096, 2049),
    # compile_torsion(...).loss (the torsion path fused with a coordinate loss) at C3's shape,
    # against the torsion path followed by the loss in torch.
    "torsion_loss": ("torsion_loss", "float32", 8192, 771),
    # C2 with chains the position-based backward does not take (the exact recompute runs for
    # them inside the same backward launch): every chain placed about 50 nm from the origin
    # (p0 = (50, 0, 0) nm, past 256 of the shortest 0.12 nm bonds), and one chain in four with
    # a near-straight bond angle (2.7 rad: sin 0.43 < 0.5).
    "c2_far": ("reconstruct", "float32", 4096, 2049),
    "c2_mixed": ("reconstruct", "float32", 4096, 2049),
}
# What the exact-fallback configs change in the C2 draws (see synthetic()).
IRREGULAR = {"c2_far": "far", "c2_mixed": "every:4"}
BOND_LENGTHS = (0.14685231, 0.15365194, 0.13405086)
BOND_ANGLES = (1.9676635, 2.062335, 2.164016)
DTYPE_CODES = {"float32": 0, "float64": 1, "float16": 2, "bfloat16": 3}
ELEM_BYTES = {"float32": 4, "float64": 8, "float16": 2, "bfloat16": 2}

# HBM bytes per step (every kernel of the forward and backward launches) from rocprofv3 --pmc
# FETCH_SIZE / WRITE_SIZE in the bench's own regime, each counter scaled by what it reads for a
# plain copy of known size, and the wave64 VALU instructions (SQ_INSTS_VALU) of the forward and
# backward launches: profiles/counters_and_traffic_bench_regime.md.  A config without an entry
# reports traffic and roofline_valu as null.
MEASURED_TRAFFIC = {
    "c1": 24429892, "c2": 510976820, "c2_far": 511569622, "c2_mixed": 511340596, "c3": 380682861,
    "c4_bf16": 827142795, "long": 914240077, "loss": 613084106, "rmsd": 616138701, "torsion_loss": 458950537,
    "short": 500206727,
}
MEASURED_VALU = {  # (forward, backward) per launch
    "c1": (1796096, 1122816), "c2": (20185088, 14049280), "c2_far": (20185088, 49795072),
    "c2_mixed": (20184064, 22985728), "c3": (10616832, 11608064), "c4_bf16": (42958848, 30072832),
    "long": (22353856, 22759616), "loss": (22122496, 14872576), "rmsd": (36209664, 18583002),
    "torsion_loss": (12034048, 12230656), "short": (27754496, 23560192),
}
# VALU issue peak: 1024 SIMDs (256 CUs x 4) at 2.4 GHz, one wave64 instruction per 4 cycles each.
VALU_PEAK_PER_S = 1024 * 2.4e9 / 4


HEADLINE_METRIC = "fwd+bwd atoms/sec @ B=4096 N=2049 fp32; % of HBM roofline"  # BASELINE.json's metric


def metric_name(config):
    """The metric a config's line measures: BASELINE.json's headline for c2, the same quantity
    named with its own kind, shape and dtype for the others."""
    if config == "c2":
        return HEADLINE_METRIC
    kind, dtype_name, B, N = CONFIGS[config]
    short = {"float32": "fp32", "float64": "fp64", "float16": "fp16", "bfloat16": "bf16"}[dtype_name]
    return f"{kind} fwd+bwd atoms/sec @ B={B} N={N} {short} ({config}); % of HBM roofline"


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=500)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--ramp-s", type=float, default=0.5,
                   help="seconds of untimed steps before the warm-up steps (GPU clock ramp)")
    p.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    p.add_argument("--abi-reps", type=int, default=0,
                   help="back-to-back launches of each C-ABI entry point to time (0 = skip)")
    p.add_argument("--sets", type=int, default=3, help="independent input batches the steps rotate over")
    p.add_argument("--graph", action="store_true",
                   help="capture each input set's step (forward + torch.autograd.grad) in a HIP graph and time replays")
    p.add_argument("--irregular", metavar="PATTERN",
                   help="reconstruct configs: chains the position-based backward refuses, as 'far' (p0 50 nm from "
                        "the origin), 'every:K' (every K-th chain) or 'first:F' (the first fraction F of the chains)")
    p.add_argument("--phases", metavar="KERNEL_TRACE_CSV",
                   help="only split a rocprofv3 kernel trace of a bench run into its in-step and back-to-back "
                        "phases (JSON) and exit; needs no GPU")
    p.add_argument("--host-breakdown", action="store_true",
                   help="reconstruct configs: time the host side of an eager step by piece (always on for c1)")
    p.add_argument("--no-graph-too", dest="graph_too", action="store_false",
                   help="skip timing the step replayed from HIP graphs beside the eager step")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-runs", type=int, default=3, help="CPU baseline runs (the median is reported)")
    p.add_argument("--cpu-seconds", type=float, default=20.0, help="rough cap on one CPU baseline run")
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


def synthetic(B, N, seed, torch, device, dtype, irregular=None):
    """Config 2 draws.  irregular="far" moves p0 to (50, 0, 0) nm, so every chain sits past
    the fp32 position-based backward's extent test; "every:K" sets the middle bond angle of
    every K-th chain (chains 0, K, 2K, ...) to 2.7 rad, past its angle test (sin 0.43 < 0.5);
    "first:F" does the same to the first fraction F of the chains (one contiguous block)."""
    gen = torch.Generator().manual_seed(seed)
    L = (torch.randn(B, N - 1, generator=gen, dtype=torch.float64) * 0.01 + 0.145).clamp_(0.12, 0.17)
    A = torch.randn(B, N - 2, generator=gen, dtype=torch.float64) * 0.08 + 2.05
    D = (torch.rand(B, N - 3, generator=gen, dtype=torch.float64) * 2 - 1) * np.pi
    g = torch.randn(B, N, 3, generator=gen, dtype=torch.float64)
    p0 = torch.randn(3, generator=gen, dtype=torch.float64)
    q, _ = torch.linalg.qr(torch.randn(3, 3, generator=gen, dtype=torch.float64))
    if irregular == "far":
        p0 = torch.tensor([50.0, 0.0, 0.0], dtype=torch.float64)
    elif irregular is not None and irregular.startswith("every:"):
        A[:: int(irregular[6:]), (N - 2) // 2] = 2.7
    elif irregular is not None and irregular.startswith("first:"):
        A[: round(B * float(irregular[6:])), (N - 2) // 2] = 2.7
    elif irregular is not None:
        raise ValueError(f"unknown irregular pattern {irregular!r}")
    cast = lambda t: t.to(device=device, dtype=dtype).contiguous()  # noqa: E731
    return cast(L), cast(A), cast(D), cast(g), cast(p0), cast(q[:, 0]), cast(q[:, 1])


def event_time_ms(torch, fn, reps):
    """Average time per call of fn(i) over reps back-to-back calls (i = 0..reps-1), under one
    pair of HIP events on the current stream: each call's own duration plus the short gap
    between launches (an event pair around each call would add a few microseconds per call)."""
    stream = torch.cuda.current_stream()
    fn(0)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(reps):
        fn(i)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def kernel_direction(name):
    """Which half of a step a library kernel belongs to, from its name (None: not ours)."""
    if "cufk_amd" not in name:  # demangled (cufk_amd::...) or mangled (..8cufk_amd..) names
        return None
    if "backward" in name or "anchor_gradients" in name:
        return "backward"
    if "forward" in name or "superpose_records" in name:
        return "forward"
    return None


def trace_phases(path):
    """Split a rocprofv3 kernel trace (``--kernel-trace --output-format csv``) of one bench run
    into its phases by the order of our dispatches: a forward or backward kernel between two of
    the other direction ran inside a step; one between two of its own direction ran back to back
    (the C-ABI passes).  Returns, per phase, the dispatch count and the mean and median duration
    of each direction, and the median gap from the previous dispatch's end (microseconds)."""
    import csv

    with open(path, newline="") as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    ours = [(kernel_direction(r["Kernel_Name"]), int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in rows]
    ours = [o for o in ours if o[0] is not None]
    acc = {}
    for prev, cur, nxt in zip(ours, ours[1:], ours[2:]):
        if prev[0] != cur[0] and nxt[0] != cur[0]:
            phase = "in_step"
        elif prev[0] == cur[0] == nxt[0]:
            phase = "back_to_back"
        else:
            continue
        a = acc.setdefault(phase, {"forward": [], "backward": [], "gap": []})
        a[cur[0]].append((cur[2] - cur[1]) / 1e3)
        a["gap"].append((cur[1] - prev[2]) / 1e3)
    med = lambda v: sorted(v)[len(v) // 2] if v else None  # noqa: E731
    out = {}
    for phase, a in acc.items():
        out[phase] = {"gap_median_us": med(a["gap"])}
        for d in ("forward", "backward"):
            v = a[d]
            out[phase][d] = {"n": len(v), "mean_us": sum(v) / len(v) if v else None, "median_us": med(v)}
    return out


def host_breakdown(torch, cufk_amd, L, A, D, g, an, abi_pair, reps=1000):
    """Host time per call (microseconds, no synchronisation inside the loop: at small configs
    the host, not the GPU, bounds these) of the pieces of one eager step: the public forward
    (Python wrapper and _C.apply, recording the backward), _C.apply alone, the backward alone
    (torch.autograd.grad on a retained graph: the autograd engine plus the binding's backward),
    the same engine hand-off for a one-op graph (L * 1.0), the step's two C-ABI calls through
    ctypes, and the whole step."""
    import time

    from cufk_amd._native import _C

    def per_call(fn):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        return (t1 - t0) / reps * 1e6

    x = cufk_amd.reconstruct(L, A, D, *an)
    y = L * 1.0
    gy = torch.ones_like(y)
    out = {
        "forward_call_us": per_call(lambda: cufk_amd.reconstruct(L, A, D, *an)),
        "apply_us": per_call(lambda: _C.apply(L, A, D, *an)),
        "backward_call_us": per_call(lambda: torch.autograd.grad(x, (L, A, D), g, retain_graph=True)),
        "engine_one_op_backward_us": per_call(lambda: torch.autograd.grad(y, (L,), gy, retain_graph=True)),
        "abi_pair_ctypes_us": per_call(abi_pair),
        "step_us": per_call(lambda: torch.autograd.grad(cufk_amd.reconstruct(L, A, D, *an), (L, A, D), g)),
    }
    out["reps"] = reps
    return out


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


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, kind, B, N, runs, seconds):
    """The reference algorithm on this host's CPU cores (oracle/cpu_torch.py): float64 forward
    plus explicit reverse adjoint in PyTorch, vectorised over chains, serial over steps.

    One small run estimates the cost per chain; the sample is then the config's whole batch or
    the largest subset that keeps one run near `seconds`.  Returns the median atoms/s over
    `runs` runs, the chain count, the per-run wall times and the thread count."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import cpu_torch as ct

    threads = torch.get_num_threads()  # torch's intra-op pool: OMP_NUM_THREADS or the host's cores
    gen = torch.Generator().manual_seed(1000)
    consts = None
    torsion = kind in ("torsion", "torsion_loss")
    if torsion:
        from oracle import nerf64 as o

        consts = o.torsion_constants(BOND_LENGTHS, BOND_ANGLES)

    def make(n):
        if torsion:
            raw = torch.randn(n, 2 * (N - 3), generator=gen, dtype=torch.float64)
            return raw, torch.randn(n, N, 3, generator=gen, dtype=torch.float64)
        L = (torch.randn(n, N - 1, generator=gen, dtype=torch.float64) * 0.01 + 0.145).clamp_(0.12, 0.17)
        A = torch.randn(n, N - 2, generator=gen, dtype=torch.float64) * 0.08 + 2.05
        D = (torch.rand(n, N - 3, generator=gen, dtype=torch.float64) * 2 - 1) * np.pi
        g = torch.randn(n, N, 3, generator=gen, dtype=torch.float64)
        p0 = torch.randn(3, generator=gen, dtype=torch.float64)
        q, _ = torch.linalg.qr(torch.randn(3, 3, generator=gen, dtype=torch.float64))
        return L, A, D, g, p0, q[:, 0].contiguous(), q[:, 1].contiguous()

    def run(inputs):
        t0 = time.perf_counter()
        if torsion:
            raw, g = inputs
            x = ct.torsion_forward(raw, consts.lengths, consts.sin, consts.cos)
            if kind == "torsion_loss":
                g = 2.0 * (x - g)  # the coordinate loss against target g
            ct.torsion_backward(raw, x, g, consts.lengths)
        else:
            L, A, D, g, p0, fd, n0 = inputs
            x = ct.forward(L, A, D, p0, fd, n0)
            if kind == "loss":
                g = 2.0 * (x - g * 0.3)  # the loss against the same target bench.py uses on the GPU
            elif kind == "rmsd":  # Kabsch by SVD, then the RMSD's grad_xyz
                t = x + g * 0.3
                xc, tc = x - x.mean(1, keepdim=True), t - t.mean(1, keepdim=True)
                U, _, Vh = torch.linalg.svd(xc.transpose(1, 2) @ tc)
                V, Ut = Vh.transpose(1, 2), U.transpose(1, 2)
                dsign = torch.sign(torch.linalg.det(V @ Ut))
                Dm = torch.diag_embed(torch.stack([torch.ones_like(dsign), torch.ones_like(dsign), dsign], -1))
                Rt = (V @ Dm @ Ut).transpose(1, 2)
                r = xc @ Rt - tc
                rmsd = r.pow(2).sum(-1).mean(-1).sqrt()
                g = (r @ Rt.transpose(1, 2)) / (N * rmsd[:, None, None])
            ct.backward(x, g)
        return time.perf_counter() - t0

    probe = max(1, min(B, 64))
    est = run(make(probe)) / probe  # also warms torch's CPU kernels
    n = int(max(1, min(B, seconds / max(est, 1e-9))))
    inputs = make(n)
    walls = sorted(run(inputs) for _ in range(max(1, runs)))
    med = walls[len(walls) // 2]
    return n * N / med, n, walls, threads


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
    if args.phases:
        print(json.dumps(trace_phases(args.phases)))
        return 0

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
    steps, fwds, bwds, regular, fonly, steps_inputs = [], [], [], [], [], []
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

            def step(L=L, A=A, D=D, g=g, p0=p0, fd=fd, n0=n0):
                xyz = cufk_amd.reconstruct_long(L, A, D, p0, fd, n0)
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
            fonly.append(lambda L=L, A=A, D=D, p0=p0, fd=fd, n0=n0: cufk_amd.reconstruct_long(L, A, D, p0, fd, n0))
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

            def step(L=L, A=A, D=D, target=target, p0=p0, fd=fd, n0=n0):
                loss = cufk_amd.reconstruct_loss(L, A, D, target, p0, fd, n0)
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
            fonly.append(lambda L=L, A=A, D=D, t=target, p0=p0, fd=fd, n0=n0: cufk_amd.reconstruct_loss(L, A, D, t, p0,
                                                                                                       fd, n0))
    elif kind == "rmsd":
        # As the coordinate loss (s(9N-6) each way) plus a 24-double superposition record per
        # chain written by the forward and read by the backward.
        fwd_bytes = s * B * (9 * N - 6) + 8 * 24 * B
        bwd_bytes = s * B * (9 * N - 6) + 8 * 24 * B
        unfused = []
        for k in range(nsets):
            L, A, D, g, p0, fd, n0 = synthetic(B, N, 2 + k, torch, device, dtype)
            with torch.no_grad():
                target = cufk_amd.reconstruct(L, A, D, p0, fd, n0) + g * 0.3
            for t in (L, A, D):
                t.requires_grad_(True)

            def step(L=L, A=A, D=D, target=target, p0=p0, fd=fd, n0=n0):
                loss = cufk_amd.reconstruct_rmsd(L, A, D, target, p0, fd, n0)
                return torch.autograd.grad(loss.sum(), (L, A, D))

            def plain(L=L, A=A, D=D, target=target, p0=p0, fd=fd, n0=n0):
                # Kabsch by SVD of the batched 3x3 cross-covariances; the rotation is held fixed in
                # the backward (its own dependence drops out at the optimum).
                x = cufk_amd.reconstruct(L, A, D, p0, fd, n0)
                xc, tc = x - x.mean(1, keepdim=True), target - target.mean(1, keepdim=True)
                U, _, Vh = torch.linalg.svd((xc.transpose(1, 2) @ tc).detach())
                V, Ut = Vh.transpose(1, 2), U.transpose(1, 2)
                dsign = torch.sign(torch.linalg.det(V @ Ut))
                Dm = torch.diag_embed(torch.stack([torch.ones_like(dsign), torch.ones_like(dsign), dsign], -1))
                Rt = (V @ Dm @ Ut).transpose(1, 2).contiguous()
                rmsd = ((xc @ Rt - tc) ** 2).sum(-1).mean(-1).sqrt()
                return torch.autograd.grad(rmsd.sum(), (L, A, D))

            loss_out = torch.empty(B, device=device, dtype=dtype)
            xyz = torch.empty(B, N, 3, device=device, dtype=dtype)
            flags = torch.empty(B, device=device, dtype=torch.uint8)
            rec = torch.empty(B, 24, device=device, dtype=torch.float64)
            gL, gA, gD = torch.empty_like(L), torch.empty_like(A), torch.empty_like(D)

            def fwd(st, L=L, A=A, D=D, target=target, p0=p0, fd=fd, n0=n0, xyz=xyz, flags=flags, loss_out=loss_out,
                    rec=rec):
                rc = lib.cufk_reconstruct_superposed_fwd(code, 2, P(L), P(A), P(D), P(p0), P(fd), P(n0), P(target),
                                                         P(xyz), P(flags), P(loss_out), P(rec), i64(B), i64(N), st)
                assert rc == 0, rc

            def bwd(st, L=L, A=A, D=D, target=target, p0=p0, fd=fd, n0=n0, xyz=xyz, flags=flags, rec=rec, gL=gL,
                    gA=gA, gD=gD):
                rc = lib.cufk_reconstruct_superposed_bwd(code, 2, P(L), P(A), P(D), P(p0), P(fd), P(n0), P(xyz),
                                                         P(flags), P(target), P(rec), None, P(gL), P(gA), P(gD),
                                                         i64(B), i64(N), st)
                assert rc == 0, rc

            steps.append(step)
            fwds.append(fwd)
            bwds.append(bwd)
            unfused.append(plain)
            fonly.append(lambda L=L, A=A, D=D, t=target, p0=p0, fd=fd, n0=n0: cufk_amd.reconstruct_rmsd(L, A, D, t, p0,
                                                                                                       fd, n0))
    elif kind == "reconstruct":
        fwd_bytes = s * B * (6 * N - 6)
        bwd_bytes = s * B * (9 * N - 12)
        for k in range(nsets):
            L, A, D, g, p0, fd, n0 = synthetic(B, N, 2 + k, torch, device, dtype,
                                               args.irregular or IRREGULAR.get(args.config))
            L.requires_grad_(True)
            A.requires_grad_(True)
            D.requires_grad_(True)

            def step(L=L, A=A, D=D, g=g, p0=p0, fd=fd, n0=n0):
                xyz = cufk_amd.reconstruct(L, A, D, p0, fd, n0)
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
            steps_inputs.append((L, A, D, g, p0, fd, n0))
            regular.append(flags)
            fonly.append(lambda L=L, A=A, D=D, p0=p0, fd=fd, n0=n0: cufk_amd.reconstruct(L, A, D, p0, fd, n0))
    else:
        import math

        class Consts(ctypes.Structure):
            _fields_ = [("length", ctypes.c_float * 3), ("sin", ctypes.c_double * 3), ("cos", ctypes.c_double * 3)]

        c = Consts((ctypes.c_float * 3)(*BOND_LENGTHS), (ctypes.c_double * 3)(*[math.sin(a) for a in BOND_ANGLES]),
                   (ctypes.c_double * 3)(*[math.cos(a) for a in BOND_ANGLES]))
        f = cufk_amd.compile_torsion(BOND_LENGTHS, BOND_ANGLES)
        fused = kind == "torsion_loss"
        # Torsion: forward s(5N-6), backward s(10N-12).  With the fused coordinate loss the
        # forward also reads the target (3N) and the backward reads the target in place of
        # grad_xyz (same count).
        fwd_bytes = s * B * (5 * N - 6 + (3 * N if fused else 0))
        bwd_bytes = s * B * (10 * N - 12)
        unfused = []
        for k in range(nsets):
            gen = torch.Generator().manual_seed(3 + k)
            raw = torch.randn(B, 2 * (N - 3), generator=gen, dtype=torch.float64).to(device=device, dtype=dtype)
            g = torch.randn(B, N, 3, generator=gen, dtype=torch.float64).to(device=device, dtype=dtype)
            raw.requires_grad_(True)

            if fused:
                def step(raw=raw, target=g):
                    return torch.autograd.grad(f.loss(raw, target).sum(), (raw,))

                def plain(raw=raw, target=g):
                    return torch.autograd.grad(((f(raw) - target) ** 2).sum(), (raw,))

                unfused.append(plain)
            else:
                def step(raw=raw, g=g):
                    xyz = f(raw)
                    return torch.autograd.grad(xyz, (raw,), g)

            xyz = torch.empty(B, N, 3, device=device, dtype=dtype)
            graw = torch.empty_like(raw)
            loss_out = torch.empty(B, device=device, dtype=dtype)

            def fwd(st, raw=raw, xyz=xyz, target=g, loss_out=loss_out):
                if fused:
                    rc = lib.cufk_torsion_loss_fwd(code, 0, P(raw), i64(raw.stride(0)), ctypes.byref(c), P(target),
                                                   P(xyz), P(loss_out), None, i64(B), i64(N), st)
                else:
                    rc = lib.cufk_torsion_fwd(code, P(raw), i64(raw.stride(0)), ctypes.byref(c), P(xyz), i64(B), i64(N),
                                              st)
                assert rc == 0, rc

            def bwd(st, raw=raw, xyz=xyz, g=g, graw=graw):
                if fused:
                    rc = lib.cufk_torsion_loss_bwd(code, 0, P(raw), i64(raw.stride(0)), P(xyz), P(g), None, None,
                                                   P(graw), i64(graw.stride(0)), ctypes.byref(c), i64(B), i64(N), st)
                else:
                    rc = lib.cufk_torsion_bwd(code, P(raw), i64(raw.stride(0)), P(xyz), P(g), P(graw),
                                              i64(graw.stride(0)), ctypes.byref(c), i64(B), i64(N), st)
                assert rc == 0, rc

            steps.append(step)
            fwds.append(fwd)
            bwds.append(bwd)
            fonly.append((lambda raw=raw, target=g: f.loss(raw, target)) if fused else (lambda raw=raw: f(raw)))

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

    stream = torch.cuda.current_stream()
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

    # 1. Clock ramp (untimed), then 2. the W warm-up steps.
    ramp_steps = 0
    t_ramp = time.perf_counter()
    while time.perf_counter() - t_ramp < args.ramp_s:
        for _ in range(10):
            steps[ramp_steps % nsets]()
            ramp_steps += 1
        torch.cuda.synchronize()
    for i in range(args.warmup):
        steps[i % nsets]()
    torch.cuda.synchronize()

    # Timed region: K steps back to back on the stream the kernels run on.
    t_start, t_end = ev(), ev()
    torch.cuda.synchronize()
    t_start.record(stream)
    for i in range(args.steps):
        steps[i % nsets]()
    t_end.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t_start.elapsed_time(t_end) / args.steps

    # 3. Forward only: K forward calls without autograd (the plain forward kernels).
    with torch.no_grad():
        for i in range(min(args.warmup, 10)):
            fonly[i % nsets]()
        torch.cuda.synchronize()
        f_start, f_end = ev(), ev()
        f_start.record(stream)
        for i in range(args.steps):
            fonly[i % nsets]()
        f_end.record(stream)
        torch.cuda.synchronize()
    ms_forward_only = f_start.elapsed_time(f_end) / args.steps

    # 4. Kernel split: K back-to-back launches of the step's forward entry point (the flagged
    # forward, through the C ABI) under one event pair, rotating over the same sets, then K
    # launches of its backward entry point over each set's saved forward output.  Inside the
    # step the backward finds part of its forward's output in the 256 MB last-level cache and the
    # next forward follows a backward whose stores bypass it; back to back over rotating sets
    # neither holds, so at large configs these durations sit a few percent above the in-step
    # ones and step_gap_us (the step minus both) goes negative.  rocprofv3's kernel trace of the
    # same run gives both phases (``--phases``).  An event pair around each launch would add a few
    # microseconds per launch on this part.
    st = ctypes.c_void_p(stream.cuda_stream)
    abi_reps = args.abi_reps if args.abi_reps > 0 else args.steps
    for i in range(nsets):
        fwds[i](st)  # each set's saved output (and regularity flags) for the backward
    t_fwd = event_time_ms(torch, lambda i: fwds[i % nsets](st), abi_reps)
    for i in range(nsets):
        fwds[i](st)
    t_bwd = event_time_ms(torch, lambda i: bwds[i % nsets](st), abi_reps)
    regular_frac = float(torch.stack(regular).float().mean()) if regular else None

    # 5. The same step replayed from HIP graphs (eager runs only, reconstruct and torsion): one
    # graph per input set, captured after warm-up on a side stream, replayed back to back.  With
    # the per-step Python, autograd-engine and launch overhead gone it shows how much of the
    # eager step is host time (all of the difference at small configs such as c1).
    graph_ms = None
    if not args.graph and kind in ("reconstruct", "torsion") and args.graph_too:
        graphs = []
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for k in range(nsets):
                for _ in range(3):
                    steps[k]()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        for k in range(nsets):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                steps[k]()
            graphs.append(graph)
        for i in range(args.warmup):
            graphs[i % nsets].replay()
        graph_ms = event_time_ms(torch, lambda i: graphs[i % nsets].replay(), args.steps)
        del graphs

    unfused_us = None
    if kind in ("loss", "rmsd", "torsion_loss"):  # the same step unfused (the loss in torch), same input sets
        for i in range(args.warmup):
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
    host = None
    if kind == "reconstruct" and (args.host_breakdown or args.config == "c1"):
        L0, A0, D0, *_ = steps_inputs[0]
        host = host_breakdown(torch, cufk_amd, L0, A0, D0, steps_inputs[0][3], steps_inputs[0][4:],
                              lambda: (fwds[0](st), bwds[0](st)))

    atoms = B * N
    step_bytes = fwd_bytes + bwd_bytes
    gbs = lambda nbytes, ms: None if ms is None else nbytes / (ms * 1e-3) / 1e9  # noqa: E731
    us = lambda ms: None if ms is None else ms * 1e3  # noqa: E731
    frac = lambda nbytes, ms: None if ms is None else gbs(nbytes, ms) / HBM_PEAK_GBS  # noqa: E731
    traffic = MEASURED_TRAFFIC.get(args.config)
    result = {
        "metric": metric_name(args.config),
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
                   "input_sets": nsets, "ramp_steps": ramp_steps},
        "forward_atoms_per_s": atoms / (ms_forward_only * 1e-3),
        "roofline": {
            "bound": "hbm",
            "kernel": f"{kind} forward + backward (one step: the two launches the metric times)",
            "achieved": gbs(step_bytes, ms_per_step),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": frac(step_bytes, ms_per_step),
            "traffic": traffic,
            "algorithmic_bytes": step_bytes,
            "avg_step_us": ms_per_step * 1e3,
        },
        "kernels": {
            "forward_us": us(t_fwd),
            "backward_us": us(t_bwd),
            "step_gap_us": us(ms_per_step - t_fwd - t_bwd),
            "split": f"forward and backward: {abi_reps} back-to-back launches each of the step's forward and backward "
                     "C-ABI entry points under one event pair (the backward over each set's saved forward output); "
                     "step_gap_us: the step minus both (negative where the step's backward reads its forward's output "
                     "from the last-level cache)",
            "forward_frac": frac(fwd_bytes, t_fwd),
            "backward_frac": frac(bwd_bytes, t_bwd),
            "forward_algorithmic_bytes": fwd_bytes,
            "backward_algorithmic_bytes": bwd_bytes,
            "forward_only_us": ms_forward_only * 1e3,
            "regular_chain_fraction": regular_frac,
            "unfused_step_us": unfused_us,
            "graph_step_us": us(graph_ms),
        },
    }
    valu = MEASURED_VALU.get(args.config)
    if valu is not None:
        # The VALU roofline of the step's forward launch (VALU-bound: the reconstruct forwards
        # issue VALU for most of their cycles), with the backward's fraction beside it.
        result["roofline_valu"] = {
            "bound": "valu",
            "kernel": f"{kind} forward launch (kernels.forward_us)",
            "achieved": valu[0] / (t_fwd * 1e-3) / 1e9,
            "peak": VALU_PEAK_PER_S / 1e9,
            "unit": "G wave64 VALU instructions/s",
            "frac": valu[0] / (t_fwd * 1e-3) / VALU_PEAK_PER_S,
            "instructions": valu[0],
            "backward_instructions": valu[1],
            "backward_frac": valu[1] / (t_bwd * 1e-3) / VALU_PEAK_PER_S,
        }
    if precision is not None:
        result["precision"] = precision
    if host is not None:
        result["host"] = host
    if not args.no_cpu_baseline:
        v, chains, walls, threads = cpu_baseline(torch, kind, B, N, args.cpu_runs, args.cpu_seconds)
        result["cpu_baseline"] = {
            "value": v,
            "unit": "atoms/s",
            "cores": threads,
            "kind": "port",
            "sample": f"serial float64 NeRF forward + reverse adjoint in PyTorch CPU (oracle/cpu_torch.py), "
                      f"{chains} chains x N={N}, median of {len(walls)} runs "
                      f"({', '.join(f'{w:.2f}' for w in walls)} s) on {threads} threads of {cpu_model()} "
                      f"(host: {os.cpu_count()} logical CPUs, {len(os.sched_getaffinity(0))} in this process's "
                      f"affinity), scaled to atoms/s",
        }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())

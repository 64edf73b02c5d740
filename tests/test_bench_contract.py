"""bench.py's contract pieces that need no GPU: the single-GPU refusal, the configurations, and
the measured-traffic table it reports as roofline.traffic, checked against the committed
rocprofv3 summary and against the algorithmic byte counts that summary lists."""

from __future__ import annotations

import importlib.util
import re
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _bench():
    spec = importlib.util.spec_from_file_location("bench_module", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2", "--steps", "1", "--warmup", "0"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stdout + proc.stderr


def test_headline_config_is_the_baseline_metric():
    b = _bench()
    assert b.CONFIGS["c2"] == ("reconstruct", "float32", 4096, 2049)
    assert b.CONFIGS["c1"] == ("reconstruct", "float32", 1024, 384)
    assert b.CONFIGS["c3"] == ("torsion", "float32", 8192, 771)
    assert b.CONFIGS["c4_bf16"] == ("reconstruct", "bfloat16", 16384, 1026)


PROFILE = ROOT / "profiles" / "counters_and_traffic_bench_regime.md"


def _int(x):
    return int(x.replace(",", ""))


def _profile_rows():
    """Per-kernel rows (config, kernel, read, written, total, algorithmic, VALU per launch) and
    per-step rows (config: traffic, algorithmic, forward VALU, backward VALU) of the summary."""
    text = PROFILE.read_text()
    kernels, steps = {}, {}
    num = r"([\d,]+)"
    for m in re.finditer(rf"^\| (\w+) \| `([^`]+)` \| [\d.]+ \| {num} \| {num} \| {num} \| {num} \| {num} \|", text, re.M):
        kernels.setdefault(m.group(1), []).append((m.group(2), *(_int(m.group(k)) for k in range(3, 8))))
    for m in re.finditer(rf"^\| (\w+) \| {num} \| {num} \| [\d.]+ \| {num} \| {num} \|$", text, re.M):
        steps[m.group(1)] = tuple(_int(m.group(k)) for k in range(2, 6))
    return kernels, steps


def test_measured_traffic_and_valu_match_the_committed_profile():
    b = _bench()
    kernels, steps = _profile_rows()
    assert set(kernels) == set(steps) == set(b.MEASURED_TRAFFIC) == set(b.MEASURED_VALU)
    for cfg, rows in kernels.items():
        for _, read, write, total, _, _ in rows:
            assert read + write == total, cfg
        assert sum(r[3] for r in rows) == steps[cfg][0] == b.MEASURED_TRAFFIC[cfg], cfg
        bwd = sum(r[5] for r in rows if any(w in r[0] for w in ("backward", "sums", "carry")))
        fwd = sum(r[5] for r in rows) - bwd
        assert (fwd, bwd) == steps[cfg][2:] == b.MEASURED_VALU[cfg], cfg


def test_profile_algorithmic_bytes_follow_the_formulas():
    """The summary's algorithmic column: forward s(6N-6) and backward s(9N-12) bytes per chain
    for reconstruct, s(5N-6) and s(10N-12) for torsion (s the element size); the per-step
    total is their sum, as the bench's own roofline counts it."""
    b = _bench()
    kernels, steps = _profile_rows()
    size = {"float32": 4, "bfloat16": 2}
    for cfg in ("c1", "c2", "c2_far", "c2_mixed", "c3", "c4_bf16", "short"):
        kind, dtype, B, N = b.CONFIGS[cfg]
        s = size[dtype]
        fwd, bwd = ((5 * N - 6), (10 * N - 12)) if kind == "torsion" else ((6 * N - 6), (9 * N - 12))
        assert [k[4] for k in kernels[cfg]] == [s * B * fwd, s * B * bwd], cfg
        assert steps[cfg][1] == s * B * (fwd + bwd), cfg


def test_c2_trace_recomputes_the_stated_roofline_fraction():
    """profiles/reconstruct_c2_kernel_stats.md: the two kernels' average durations give the step
    fraction it states (algorithmic bytes / (forward + backward) / 8 TB/s)."""
    text = (ROOT / "profiles" / "reconstruct_c2_kernel_stats.md").read_text()
    avg = {m.group(1): int(m.group(2)) for m in re.finditer(r"^\| (reconstruct_\w+) \| \d+ \| (\d+) \|", text, re.M)}
    step_ns = avg["reconstruct_forward_kernel"] + avg["reconstruct_backward_saved_kernel"]
    B, N = 4096, 2049
    frac = 4 * B * (15 * N - 18) / (step_ns * 1e-9) / 8e12
    stated = float(re.search(r"\*\*(0\.\d+)\*\* of 8 TB/s", text).group(1))
    assert abs(frac - stated) <= 0.0015, (frac, stated)


def test_metric_names_follow_the_config():
    b = _bench()
    assert b.metric_name("c2") == "fwd+bwd atoms/sec @ B=4096 N=2049 fp32; % of HBM roofline"
    assert b.metric_name("c2") == __import__("json").loads((ROOT / "BASELINE.json").read_text())["metric"]
    assert b.metric_name("c1") == "reconstruct fwd+bwd atoms/sec @ B=1024 N=384 fp32 (c1); % of HBM roofline"
    assert b.metric_name("c4_bf16") == "reconstruct fwd+bwd atoms/sec @ B=16384 N=1026 bf16 (c4_bf16); % of HBM roofline"
    assert b.metric_name("c3").startswith("torsion fwd+bwd atoms/sec @ B=8192 N=771 fp32")
    assert len({b.metric_name(c) for c in b.CONFIGS}) == len(b.CONFIGS)


def test_exact_fallback_configs_break_the_position_tests():
    """c2_far puts every chain past the fp32 extent test (max |x| <= 256 x shortest bond); c2_mixed
    gives exactly every fourth chain an angle past the sine test (sin < 0.5), the rest pass it."""
    import math

    import torch

    from oracle import cpu_torch as ct

    b = _bench()
    B, N = 64, 2049
    L, A, D, g, p0, fd, n0 = b.synthetic(8, N, 2, torch, "cpu", torch.float64, "far")
    assert p0.tolist() == [50.0, 0.0, 0.0]
    x = ct.forward(L, A, D, p0, fd, n0)
    assert (x.abs().amax(dim=(1, 2)) > 256 * L.amin(dim=1)).all()
    L, A, D, *_ = b.synthetic(B, N, 2, torch, "cpu", torch.float64, b.IRREGULAR["c2_mixed"])
    bad = (torch.sin(A) < 0.5).any(dim=1)
    assert bad.tolist() == [i % 4 == 0 for i in range(B)]
    for pattern, want in (("every:16", [i % 16 == 0 for i in range(B)]), ("first:0.25", [i < 16 for i in range(B)])):
        A3 = b.synthetic(B, N, 2, torch, "cpu", torch.float64, pattern)[1]
        assert (torch.sin(A3) < 0.5).any(dim=1).tolist() == want, pattern
    assert math.isclose(float(torch.sin(torch.tensor(2.7))), 0.427, abs_tol=1e-3)
    L2, A2, *_ = b.synthetic(B, N, 2, torch, "cpu", torch.float64)
    assert torch.equal(L, L2) and torch.equal(A[1::4], A2[1::4])


def test_trace_phases_split(tmp_path):
    """--phases: a dispatch between two of the other direction is in a step, one between two of
    its own direction is back to back; torch's kernels are not ours and are skipped."""
    b = _bench()
    head = "Kind,Kernel_Name,Start_Timestamp,End_Timestamp\n"
    f, bw, other = "void cufk_amd::reconstruct_forward_kernel<float>(x)", "void cufk_amd::reconstruct_backward_saved_kernel<float>(x)", "void at::native::copy(x)"
    seq = [(f, 0, 40), (bw, 40, 90), (other, 90, 95), (f, 100, 140), (bw, 140, 190), (f, 190, 230), (bw, 232, 282),
           (f, 300, 345), (f, 345, 390), (f, 391, 436), (f, 436, 481)]
    lines = "".join(f'K,"{n}",{a * 1000},{e * 1000}\n' for n, a, e in seq)
    path = tmp_path / "trace.csv"
    path.write_text(head + lines)
    out = b.trace_phases(str(path))
    assert out["in_step"]["forward"]["n"] == 2 and out["in_step"]["backward"]["n"] == 3
    assert out["in_step"]["forward"]["mean_us"] == 40.0 and out["in_step"]["backward"]["mean_us"] == 50.0
    assert out["back_to_back"]["forward"]["n"] == 2 and out["back_to_back"]["forward"]["mean_us"] == 45.0
    assert out["back_to_back"]["backward"]["n"] == 0 and out["back_to_back"]["gap_median_us"] == 1.0
    assert b.kernel_direction(other) is None and b.kernel_direction(f) == "forward"

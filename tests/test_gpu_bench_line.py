"""bench.py's JSON line on the GPU: a short run per config checks the fields the driver and the
tables read (metric, value, roofline, the kernel split and its step gap, the graph-replayed step)
and, for the exact-fallback configs, the regular-chain fraction their inputs are built to give."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent


def _line(config, *extra):
    cmd = [sys.executable, str(ROOT / "bench.py"), "--config", config, "--steps", "4", "--warmup", "2", "--ramp-s", "0",
           "--sets", "1", "--no-cpu-baseline", *extra]
    print("bench:", " ".join(cmd[1:]), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return json.loads(proc.stdout.strip().splitlines()[-1])


@pytest.mark.parametrize("config", ["c1", "c3"])
def test_bench_line_fields(device, config):
    sys.path.insert(0, str(ROOT))
    import bench

    r = _line(config)
    k = r["kernels"]
    assert r["metric"] == bench.metric_name(config) and r["n_gpus"] == 1 and r["value"] > 0
    assert r["roofline"]["bound"] == "hbm" and 0 < r["roofline"]["frac"] < 1
    assert k["forward_us"] > 0 and k["backward_us"] > 0 and k["graph_step_us"] > 0
    step_us = r["ms_per_step"] * 1e3
    assert k["step_gap_us"] == pytest.approx(step_us - k["forward_us"] - k["backward_us"], abs=1e-6)
    assert k["forward_frac"] < 1 and k["backward_frac"] < 1
    if config == "c1":
        h = r["host"]
        assert 0 < h["apply_us"] <= h["forward_call_us"] and h["backward_call_us"] > 0 and h["step_us"] > 0
    v = r["roofline_valu"]
    assert v["bound"] == "valu" and 0 < v["frac"] < 1 and 0 < v["backward_frac"] < 1
    assert v["achieved"] == pytest.approx(v["instructions"] / (k["forward_us"] * 1e-6) / 1e9)


@pytest.mark.parametrize("config,fraction", [("c2_far", 0.0), ("c2_mixed", 0.75)])
def test_exact_fallback_configs(device, config, fraction):
    r = _line(config, "--no-graph-too")
    assert r["kernels"]["regular_chain_fraction"] == fraction
    assert r["kernels"]["graph_step_us"] is None

"""bench.py on the GPU: every workload prints one JSON line that keeps the
driver's contract (metric, value, unit, steps, timing, roofline object,
cpu_baseline slot) and whose output matches the CPU oracle.

Each workload runs in a child process with a few steps and without the
host-array leg; the small configurations (1 and 2) also run the CPU oracle
leg, which checks the GPU output, and the 512 MiB workloads skip it (their
parity has tests of its own: test_gpu_config_shapes.py, test_gpu_fft_large.py).
The GPU work is the same plan and kernels the full run times.
"""

from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")

FFT = ["cfg1", "cfg2_256", "cfg2_4096", "cfg3", "cfg3_split", "cfg4", "cfg5", "1d_8192", "1d_16384",
       "1d_32768", "2d_64", "2d_128"]
OPS = ["cmul", "cmul_split", "deinterleave", "interleave", "transpose"]


SMALL = {"cfg1", "cfg2_256", "cfg2_4096"}


def run_bench(workload, *extra):
    cpu = ["--cpu-budget", "0"] if workload in SMALL else ["--no-cpu"]
    print(f"[case] bench.py --workload {workload} {' '.join(cpu + list(extra))}", flush=True)
    r = subprocess.run([sys.executable, BENCH, "--workload", workload, "--steps", "4", "--warmup", "2",
                        "--no-host-path", "--ramp-ms", "5", *cpu, *extra],
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, r.stdout
    return json.loads(lines[0])


def test_every_workload_is_in_the_test_lists():
    import bench

    assert sorted(FFT + OPS) == sorted(bench.WORKLOADS)


@pytest.mark.parametrize("workload", FFT + OPS)
def test_bench_line_keeps_the_contract(workload):
    d = run_bench(workload)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 4 and d["warmup"] == 2
    assert d["value"] > 0 and d["ms_per_step"] > 0 and d["higher_is_better"] is True
    assert d["config"]["name"] == workload
    rf = d["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert 0 < rf["achieved"] and rf["frac"] == pytest.approx(rf["achieved"] / rf["peak"], abs=1e-4)
    if workload in FFT:
        assert d["config"]["dims"] in (1, 2)
    if workload in SMALL:
        assert d["rel_l2_vs_cpu"] <= 1e-4
        assert d["cpu_baseline"]["kind"] == "port" and d["cpu_baseline"]["cores"] == 1
    else:
        assert d["cpu_baseline"] is None


def test_bench_graph_replay_line():
    d = run_bench("cfg1", "--graph", "2")
    assert d["value"] > 0 and "graph" in d["launch_mode"]

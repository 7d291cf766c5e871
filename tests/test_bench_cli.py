"""CPU checks of bench.py's contract that need no GPU: the one-GPU refusal,
argument validation, the workload table and the sysfs clock parsing."""

from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def run_bench(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("args", [["--steps", "0"], ["--warmup", "-1"], ["--graph", "3", "--steps", "10"],
                                  ["--configs", "cfg3"], ["--configs", "cfg1,bogus"], ["--config-steps", "0"],
                                  ["--config-warmup", "-1"]])
def test_bad_arguments_are_refused(args):
    r = run_bench(*args)
    assert r.returncode == 2 and r.stdout == ""


def test_workloads_cover_every_baseline_config():
    import bench

    for name in ("cfg1", "cfg2_256", "cfg2_4096", "cfg3", "cfg4", "cfg5"):
        assert name in bench.FFT_WORKLOADS
    dims, log_n, batch, seed, dist, steps, layout, _ = bench.FFT_WORKLOADS["cfg3"]
    assert (dims, log_n, batch, seed, dist, layout) == (1, 10, 65536, 3, "normal", "interleaved")
    assert bench.FFT_WORKLOADS["cfg4"][:5] == (1, 24, 4, 4, "normal")
    assert bench.FFT_WORKLOADS["cfg5"][:5] == (2, 12, 2, 5, "uniform")
    assert [d for d, _ in bench.FFT_WORKLOADS["cfg2_256"][5]] == ["forward", "inverse"]


def test_clock_sampler_reads_the_marked_level(tmp_path):
    import bench

    (tmp_path / "pp_dpm_sclk").write_text("0: 500Mhz\n1: 1753Mhz *\n2: 2400Mhz\n")
    (tmp_path / "pp_dpm_mclk").write_text("0: 2000Mhz *\n")
    c = bench.ClockSampler(period_s=0.001)
    c.dir = str(tmp_path)
    with c:
        import time

        time.sleep(0.01)
    rep = c.report()
    assert rep["mclk_mhz"] == 2000
    assert rep["sclk_samples"] >= 1 and rep["sclk_mhz_median"] == 1753 and rep["sclk_mhz_max"] == 1753


def test_clock_sampler_without_sysfs_reports_nothing():
    import bench

    c = bench.ClockSampler()
    c.dir = None
    with c:
        pass
    assert c.report() is None


def test_throughput_gate():
    # --min-frac: the JSON line carries the gate; the exit status fails it
    import bench

    res = {"roofline": {"frac": 0.7643, "kernel": "fg_fft_n10"}}
    assert bench.gate_check(res, None) is None
    assert bench.gate_check(res, 0.70) == {"min_frac": 0.70, "frac": 0.7643, "kernel": "fg_fft_n10", "passed": True}
    assert bench.gate_check(res, 0.80)["passed"] is False


def test_single_pass_workloads():
    import bench

    for name, log_n, batch in (("1d_8192", 13, 8192), ("1d_16384", 14, 4096), ("1d_32768", 15, 2048),
                               ("1d_2p16", 16, 1024), ("1d_2p18", 18, 256), ("1d_2p20", 20, 64)):
        dims, ln, b, *_ = bench.FFT_WORKLOADS[name]
        assert (dims, ln, b) == (1, log_n, batch) and b << ln == 1 << 26   # 512 MiB
    for name, log_n, batch in (("2d_64", 6, 16384), ("2d_128", 7, 4096), ("2d_512", 9, 256), ("2d_1024", 10, 64)):
        dims, ln, b, *_ = bench.FFT_WORKLOADS[name]
        assert (dims, ln, b) == (2, log_n, batch) and b << (2 * ln) == 1 << 26


class _Ev:
    """A stand-in for hip.Event: a time stamp in ms."""

    def __init__(self, t):
        self.t = t

    def elapsed_ms(self, end):
        return end.t - self.t


class _Wl:
    def __init__(self, streams, keys, execs):
        self.launch_streams, self.launch_keys, self.exec_bounds = streams, keys, execs


def test_launch_durations_one_stream_are_event_gaps():
    import bench

    wl = _Wl([0, 0, 0], ["0:a", "1:b", "2:c"], [(0, 3)])
    evs = [[_Ev(1), _Ev(2), _Ev(4)], [_Ev(5), _Ev(7), _Ev(8)]]
    got = bench.launch_durations(_Ev(0), evs, wl)
    assert got == {"0:a": [1, 1], "1:b": [1, 2], "2:c": [2, 1]}


def test_launch_durations_two_streams_use_each_streams_previous_event():
    # four chunks of one pass, odd chunks on the second stream: each launch
    # runs from the previous event of its stream, the first ones from the
    # end of the previous execution (where the plan forks)
    import bench

    wl = _Wl([0, 1, 0, 1], ["0:k"] * 4, [(0, 4)])
    evs = [[_Ev(3), _Ev(4), _Ev(6), _Ev(7)], [_Ev(10), _Ev(11), _Ev(13), _Ev(14)]]
    got = bench.launch_durations(_Ev(0), evs, wl)
    assert got == {"0:k": [3, 4, 3, 3, 3, 4, 3, 3]}


def test_launch_durations_two_executions_per_step():
    # forward then inverse per step (config 2's shape): the inverse starts
    # where the forward's last event is
    import bench

    wl = _Wl([0, 0], ["0:f", "0:i"], [(0, 1), (1, 2)])
    evs = [[_Ev(2), _Ev(5)], [_Ev(6), _Ev(9)]]
    got = bench.launch_durations(_Ev(0), evs, wl)
    assert got == {"0:f": [2, 1], "0:i": [3, 3]}


def test_extra_configs_are_the_other_baseline_configs():
    # the default run reports configs 1, 2, 4 and 5 beside config 3, timed as
    # the reference bench times (10 warmup, 100 timed, the median step)
    import bench

    assert bench.EXTRA_CONFIGS == ["cfg1", "cfg2_256", "cfg2_4096", "cfg4", "cfg5"]
    assert (bench.CONFIG_STEPS, bench.CONFIG_WARMUP) == (100, 10)


class _FakeFft:
    """The parts of bench.FftWorkload that pass_table / check_config read,
    over a small forward + inverse chain computed with numpy in fp64 (the
    'GPU output' here) and the real C oracle as the checker."""

    def __init__(self, dims, log_n, batch, steps):
        import numpy as np

        rng = np.random.default_rng(7)
        self.np = np
        self.dims, self.log_n, self.batch, self.steps = dims, log_n, batch, steps
        self.elems = (1 << log_n) if dims == 1 else 1 << (2 * log_n)
        n = self.elems * batch
        self.x = (rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)).astype(np.complex64)
        self.algo_bytes = 16 * n * len(steps)
        self.bytes_per_launch = 16 * n
        self.real = bench_real(self)

    def cpu(self, threads):
        return self.real.cpu(threads)

    @property
    def cpu_outputs(self):
        return self.real.cpu_outputs


def bench_real(fake):
    import bench

    wl = bench.FftWorkload.__new__(bench.FftWorkload)
    wl.np, wl.dims, wl.log_n, wl.batch, wl.steps, wl.x = fake.np, fake.dims, fake.log_n, fake.batch, fake.steps, fake.x
    return wl


def _numpy_chain(fake):
    np = fake.np
    shape = (fake.batch, 1 << fake.log_n) if fake.dims == 1 else (fake.batch, 1 << fake.log_n, 1 << fake.log_n)
    y = fake.x.reshape(shape).astype(np.complex128)
    outs = []
    for direction, normalize in fake.steps:
        f = np.fft.fft if fake.dims == 1 else np.fft.fft2
        fi = np.fft.ifft if fake.dims == 1 else np.fft.ifft2
        y = f(y) if direction == "forward" else (fi(y) if normalize else fi(y) * (y[0].size))
        outs.append(y.reshape(-1).astype(np.complex64))
    return outs


@pytest.mark.parametrize("dims,log_n,batch,steps", [
    (1, 8, 4, [("forward", False), ("inverse", True)]),
    (1, 10, 3, [("forward", False)]),
    (2, 5, 2, [("forward", False)]),
])
def test_check_config_keys_and_verdict(dims, log_n, batch, steps):
    # the oracle's verdict on a config record: per-step rel-L2 against the C
    # oracle, the round trip of forward + inverse chains, the fp64 bins, the
    # oracle's own time; numpy's complex128 transform passes all of them
    import bench

    fake = _FakeFft(dims, log_n, batch, steps)
    outs = _numpy_chain(fake)
    rec = {}
    bench.check_config(fake.np, rec, fake, outs)
    assert rec["parity_ok"] is True
    assert len(rec["rel_l2_vs_cpu_per_step"]) == len(steps)
    assert 0 <= rec["rel_l2_vs_cpu"] <= 1e-5 and rec["fp64_bins_rel_l2"] <= 1e-5
    assert ("roundtrip_rel_l2" in rec) == (len(steps) == 2)
    assert set(rec["cpu_oracle"]) >= {"seconds", "threads", "gbs", "note"}
    # a planted mistake (one bin conjugated in the first step's output) fails the verdict
    bad = [o.copy() for o in outs]
    bad[0][1] = np.conj(bad[0][1]) + 1.0
    rec2 = {}
    bench.check_config(fake.np, rec2, fake, bad)
    assert rec2["rel_l2_vs_cpu"] > 1e-4 and rec2["parity_ok"] is False


def test_pass_table_rates():
    import bench

    class W:
        bytes_per_launch = 1 << 28

    per = {"1:fg_tile_b": [0.05, 0.04, 0.06], "0:fg_tile_a": [0.04, 0.04]}
    rows = bench.pass_table(np, W, per)
    assert [r["pass"] for r in rows] == [0, 1] and [r["kernel"] for r in rows] == ["fg_tile_a", "fg_tile_b"]
    assert rows[0]["avg_ms"] == 0.04 and rows[1]["median_ms"] == 0.05 and rows[1]["launches"] == 3
    assert rows[0]["gbs"] == pytest.approx((1 << 28) / 0.04e-3 / 1e9, abs=0.051)
    assert rows[0]["frac"] == pytest.approx(rows[0]["gbs"] / 8000.0, abs=1e-4)


def test_shape_copy_geometry_is_config5s_column_pass():
    # bench.py's shape_cfg5col launches the column pass's geometry: tiles of 8
    # columns over the rows of each parity, element stride 2C, in place, line
    # groups; every element of both images is read and written exactly once
    import bench

    g = bench.cfg5_column_geom(12)
    C = 4096
    assert (g.t0n, g.t1n, g.is0, g.is1, g.is2, g.ies, g.ics) == (C // 8, 2, 8, C, C * C, 2 * C, 1)
    assert (g.os0, g.os1, g.os2, g.oes, g.ocs) == (g.is0, g.is1, g.is2, g.ies, g.ics)
    assert g.remap == 2 and g.log_m == 0 and g.flags == 0 and g.scale == 1.0
    tiles = g.t0n * g.t1n * 2
    assert tiles % (8 * 2) == 0          # the line-group order applies (grid a multiple of 8 s)
    # one image's tiles cover its C * C elements exactly once; the second
    # image's tiles are the first's shifted by is2 = C * C
    b = np.arange(g.t0n * g.t1n)
    t0, t1 = b % g.t0n, b // g.t0n
    base = t0 * g.is0 + t1 * g.is1
    idx = (base[:, None, None] + np.arange(8)[None, :, None] + np.arange(2048)[None, None, :] * g.ies).ravel()
    counts = np.bincount(idx, minlength=C * C)
    assert len(counts) == C * C and counts.min() == 1 and counts.max() == 1


def test_shape_copy_workloads_are_listed():
    import bench

    for name in ("shape_n10", "shape_n14", "shape_n15", "shape_cfg5col", "shape_cfg5row"):
        assert name in bench.OP_WORKLOADS and name in bench.WORKLOADS


def test_reference_table_is_the_published_one():
    # README.md:137-144 of the reference: µs per FFT at batch 256
    import bench

    assert {k: v[0] for k, v in bench.REFERENCE_US_PER_FFT.items()} == {"cfg1": 0.102, "cfg2_256": 0.035,
                                                                        "cfg2_4096": 0.509}
    for name in bench.REFERENCE_US_PER_FFT:
        assert bench.FFT_WORKLOADS[name][2] == 256

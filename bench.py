#!/usr/bin/env python3
"""Benchmark of the ferrum-gpu FFT hot path on one MI355X.

Workload (the one the north-star target is quoted on):
batched 1D forward C2C complex64 FFT, N = 1024, batch = 65536 (512 MiB in,
512 MiB out), re/im iid N(0,1) from seed 3, device-resident buffers.

A "step" is one execution of the plan over the whole batch.  W untimed
warmup steps, then K timed steps between two device synchronisations; every
step is also bracketed by HIP events on the stream the kernel runs on, which
gives the kernel's average launch duration for the roofline.

Prints ONE JSON line on stdout (progress goes to stderr):
  value        = algorithmic bytes per step (16 * N * batch) / wall time per step, GB/s
  roofline     = the dominant kernel's achieved algorithmic GB/s vs 8 TB/s HBM peak
  cpu_baseline = the CPU Stockham oracle (C restatement of the reference's
                 crates/ferrum-gpu-fft/src/cpu.rs), timed on this host
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "ferrum-gpu_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E peak, 8 TB/s
WORKLOADS = {
    # name: (log_n, batch, seed, distribution, description)
    "cfg3": (10, 65536, 3, "normal", "1D forward C2C FFT N=1024 batch=65536 complex64, re/im iid N(0,1) seed 3"),
    "cfg1": (10, 256, 1, "uniform", "1D forward C2C FFT N=1024 batch=256 complex64, re/im iid U[-1,1) seed 1"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_input(np, log_n, batch, seed, dist):
    rng = np.random.default_rng(seed)
    size = batch << log_n
    if dist == "normal":
        re = rng.standard_normal(size, dtype=np.float32)
        im = rng.standard_normal(size, dtype=np.float32)
    else:
        re = rng.uniform(-1, 1, size).astype(np.float32)
        im = rng.uniform(-1, 1, size).astype(np.float32)
    x = np.empty(size, np.complex64)
    x.real, x.imag = re, im
    return x


def traffic_for(kernel: str, workload: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE)
    and scaled by the plain copy kernel's reading, if such a measurement is
    committed under profiles/ for this kernel and workload; else None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
        entry = table.get(f"{kernel}@{workload}")
        return None if entry is None else float(entry["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def cpu_baseline(np, x, log_n, gpu_out, budget_s: float):
    """Time the CPU oracle on this host (the reported baseline, never the target)."""
    import oracle  # test infrastructure: used here only as the timed CPU baseline and checker

    n = 1 << log_n
    batch = x.size // n
    # 1 thread: the reference CPU path is single-threaded (cpu.rs:101).
    lanes = batch
    t0 = time.perf_counter()
    ref = oracle.fft_1d(x, log_n)
    t1 = time.perf_counter()
    once = t1 - t0
    reps = [once]
    while sum(reps) < budget_s and len(reps) < 50:
        t0 = time.perf_counter()
        oracle.fft_1d(x, log_n)
        reps.append(time.perf_counter() - t0)
    single = float(np.median(reps))
    # all cores the box gives this process (capped at 16, the box's CPU share)
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    threads = max(1, min(16, cores))
    multi_reps = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.fft_1d(x, log_n, threads=threads)
        multi_reps.append(time.perf_counter() - t0)
    multi = float(np.median(multi_reps))
    err = float(np.linalg.norm((gpu_out - ref).astype(np.complex128)) / np.linalg.norm(ref.astype(np.complex128)))
    nbytes = 16 * n * lanes
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    base = {
        "value": round(nbytes / single / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"full workload ({lanes} transforms of N={n}), median of {len(reps)} passes, "
                  f"{single:.3f} s/pass, oracle/oracle.c -O3 single thread",
        "gflops": round(5 * n * log_n * lanes / single / 1e9, 3),
        "cpu_model": cpu_model,
    }
    multi_d = {"value": round(nbytes / multi / 1e9, 4), "unit": "GB/s", "cores": threads,
               "seconds_per_pass": round(multi, 4)}
    return base, multi_d, err


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # The GPU reaches steady clocks after ~100 back-to-back launches of this
    # kernel (~20 ms); fewer warmup steps time the ramp, not the kernel.
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="cfg3", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of single-thread CPU timing")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "batched transforms shard by batch with no communication, so per-GPU work is the "
              "--gpus 1 workload", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    import numpy as np

    import ferrum_gpu
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import Device, DeviceBuffer, Event

    log_n, batch, seed, dist, desc = WORKLOADS[args.workload]
    n = 1 << log_n
    nbytes_io = 8 * n * batch
    algo_bytes = 2 * nbytes_io
    flops = 5.0 * n * log_n * batch

    dev = Device(0)
    info = dev.info()
    log(f"device {info}")
    log(f"workload {args.workload}: {desc}")
    x = make_input(np, log_n, batch, seed, dist)
    d_in, d_out = DeviceBuffer(dev, nbytes_io), DeviceBuffer(dev, nbytes_io)
    d_in.copy_from_host(x)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, dev)
    desc_plan = plan.describe()
    stream = dev.default_stream
    log(f"plan {desc_plan}")

    for _ in range(args.warmup):
        plan.execute(d_in, d_out, "forward", False, stream)
    dev.sync()
    log(f"warmup {args.warmup} done")

    evs = [Event(dev) for _ in range(args.steps + 1)]
    dev.sync()
    t0 = time.perf_counter()
    evs[0].record(stream)
    for k in range(args.steps):
        plan.execute(d_in, d_out, "forward", False, stream)
        evs[k + 1].record(stream)
    dev.sync()
    wall = time.perf_counter() - t0
    per_launch_ms = [evs[k].elapsed_ms(evs[k + 1]) for k in range(args.steps)]
    log(f"timed {args.steps} steps in {wall * 1e3:.3f} ms")

    ms_per_step = wall * 1e3 / args.steps
    value = algo_bytes / (ms_per_step * 1e-3) / 1e9
    avg_launch_ms = float(np.mean(per_launch_ms))
    med_launch_ms = float(np.median(per_launch_ms))
    achieved = algo_bytes / (avg_launch_ms * 1e-3) / 1e9

    # HBM yardstick: the code object's plain copy kernel over the same bytes.
    c0, c1 = Event(dev), Event(dev)
    copy_ms = []
    for _ in range(max(3, min(args.steps, 20))):
        c0.record(stream)
        N.check(N.lib.fg_stream_copy(dev.handle, d_in._p, d_out._p, nbytes_io, stream))
        c1.record(stream)
        c1.synchronize()
        copy_ms.append(c0.elapsed_ms(c1))
    copy_gbs = algo_bytes / (float(np.median(copy_ms)) * 1e-3) / 1e9

    # Output of the timed plan (re-run: the copy above overwrote d_out).
    plan.execute(d_in, d_out, "forward", False, stream)
    dev.sync()
    out = np.empty_like(x)
    d_out.copy_to_host(out)

    base = multi = None
    err = None
    if not args.no_cpu:
        log("cpu baseline ...")
        base, multi, err = cpu_baseline(np, x, log_n, out, args.cpu_budget)
        log(f"cpu baseline {base['value']} GB/s (1 core), {multi['value']} GB/s ({multi['cores']} cores); "
            f"gpu-vs-cpu rel_l2 {err:.3e}")

    traffic = traffic_for(desc_plan["main_kernel"], args.workload)
    result = {
        "metric": "batched C2C FFT GB/s (% HBM peak) + GFLOP/s (5Nlog2N), complex64",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": desc, "N": n, "batch": batch, "direction": "forward",
                   "layout": "interleaved complex64, device-resident"},
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "gflops": round(flops / (ms_per_step * 1e-3) / 1e9, 2),
        "kernel_avg_ms": round(avg_launch_ms, 5),
        "kernel_median_ms": round(med_launch_ms, 5),
        "stream_copy_gbs": round(copy_gbs, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": desc_plan["main_kernel"],
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": algo_bytes,
        },
        "cpu_baseline": base,
        "cpu_baseline_all_cores": multi,
        "rel_l2_vs_cpu": err,
        "device": info,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

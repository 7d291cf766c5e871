#!/usr/bin/env python3
"""Benchmark of the ferrum-gpu FFT hot path on one MI355X.

Default workload (the one the north-star target is quoted
on): batched 1D forward C2C complex64 FFT, N = 1024, batch = 65536 (512 MiB in,
512 MiB out), re/im iid N(0,1) from seed 3, device-resident buffers.
`--workload` selects the other BASELINE configurations (cfg1, cfg2_256,
cfg2_4096, cfg4, cfg5) for the numbers quoted in DESIGN.md.

A "step" is one pass of the hot path over the workload's batch (for cfg2: the
forward and the normalised inverse transform).  W untimed warmup steps, then
K timed steps between two device synchronisations.  Every kernel launch of the
timed steps is bracketed by HIP events recorded on the stream it runs on,
which gives each kernel's average duration for the roofline.

Prints ONE JSON line on stdout (progress goes to stderr):
  value        = algorithmic bytes per step (16 * elems * batch per transform
                 executed) / wall time per step, GB/s
  roofline     = the dominant kernel: bytes it moves per launch (it reads and
                 writes the whole array once) / its average launch duration,
                 against the 8 TB/s HBM peak
  cpu_baseline = the CPU Stockham oracle (C restatement of the reference's
                 crates/ferrum-gpu-fft/src/cpu.rs / cpu_2d.rs) timed on this host
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import threading
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "ferrum-gpu_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E peak, 8 TB/s

# name: dims, log_n, batch, seed, distribution, [(direction, normalize) per step], description
WORKLOADS = {
    "cfg3": (1, 10, 65536, 3, "normal", [("forward", False)],
             "1D forward C2C FFT N=1024 batch=65536 complex64, re/im iid N(0,1) seed 3"),
    "cfg1": (1, 10, 256, 1, "uniform", [("forward", False)],
             "1D forward C2C FFT N=1024 batch=256 complex64, re/im iid U[-1,1) seed 1"),
    "cfg2_256": (1, 8, 256, 2, "uniform", [("forward", False), ("inverse", True)],
                 "1D forward+inverse C2C FFT N=256 batch=256 complex64, re/im iid U[-1,1) seed 2"),
    "cfg2_4096": (1, 12, 256, 2, "uniform", [("forward", False), ("inverse", True)],
                  "1D forward+inverse C2C FFT N=4096 batch=256 complex64, re/im iid U[-1,1) seed 2"),
    "cfg4": (1, 24, 4, 4, "normal", [("forward", False)],
             "1D forward C2C FFT N=2^24 batch=4 complex64, re/im iid N(0,1) seed 4"),
    "cfg5": (2, 12, 2, 5, "uniform", [("forward", False)],
             "2D forward C2C FFT 4096x4096 batch=2 complex64, re/im iid U[-1,1) seed 5"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_input(np, size, seed, dist):
    rng = np.random.default_rng(seed)
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


def host_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(np, x, dims, log_n, batch, steps, gpu_out, budget_s: float):
    """Time the CPU oracle on this host (a reported baseline, never the target)
    and use its result as the checker of the GPU output."""
    import oracle  # test infrastructure: only the timed CPU baseline and checker

    elems = (1 << log_n) if dims == 1 else (1 << (2 * log_n))

    def run(buf, direction, normalize, threads):
        if dims == 1:
            return oracle.fft_1d(buf, log_n, direction, normalize, threads=threads)
        if threads <= 1 or batch < 2:
            return oracle.fft_2d(buf, log_n, direction, normalize)
        imgs = buf.reshape(batch, -1)
        out = np.empty_like(imgs)
        bounds = np.linspace(0, batch, min(threads, batch) + 1).astype(int)

        def part(lo, hi):
            out[lo:hi] = oracle.fft_2d(imgs[lo:hi], log_n, direction, normalize).reshape(hi - lo, -1)

        ts = [threading.Thread(target=part, args=(bounds[i], bounds[i + 1])) for i in range(len(bounds) - 1)]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        return out.reshape(-1)

    def one_step(threads):
        y = x
        for direction, normalize in steps:
            y = run(y, direction, normalize, threads)
        return y

    t0 = time.perf_counter()
    ref = one_step(1)
    reps = [time.perf_counter() - t0]
    while sum(reps) < budget_s and len(reps) < 50:
        t0 = time.perf_counter()
        one_step(1)
        reps.append(time.perf_counter() - t0)
    single = float(np.median(reps))
    threads = max(1, min(16, host_cores()))
    multi_reps = []
    for _ in range(3):
        t0 = time.perf_counter()
        one_step(threads)
        multi_reps.append(time.perf_counter() - t0)
    multi = float(np.median(multi_reps))
    err = float(np.linalg.norm((gpu_out - ref).astype(np.complex128)) / np.linalg.norm(ref.astype(np.complex128)))
    nbytes = 16 * elems * batch * len(steps)
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
        "sample": f"full workload ({batch} transforms x {len(steps)} direction(s)), median of {len(reps)} "
                  f"passes, {single:.3f} s/pass, oracle/oracle.c -O3, one thread",
        "cpu_model": cpu_model,
    }
    multi_d = {"value": round(nbytes / multi / 1e9, 4), "unit": "GB/s", "cores": threads,
               "seconds_per_pass": round(multi, 4)}
    return base, multi_d, err


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # The GPU reaches steady clocks after ~100 back-to-back launches of the
    # config-3 kernel (~20 ms); fewer warmup steps time the ramp, not the kernel.
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

    dims, log_n, batch, seed, dist, steps, desc = WORKLOADS[args.workload]
    elems = (1 << log_n) if dims == 1 else (1 << (2 * log_n))
    nbytes_io = 8 * elems * batch
    algo_bytes = 2 * nbytes_io * len(steps)           # per step
    flops_per_transform = 5.0 * elems * (log_n if dims == 1 else 2 * log_n)
    flops = flops_per_transform * batch * len(steps)

    dev = Device(0)
    info = dev.info()
    log(f"device {info}")
    log(f"workload {args.workload}: {desc}")
    x = make_input(np, elems * batch, seed, dist)
    bufs = [DeviceBuffer(dev, nbytes_io) for _ in range(len(steps) + 1)]
    bufs[0].copy_from_host(x)
    plan = (ferrum_gpu.fft.Plan1D if dims == 1 else ferrum_gpu.fft.Plan2D)(log_n, batch, dev)
    kernels = plan.kernel_names()
    launches = len(kernels)
    stream = dev.default_stream
    log(f"plan {plan.describe()} kernels {kernels}")

    def step(events=None):
        for j, (direction, normalize) in enumerate(steps):
            if events is None:
                plan.execute(bufs[j], bufs[j + 1], direction, normalize, stream)
            else:
                plan.execute_recording(bufs[j], bufs[j + 1], events[j], direction, normalize, stream)

    for _ in range(args.warmup):
        step()
    dev.sync()
    log(f"warmup {args.warmup} done")

    # One event after every launch (plus one before the first): launch i ran
    # between consecutive events.  One marker per launch costs ~2 us of gap per
    # launch; a pair per launch measured ~6 us.
    start = Event(dev)
    evs = [[[Event(dev) for _ in range(launches)] for _ in steps] for _ in range(args.steps)]
    dev.sync()
    t0 = time.perf_counter()
    start.record(stream)
    for k in range(args.steps):
        step(evs[k])
    dev.sync()
    wall = time.perf_counter() - t0
    log(f"timed {args.steps} steps in {wall * 1e3:.3f} ms")

    per_kernel: dict[str, list[float]] = {}
    prev = start
    for k in range(args.steps):
        for j in range(len(steps)):
            for i, name in enumerate(kernels):
                per_kernel.setdefault(f"{i}:{name}", []).append(prev.elapsed_ms(evs[k][j][i]))
                prev = evs[k][j][i]
    kernel_ms = {key: float(np.mean(v)) for key, v in per_kernel.items()}
    dominant = max(kernel_ms, key=lambda key: kernel_ms[key] * len(per_kernel[key]))
    dom_name = dominant.split(":", 1)[1]
    dom_avg = kernel_ms[dominant]
    bytes_per_launch = 2 * nbytes_io                  # each launch reads and writes the whole array once
    achieved = bytes_per_launch / (dom_avg * 1e-3) / 1e9

    ms_per_step = wall * 1e3 / args.steps
    value = algo_bytes / (ms_per_step * 1e-3) / 1e9

    # HBM yardstick: the code object's plain copy kernel over the same bytes.
    c0, c1 = Event(dev), Event(dev)
    copy_ms = []
    for _ in range(20):
        c0.record(stream)
        N.check(N.lib.fg_stream_copy(dev.handle, bufs[0]._p, bufs[1]._p, nbytes_io, stream))
        c1.record(stream)
        c1.synchronize()
        copy_ms.append(c0.elapsed_ms(c1))
    copy_gbs = 2 * nbytes_io / (float(np.median(copy_ms)) * 1e-3) / 1e9

    # Output of one step (recomputed: the copy above overwrote bufs[1]).
    step()
    dev.sync()
    out = np.empty_like(x)
    bufs[-1].copy_to_host(out)

    base = multi = err = None
    if not args.no_cpu:
        log("cpu baseline ...")
        base, multi, err = cpu_baseline(np, x, dims, log_n, batch, steps, out, args.cpu_budget)
        log(f"cpu baseline {base['value']} GB/s (1 core), {multi['value']} GB/s ({multi['cores']} cores); "
            f"gpu-vs-cpu rel_l2 {err:.3e}")

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
        "config": {"workload": desc, "name": args.workload, "dims": dims, "log_n": log_n, "batch": batch,
                   "directions": [d for d, _ in steps], "layout": "interleaved complex64, device-resident"},
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "gflops": round(flops / (ms_per_step * 1e-3) / 1e9, 2),
        "kernels_avg_ms": {key: round(v, 5) for key, v in kernel_ms.items()},
        "stream_copy_gbs": round(copy_gbs, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": dom_name,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_for(dom_name, args.workload),
            "bytes_per_launch": bytes_per_launch,
            "avg_launch_ms": round(dom_avg, 5),
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

#!/usr/bin/env python3
"""Benchmark of the ferrum-gpu FFT hot path on one MI355X.

Default workload (the one the north-star target is quoted
on): batched 1D forward C2C complex64 FFT, N = 1024, batch = 65536 (512 MiB in,
512 MiB out), re/im iid N(0,1) from seed 3, device-resident buffers.
`--workload` selects the other BASELINE configurations (cfg1, cfg2_256,
cfg2_4096, cfg4, cfg5), 1D lengths 8192 .. 32768 on the single-pass path
(1d_8192, 1d_16384, 1d_32768) and 2^16 / 2^18 / 2^20 on the two-pass path
(1d_2p16, 1d_2p18, 1d_2p20), 2D images on the one-pass path (2d_64, 2d_128) and
on the two-pass path (2d_512, 2d_1024), all 512 MiB batches and the operations beside the path (cfg3_split: config 3
in the split layout; cmul, cmul_split, deinterleave, interleave: the pointwise
kernels over config 3's 2^26 elements; transpose: an 8192 x 8192 complex64
matrix).

A "step" is one pass of the workload over its batch (for cfg2: the forward and
the normalised inverse transform).  A clock ramp (--ramp-ms of plain copy
kernels, not workload steps), W untimed warmup steps, then K timed steps
between two device synchronisations; `steady_state` compares the first and
last quarter of the timed launches, so a run still on a rising clock shows.  Every kernel launch of the timed steps
is followed by a HIP event recorded on the stream it runs on (plus one event
before the first), which gives each kernel's duration for the roofline.  With
--graph G the steps are recorded G at a time into a HIP graph and the timed
steps run as K / G replays (for the launch-bound configurations 1 and 2).

With the default workload the same run then times the other BASELINE
configurations (cfg1, cfg2_256, cfg2_4096, cfg4, cfg5) the way the reference's
bench does (10 warmup and 100 timed steps, the median step;
crates/ferrum-gpu-bench/src/lib.rs:31-37,148-213) and reports them under
`configs` in the same line: per-step and per-pass times, physical bytes for the
multi-pass plans, and the relative L2 error against the CPU oracle.

Prints ONE JSON line on stdout (progress goes to stderr):
  value        = algorithmic bytes per step / wall time per step, GB/s (FFT:
                 16 * elems * batch per transform executed)
  roofline     = the dominant kernel: algorithmic bytes it moves per launch /
                 its average launch duration, against the 8 TB/s HBM peak
  cpu_baseline = the CPU oracle (C restatement of the reference's CPU path)
                 timed on this host, also the checker of the GPU output
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

# FFT workloads: name -> (dims, log_n, batch, seed, distribution,
# [(direction, normalize) per step], layout, description)
FFT_WORKLOADS = {
    "cfg3": (1, 10, 65536, 3, "normal", [("forward", False)], "interleaved",
             "1D forward C2C FFT N=1024 batch=65536 complex64, re/im iid N(0,1) seed 3"),
    "cfg1": (1, 10, 256, 1, "uniform", [("forward", False)], "interleaved",
             "1D forward C2C FFT N=1024 batch=256 complex64, re/im iid U[-1,1) seed 1"),
    "cfg2_256": (1, 8, 256, 2, "uniform", [("forward", False), ("inverse", True)], "interleaved",
                 "1D forward+inverse C2C FFT N=256 batch=256 complex64, re/im iid U[-1,1) seed 2"),
    "cfg2_4096": (1, 12, 256, 2, "uniform", [("forward", False), ("inverse", True)], "interleaved",
                  "1D forward+inverse C2C FFT N=4096 batch=256 complex64, re/im iid U[-1,1) seed 2"),
    "cfg4": (1, 24, 4, 4, "normal", [("forward", False)], "interleaved",
             "1D forward C2C FFT N=2^24 batch=4 complex64, re/im iid N(0,1) seed 4"),
    "cfg5": (2, 12, 2, 5, "uniform", [("forward", False)], "interleaved",
             "2D forward C2C FFT 4096x4096 batch=2 complex64, re/im iid U[-1,1) seed 5"),
    "1d_8192": (1, 13, 8192, 8, "normal", [("forward", False)], "interleaved",
                "1D forward C2C FFT N=8192 batch=8192 complex64 (single pass), re/im iid N(0,1) seed 8"),
    "1d_16384": (1, 14, 4096, 9, "normal", [("forward", False)], "interleaved",
                 "1D forward C2C FFT N=16384 batch=4096 complex64 (single pass), re/im iid N(0,1) seed 9"),
    "1d_32768": (1, 15, 2048, 10, "normal", [("forward", False)], "interleaved",
                 "1D forward C2C FFT N=32768 batch=2048 complex64 (single pass), re/im iid N(0,1) seed 10"),
    "1d_2p16": (1, 16, 1024, 11, "normal", [("forward", False)], "interleaved",
                "1D forward C2C FFT N=2^16 batch=1024 complex64 (two passes), re/im iid N(0,1) seed 11"),
    "1d_2p18": (1, 18, 256, 12, "normal", [("forward", False)], "interleaved",
                "1D forward C2C FFT N=2^18 batch=256 complex64 (two passes), re/im iid N(0,1) seed 12"),
    "1d_2p20": (1, 20, 64, 13, "normal", [("forward", False)], "interleaved",
                "1D forward C2C FFT N=2^20 batch=64 complex64 (two passes), re/im iid N(0,1) seed 13"),
    "2d_512": (2, 9, 256, 14, "uniform", [("forward", False)], "interleaved",
               "2D forward C2C FFT 512x512 batch=256 complex64 (two passes), re/im iid U[-1,1) seed 14"),
    "2d_1024": (2, 10, 64, 15, "uniform", [("forward", False)], "interleaved",
                "2D forward C2C FFT 1024x1024 batch=64 complex64 (two passes), re/im iid U[-1,1) seed 15"),
    "2d_64": (2, 6, 16384, 6, "uniform", [("forward", False)], "interleaved",
              "2D forward C2C FFT 64x64 batch=16384 complex64 (one-pass path), re/im iid U[-1,1) seed 6"),
    "2d_128": (2, 7, 4096, 7, "uniform", [("forward", False)], "interleaved",
               "2D forward C2C FFT 128x128 batch=4096 complex64 (one-pass path), re/im iid U[-1,1) seed 7"),
    "cfg3_split": (1, 10, 65536, 3, "normal", [("forward", False)], "split",
                   "1D forward C2C FFT N=1024 batch=65536, split layout (re, im f32 arrays), "
                   "re/im iid N(0,1) seed 3"),
}
# Elementwise / data-movement workloads: name -> (elements, description)
OP_WORKLOADS = {
    "cmul": (1 << 26, "pointwise complex multiply out=a*b, 2^26 interleaved complex64, N(0,1) seeds 3/13"),
    "cmul_split": (1 << 26, "pointwise complex multiply, split layout, 2^26 elements, N(0,1) seeds 3/13"),
    "deinterleave": (1 << 26, "interleaved complex64 -> (re, im) f32 arrays, 2^26 elements, N(0,1) seed 3"),
    "interleave": (1 << 26, "(re, im) f32 arrays -> interleaved complex64, 2^26 elements, N(0,1) seed 3"),
    "transpose": (1 << 26, "out-of-place transpose of an 8192x8192 complex64 matrix, N(0,1) seed 3"),
    # Shape copies (fg_copy_shape_*): out = in with an FFT kernel's access
    # shape, workgroup size and LDS, no arithmetic -- that kernel's
    # memory-only floor on the same bytes.
    "shape_n10": (1 << 26, "copy with fg_fft_n10's access shape (config 3: 65536 x 1024 complex64), N(0,1) seed 3"),
    "shape_n14": (1 << 26, "copy with fg_fft_n14's access shape (4096 x 16384 complex64), N(0,1) seed 3"),
    "shape_n15": (1 << 26, "copy with fg_fft_n15's access shape (2048 x 32768 complex64), N(0,1) seed 3"),
    "shape_cfg5col": (1 << 25, "in-place copy with config 5's column pass geometry (fg_tile_l11_g8_h_cc over two "
                               "4096x4096 images: 2048-row tiles of 8 columns per row parity), U[-1,1) seed 5"),
    "shape_cfg5row": (1 << 25, "copy with config 5's row-pair pass shape (fg_fft2d_rowpair_n12: rows r and r + 2048 "
                               "of two 4096x4096 images in, rows 2r and 2r + 1 out), U[-1,1) seed 5"),
}
WORKLOADS = sorted(FFT_WORKLOADS) + sorted(OP_WORKLOADS)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_input(np, dev, size, seed, dist):
    """`size` complex64 values from the library's seeded generator (splitmix64;
    uniform in [-1, 1) or standard normal), generated on the device and copied
    to the host, where the CPU baseline reads them."""
    from ferrum_gpu import synthetic
    from ferrum_gpu.hip import DeviceBuffer

    buf = DeviceBuffer(dev, 8 * size)
    (synthetic.normal if dist == "normal" else synthetic.uniform)(dev, buf, size, seed)
    dev.sync()
    x = np.empty(size, np.complex64)
    buf.copy_to_host(x)
    buf.free()
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


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


class ClockSampler:
    """Samples the GPU's current shader clock from the kernel driver's sysfs
    table (`pp_dpm_sclk`, the level marked `*`) every few ms while active,
    the record the reference's bench keeps by locking clocks
    (tools/bench-gpu-lock.sh).  Plain file reads; the first DRM card with the
    table is taken (this build runs on one GPU).  Every failure leaves the
    report empty rather than stopping the bench."""

    def __init__(self, period_s: float = 0.002):
        import glob

        cards = sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk"))
        self.dir = os.path.dirname(cards[0]) if cards else None
        self.period = period_s
        self.samples: list[int] = []
        self._stop = threading.Event()
        self._thread = None

    def _level(self, name: str):
        try:
            with open(os.path.join(self.dir, name)) as f:
                for line in f:
                    if line.rstrip().endswith("*"):
                        return int(line.split(":")[1].strip().rstrip("*").strip().lower().rstrip("mhz"))
        except (OSError, ValueError, IndexError):
            return None
        return None

    def _run(self):
        while not self._stop.is_set():
            v = self._level("pp_dpm_sclk")
            if v is not None:
                self.samples.append(v)
            self._stop.wait(self.period)

    def __enter__(self):
        if self.dir:
            self._thread = threading.Thread(target=self._run, daemon=True)
            self._thread.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        if self._thread:
            self._thread.join()
        return False

    def report(self):
        if not self.dir:
            return None
        import statistics

        rep = {"source": self.dir + "/pp_dpm_{sclk,mclk}", "mclk_mhz": self._level("pp_dpm_mclk"),
               "sclk_samples": len(self.samples)}
        if self.samples:
            rep["sclk_mhz_median"] = statistics.median(self.samples)
            rep["sclk_mhz_max"] = max(self.samples)
        return rep


def in_threads(n_items: int, threads: int, part) -> None:
    """part(lo, hi) over [0, n_items) split across up to `threads` threads (the
    oracle's C calls drop the GIL)."""
    import numpy as np

    bounds = np.linspace(0, n_items, min(threads, n_items) + 1).astype(int)
    ts = [threading.Thread(target=part, args=(bounds[i], bounds[i + 1])) for i in range(len(bounds) - 1)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()


# ------------------------------------------------------------------ workloads
#
# A workload uploads its inputs, lists the kernels one step launches (with a
# key per launch that groups repeated launches of the same plan position), runs
# a step with an optional event after each launch, returns its output, and
# computes the same output with the CPU oracle (timed for cpu_baseline).


class FftWorkload:
    def __init__(self, name, np, dev):
        import ferrum_gpu
        from ferrum_gpu.hip import DeviceBuffer

        dims, log_n, batch, seed, dist, steps, layout, desc = FFT_WORKLOADS[name]
        self.np, self.dev, self.desc = np, dev, desc
        self.dims, self.log_n, self.batch, self.steps, self.layout = dims, log_n, batch, steps, layout
        self.elems = (1 << log_n) if dims == 1 else (1 << (2 * log_n))
        n = self.elems * batch
        self.nbytes_io = 8 * n
        self.algo_bytes = 2 * self.nbytes_io * len(steps)
        self.flops = 5.0 * self.elems * (log_n if dims == 1 else 2 * log_n) * batch * len(steps)
        self.exact = False
        self.x = make_input(np, dev, n, seed, dist)
        self.plan = (ferrum_gpu.fft.Plan1D if dims == 1 else ferrum_gpu.fft.Plan2D)(log_n, batch, dev)
        kernels = self.plan.kernel_names()
        if layout == "split":
            if self.plan.describe()["launches"] != 1:
                raise SystemExit("bench.py: split workloads are single-pass plans")
            kernels = [kernels[0] + "_split"]
            # (re, im) per stage of the chain: inputs, then one output per step
            self.parts = [(DeviceBuffer(dev, 4 * n), DeviceBuffer(dev, 4 * n)) for _ in range(len(steps) + 1)]
            self.parts[0][0].copy_from_host(np.ascontiguousarray(self.x.real))
            self.parts[0][1].copy_from_host(np.ascontiguousarray(self.x.imag))
            self.copy_bufs = (self.parts[0][0], self.parts[1][0], 4 * n)
        else:
            self.bufs = [DeviceBuffer(dev, self.nbytes_io) for _ in range(len(steps) + 1)]
            self.bufs[0].copy_from_host(self.x)
            self.copy_bufs = (self.bufs[0], self.bufs[1], self.nbytes_io)
        self.describe = self.plan.describe()
        # Multi-launch plans run pass after pass over one chunk of transforms
        # (images) at a time: launch i is pass i % passes of a chunk, and each
        # launch reads and writes one chunk once.
        passes = 1 if layout == "split" else self.describe["passes"]
        units = batch if layout == "split" else self.describe["units_per_chunk"]
        if batch % units:
            raise SystemExit("bench.py: workload batch is not a whole number of chunks")
        self.kernels = kernels
        self.launch_names = kernels * len(steps)
        self.launch_keys = [f"{i % passes}:{k}" for _ in steps for i, k in enumerate(kernels)]
        self.bytes_per_launch = 16 * self.elems * units
        # Two-stream plans run the odd chunks on the plan's second stream:
        # launch i of an execution (chunk i // passes) stamps its event there.
        self.streams = 1 if layout == "split" else self.describe["streams"]
        self._passes = passes
        L = len(kernels)
        self.launch_streams = [(i // passes) % 2 if self.streams == 2 else 0 for _ in steps for i in range(L)]
        self.exec_bounds = [(j * L, (j + 1) * L) for j in range(len(steps))]

    def set_streams(self, n):
        """Runs the plan's chunks on n streams (the plan's set_streams) and
        keeps the per-launch stream map of launch_durations in step."""
        self.plan.set_streams(n)
        self.streams = n
        L = len(self.kernels)
        self.launch_streams = [(i // self._passes) % 2 if n == 2 else 0 for _ in self.steps for i in range(L)]

    def bind_events(self, events):
        """The per-step form run() takes of one step's launch events (built
        before the timed loop: for interleaved plans, one EventList per
        execute call)."""
        from ferrum_gpu.hip import EventList

        if self.layout == "split":
            return list(events)
        L = len(self.kernels)
        return [EventList(events[j * L:(j + 1) * L]) for j in range(len(self.steps))]

    def run(self, stream, events=None):
        """One step; ``events`` is None or what bind_events returned."""
        for j, (direction, normalize) in enumerate(self.steps):
            if self.layout == "split":
                (ir, ii), (orr, oi) = self.parts[j], self.parts[j + 1]
                self.plan.execute_split(ir, ii, orr, oi, direction, normalize, stream)
                if events is not None:
                    events[j].record(stream)
            elif events is None:
                self.plan.execute(self.bufs[j], self.bufs[j + 1], direction, normalize, stream)
            else:
                self.plan.execute_recording(self.bufs[j], self.bufs[j + 1], events[j], direction, normalize,
                                            stream)

    def step_outputs(self):
        """The output of every step of the chain (interleaved layout)."""
        outs = []
        for buf in self.bufs[1:]:
            out = self.np.empty_like(self.x)
            buf.copy_to_host(out)
            outs.append(out)
        return outs

    def free(self):
        """Release the device buffers and the plan (the bench's other
        configurations run in the same process)."""
        for b in getattr(self, "bufs", []):
            b.free()
        for pair in getattr(self, "parts", []):
            for b in pair:
                b.free()
        self.plan.destroy()

    def output(self):
        np = self.np
        n = self.elems * self.batch
        if self.layout == "split":
            re, im = np.empty(n, np.float32), np.empty(n, np.float32)
            self.parts[-1][0].copy_to_host(re)
            self.parts[-1][1].copy_to_host(im)
            out = np.empty(n, np.complex64)
            out.real, out.imag = re, im
            return out
        out = np.empty_like(self.x)
        self.bufs[-1].copy_to_host(out)
        return out

    def cpu(self, threads: int):
        import oracle  # test infrastructure: only the timed CPU baseline and checker

        np = self.np

        def run(buf, direction, normalize):
            if self.dims == 1:
                return oracle.fft_1d(buf, self.log_n, direction, normalize, threads=threads)
            if threads <= 1 or self.batch < 2:
                return oracle.fft_2d(buf, self.log_n, direction, normalize)
            imgs = buf.reshape(self.batch, -1)
            out = np.empty_like(imgs)

            def part(lo, hi):
                out[lo:hi] = oracle.fft_2d(imgs[lo:hi], self.log_n, direction, normalize).reshape(hi - lo, -1)

            in_threads(self.batch, threads, part)
            return out.reshape(-1)

        y = self.x
        self.cpu_outputs = []
        for direction, normalize in self.steps:
            y = run(y, direction, normalize)
            self.cpu_outputs.append(y)
        return y

    def config(self):
        layout = ("split re/im f32 arrays" if self.layout == "split" else "interleaved complex64") + \
            ", device-resident"
        return {"dims": self.dims, "log_n": self.log_n, "batch": self.batch,
                "directions": [d for d, _ in self.steps], "layout": layout}

    def sample(self):
        return f"full workload ({self.batch} transforms x {len(self.steps)} direction(s))"


class TileGeomC:
    """ctypes mirror of TileGeom (ferrum-gpu_amd/csrc/kernels/tile_geom.h)."""

    @staticmethod
    def make(**kw):
        import ctypes

        class TileGeom(ctypes.Structure):
            _fields_ = ([(n, ctypes.c_uint64) for n in ("is0", "is1", "is2", "os0", "os1", "os2", "ics", "ies",
                                                        "ocs", "oes")] +
                        [(n, ctypes.c_uint32) for n in ("t0n", "t1n", "twc", "tw0", "tw1", "log_m", "flags")] +
                        [("scale", ctypes.c_float), ("remap", ctypes.c_uint32)])

        g = TileGeom()
        g.scale = 1.0
        for k, v in kw.items():
            setattr(g, k, v)
        return g


def cfg5_column_geom(log_n: int):
    """The geometry of the column pass of a 2D plan of 2^log_n x 2^log_n
    images after the row pairs (FftPlan::make_2d): tiles of 8 columns over
    the rows of each parity (element stride 2C), in place, line-group order."""
    C = 1 << log_n
    return TileGeomC.make(t0n=C // 8, t1n=2, is0=8, os0=8, is1=C, os1=C, is2=C * C, os2=C * C, ics=1, ocs=1,
                          ies=2 * C, oes=2 * C, remap=2)


class OpWorkload:
    """One launch per step of a pointwise kernel, the transpose or a shape copy."""

    def __init__(self, name, np, dev):
        from ferrum_gpu.hip import DeviceBuffer

        self.name, self.np, self.dev = name, np, dev
        n, self.desc = OP_WORKLOADS[name]
        self.n = n
        self.exact = True
        self.flops = 6.0 * n if name.startswith("cmul") else 0.0
        a = make_input(np, dev, n, 3, "normal")
        self.inputs = [a]
        # contiguous parts, prepared once for the split-layout kernels and the CPU leg
        self.parts = [np.ascontiguousarray(a.real), np.ascontiguousarray(a.imag)]
        f4 = 4 * n
        if name == "cmul":
            b = make_input(np, dev, n, 13, "normal")
            self.inputs.append(b)
            self.d_in = [DeviceBuffer(dev, 8 * n), DeviceBuffer(dev, 8 * n)]
            self.d_in[0].copy_from_host(a)
            self.d_in[1].copy_from_host(b)
            self.d_out = [DeviceBuffer(dev, 8 * n)]
            self.algo_bytes = 24 * n
            kernel = "fg_cmul_c64_vec"
        elif name == "cmul_split":
            b = make_input(np, dev, n, 13, "normal")
            self.inputs.append(b)
            self.parts += [np.ascontiguousarray(b.real), np.ascontiguousarray(b.imag)]
            self.d_in = [DeviceBuffer(dev, f4) for _ in range(4)]
            for buf, part in zip(self.d_in, self.parts):
                buf.copy_from_host(part)
            self.d_out = [DeviceBuffer(dev, f4), DeviceBuffer(dev, f4)]
            self.algo_bytes = 24 * n
            kernel = "fg_cmul_split_vec"
        elif name == "deinterleave":
            self.d_in = [DeviceBuffer(dev, 8 * n)]
            self.d_in[0].copy_from_host(a)
            self.d_out = [DeviceBuffer(dev, f4), DeviceBuffer(dev, f4)]
            self.algo_bytes = 16 * n
            kernel = "fg_deinterleave_c64_vec"
        elif name == "interleave":
            self.d_in = [DeviceBuffer(dev, f4), DeviceBuffer(dev, f4)]
            self.d_in[0].copy_from_host(self.parts[0])
            self.d_in[1].copy_from_host(self.parts[1])
            self.d_out = [DeviceBuffer(dev, 8 * n)]
            self.algo_bytes = 16 * n
            kernel = "fg_interleave_c64_vec"
        elif name.startswith("shape_"):
            import ctypes

            from ferrum_gpu.hip import Module

            if name == "shape_cfg5row":
                a = make_input(np, dev, n, 5, "uniform")
                self.inputs = [a]
                self.parts = []
                self.d_in = [DeviceBuffer(dev, 8 * n)]
                self.d_in[0].copy_from_host(a)
                self.d_out = [DeviceBuffer(dev, 8 * n)]
                self.pairs = ctypes.c_uint64(n >> 13)      # 2048 row pairs per 4096 x 4096 image
                self.log_rows = ctypes.c_uint32(12)
                self.grid = n >> 13
                self.block = 256
                kernel = "fg_copy_shape_rowpair_n12"
            elif name == "shape_cfg5col":
                a = make_input(np, dev, n, 5, "uniform")
                self.inputs = [a]
                self.parts = []
                self.d_in = [DeviceBuffer(dev, 8 * n)]
                self.d_in[0].copy_from_host(a)
                self.d_out = self.d_in            # in place, as the column pass runs
                self.geom = cfg5_column_geom(12)
                self.grid = (4096 // 8) * 2 * (n >> 24)
                self.block = 512
                kernel = "fg_copy_shape_tile_l11_g8_h_cc"
            else:
                log_n = int(name[len("shape_n"):])
                self.d_in = [DeviceBuffer(dev, 8 * n)]
                self.d_in[0].copy_from_host(a)
                self.d_out = [DeviceBuffer(dev, 8 * n)]
                self.batch = ctypes.c_uint64(n >> log_n)
                self.grid = (n >> log_n) // 2 if log_n == 10 else n >> log_n
                self.block = 128 if log_n == 10 else (1 << log_n) // 32
                kernel = f"fg_copy_shape_n{log_n}"
            self.algo_bytes = 16 * n
            self.exact = True
            self.fn = Module(dev).kernel(kernel)
        else:  # transpose
            self.side = 1 << 13
            assert self.side * self.side == n
            self.d_in = [DeviceBuffer(dev, 8 * n)]
            self.d_in[0].copy_from_host(a)
            self.d_out = [DeviceBuffer(dev, 8 * n)]
            self.algo_bytes = 16 * n
            kernel = "fg_transpose_c64_t128"   # 128 x 128 tiles for sides of at least 128
        self.kernels = [kernel]
        self.launch_names = [kernel]
        self.launch_keys = [f"0:{kernel}"]
        self.streams = 1
        self.launch_streams = [0]
        self.exec_bounds = [(0, 1)]
        self.bytes_per_launch = self.algo_bytes
        self.copy_bufs = (self.d_in[0], self.d_out[0], (min(self.d_in[0].nbytes, self.d_out[0].nbytes) // 16) * 16)
        self.describe = {"launches": 1, "main_kernel": kernel, "workspace_bytes": 0}

    def run(self, stream, events=None):
        import ferrum_gpu
        from ferrum_gpu import pointwise

        d, i, o = self.dev, self.d_in, self.d_out
        if self.name.startswith("shape_"):
            import ctypes

            ptrs = [ctypes.c_void_p(i[0].ptr), ctypes.c_void_p(o[0].ptr)]
            if self.name == "shape_cfg5col":
                args = ptrs + [self.geom]
            elif self.name == "shape_cfg5row":
                args = ptrs + [self.pairs, self.log_rows]
            else:
                args = ptrs + [self.batch]
            self.fn.launch((self.grid,), (self.block,), args, stream=stream)
        elif self.name == "cmul":
            pointwise.cmul(d, i[0], i[1], o[0], self.n, stream)
        elif self.name == "cmul_split":
            pointwise.cmul_split(d, i[0], i[1], i[2], i[3], o[0], o[1], self.n, stream)
        elif self.name == "deinterleave":
            pointwise.deinterleave(d, i[0], o[0], o[1], self.n, stream)
        elif self.name == "interleave":
            pointwise.interleave(d, i[0], i[1], o[0], self.n, stream)
        else:
            ferrum_gpu.fft.transpose(d, i[0], o[0], self.side, self.side, 1, stream)
        if events is not None:
            events[0].record(stream)

    def bind_events(self, events):
        return list(events)

    def output(self):
        np = self.np
        if len(self.d_out) == 2:
            outs = [np.empty(self.n, np.float32) for _ in range(2)]
            for buf, h in zip(self.d_out, outs):
                buf.copy_to_host(h)
            return np.concatenate(outs)
        out = np.empty(self.n, np.complex64)
        self.d_out[0].copy_to_host(out)
        return out

    def cpu(self, threads: int):
        import oracle  # test infrastructure: only the timed CPU baseline and checker

        np = self.np
        a = self.inputs[0]
        if self.name == "shape_cfg5row":
            # row r of each image's first half to row 2r, row r + 2048 to row 2r + 1
            imgs = a.reshape(-1, 2, 2048, 4096)
            return np.ascontiguousarray(imgs.transpose(0, 2, 1, 3)).reshape(-1)
        if self.name.startswith("shape_"):
            return a.copy()   # a copy: the output is the input
        if self.name == "transpose":
            out = a.copy()
            side = self.side
            if threads <= 1:
                oracle.transpose_square(out, side)
                return out
            # the oracle transposes one square in place; by threads, transpose
            # row blocks out of place with the same element order
            src, dst = a.reshape(side, side), out.reshape(side, side)

            def part(lo, hi):
                dst[:, lo:hi] = src[lo:hi, :].T

            in_threads(side, threads, part)
            return out
        n = self.n
        if self.name == "cmul":
            fn = lambda lo, hi: oracle.cmul_interleaved(a[lo:hi], self.inputs[1][lo:hi])  # noqa: E731
            res = np.empty(n, np.complex64)
        elif self.name == "cmul_split":
            ar, ai, br, bi = self.parts
            res = np.empty(2 * n, np.float32)

            def fn(lo, hi):
                return oracle.cmul_split(ar[lo:hi], ai[lo:hi], br[lo:hi], bi[lo:hi])
        elif self.name == "deinterleave":
            res = np.empty(2 * n, np.float32)
            fn = lambda lo, hi: oracle.deinterleave(a[lo:hi])  # noqa: E731
        else:
            res = np.empty(n, np.complex64)
            fn = lambda lo, hi: oracle.interleave(self.parts[0][lo:hi], self.parts[1][lo:hi])  # noqa: E731

        def part(lo, hi):
            r = fn(lo, hi)
            if isinstance(r, tuple):
                res[lo:hi], res[n + lo:n + hi] = r
            else:
                res[lo:hi] = r

        in_threads(n, max(1, threads), part)
        return res

    def config(self):
        if self.name == "transpose":
            return {"rows": self.side, "cols": self.side, "batch": 1, "layout": "interleaved complex64"}
        if self.name.startswith("shape_"):
            return {"elements": self.n, "kernel": self.kernels[0], "grid": self.grid, "block": self.block,
                    "layout": "interleaved complex64" + (", in place" if self.name == "shape_cfg5col" else "")}
        return {"elements": self.n,
                "layout": "split re/im f32 arrays" if self.name == "cmul_split" else "see workload"}

    def sample(self):
        if self.name == "transpose":
            return f"full workload ({self.side}x{self.side}; one thread: a copy, then the oracle's in-place swap)"
        return f"full workload ({self.n} elements)"


def host_path_rate(np, wl, dev, reps: int = 5):
    """The same step through the host-array entry points (fft_1d_c2c_pow2 /
    fft_2d_c2c_pow2 on numpy arrays): host-to-device copy, kernels, copy back.
    Reported beside `value`, never as it."""
    import ferrum_gpu

    x = wl.x if wl.dims == 1 else wl.x.reshape(wl.batch, 1 << wl.log_n, 1 << wl.log_n)
    fn = ferrum_gpu.fft.fft_1d_c2c_pow2 if wl.dims == 1 else ferrum_gpu.fft.fft_2d_c2c_pow2

    def step():
        y = x
        for direction, normalize in wl.steps:
            y = fn(y, wl.log_n, direction, normalize, device=dev)
        return y

    step()  # plan and staging buffers are created on the first call
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    return {"value": round(wl.algo_bytes / t / 1e9, 2), "unit": "GB/s", "ms_per_step": round(t * 1e3, 3),
            "note": "numpy in, numpy out: includes both PCIe copies and the output allocation; median of "
                    f"{reps} steps"}


def cpu_baseline(np, wl, gpu_out, budget_s: float):
    """Time the CPU oracle on this host (a reported baseline, never the target)
    and use its result as the checker of the GPU output."""
    t0 = time.perf_counter()
    ref = wl.cpu(1)
    reps = [time.perf_counter() - t0]
    while sum(reps) < budget_s and len(reps) < 50:
        t0 = time.perf_counter()
        wl.cpu(1)
        reps.append(time.perf_counter() - t0)
    single = float(np.median(reps))
    threads = max(1, min(16, host_cores()))
    multi_reps = []
    for _ in range(3):
        t0 = time.perf_counter()
        wl.cpu(threads)
        multi_reps.append(time.perf_counter() - t0)
    multi = float(np.median(multi_reps))
    if wl.exact:
        err = 0.0 if np.array_equal(gpu_out, ref) else float(
            np.max(np.abs(gpu_out.astype(np.complex128) - ref.astype(np.complex128))))
    else:
        err = float(np.linalg.norm((gpu_out - ref).astype(np.complex128)) /
                    np.linalg.norm(ref.astype(np.complex128)))
    base = {
        "value": round(wl.algo_bytes / single / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{wl.sample()}, median of {len(reps)} passes, {single:.3f} s/pass, "
                  "oracle/oracle.c -O3, one thread",
        "cpu_model": cpu_model(),
    }
    multi_d = {"value": round(wl.algo_bytes / multi / 1e9, 4), "unit": "GB/s", "cores": threads,
               "seconds_per_pass": round(multi, 4)}
    return base, multi_d, err


def clock_ramp(N, dev, wl, stream, ramp_ms: float):
    """Plain copy kernels over the workload's own buffers for ramp_ms of wall
    time, before the warmup steps: the shader clock idles low and needs tens of
    milliseconds of work to rise, which a short warmup does not give.  Not a
    step of the workload and not timed; reported in the JSON line."""
    if ramp_ms <= 0:
        return None
    src, dst, nbytes = wl.copy_bufs   # the yardstick's own size: every fg_copy_f4 dispatch moves the same bytes
    t0 = time.perf_counter()
    copies = 0
    while (time.perf_counter() - t0) * 1e3 < ramp_ms:
        for _ in range(8):
            N.check(N.lib.fg_stream_copy(dev.handle, src._p, dst._p, nbytes, stream))
        copies += 8
        dev.sync()
    return {"kernel": "fg_copy_f4", "copies": copies, "bytes_per_copy": nbytes,
            "ms": round((time.perf_counter() - t0) * 1e3, 1),
            "note": "untimed plain-copy launches before the warmup steps (clock ramp), not workload steps"}


def launch_durations(start, evs, wl) -> dict:
    """Per-launch GPU time from the events stamped after each launch of the
    timed steps (evs[k][i], launch i of step k): launch i ran from the
    previous event on its own stream, or from the end of the previous plan
    execution (the latest event of it, where a two-stream plan forks), to its
    own event.  One-stream plans: the gap between consecutive events."""
    t = [[start.elapsed_ms(e) for e in row] for row in evs]
    out: dict[str, list[float]] = {}
    exec_start = 0.0
    for k in range(len(evs)):
        for lo, hi in wl.exec_bounds:
            last: dict[int, float] = {}
            for i in range(lo, hi):
                s = wl.launch_streams[i]
                out.setdefault(wl.launch_keys[i], []).append(t[k][i] - last.get(s, exec_start))
                last[s] = t[k][i]
            exec_start = max(t[k][lo:hi])
    return out


def steady_state(np, per_kernel, dominant_key: str, graph: bool):
    """Whether the timed launches ran at a steady clock: the median duration of
    the dominant kernel's first quarter of timed launches against its last
    quarter (a ratio well above 1 means the first timed steps still ran on a
    rising clock)."""
    v = per_kernel[dominant_key]
    if graph or len(v) < 8:
        return {"launches": len(v), "note": "too few per-launch timings to compare quarters" if not graph
                else "graph replays are timed as a whole"}
    q = len(v) // 4
    first, last = float(np.median(v[:q])), float(np.median(v[-q:]))
    ratio = first / last if last > 0 else None
    return {"launches": len(v), "first_quarter_median_ms": round(first, 5),
            "last_quarter_median_ms": round(last, 5), "ratio": None if ratio is None else round(ratio, 4),
            "pre_ramp": bool(ratio is not None and ratio > 1.02)}


# The BASELINE configurations the default run reports beside config 3, and
# the reference bench's method for them: 10 warmup launches, then 100 timed
# ones, the median reported (crates/ferrum-gpu-bench/src/lib.rs:31-37,148-213).
EXTRA_CONFIGS = ["cfg1", "cfg2_256", "cfg2_4096", "cfg4", "cfg5"]
CONFIG_STEPS, CONFIG_WARMUP = 100, 10
GRAPH_STEPS_PER_REPLAY = 20
# The reference's one published table (README.md:123-153): batched 1D forward
# C2C at batch 256, µs per FFT = median event-timed launch / batch, on an RTX
# 5060 Laptop GPU (sm_120) at a locked 1500 MHz graphics clock, CUDA 13.1.
# Configs 1 and 2 are exactly those shapes.
REFERENCE_US_PER_FFT = {
    "cfg1": (0.102, "fft_c2c_1024"),
    "cfg2_256": (0.035, "fft_c2c_256"),
    "cfg2_4096": (0.509, "fft_c2c_4096"),
}
REFERENCE_TABLE_NOTE = ("the reference's published table (README.md:123-153): median of 100 event-timed "
                        "launches / batch 256, RTX 5060 Laptop GPU (sm_120), graphics clock locked at 1500 MHz, "
                        "CUDA 13.1 -- other hardware")


def timed_steps(dev, wl, stream, steps: int, warmup: int, clocks=None) -> dict:
    """`warmup` untimed steps, then `steps` timed ones back to back with an
    event stamped by every launch (plus one before the first).  Returns the
    host wall time, each launch key's durations (launch_durations) and each
    step's GPU time (from the end of the previous step's last launch to the
    end of its own)."""
    from ferrum_gpu.hip import Event

    # The events exist before the warmup steps, so that the GPU does not sit
    # idle (and the shader clock does not drop) between the last warmup step
    # and the timed ones while the host creates them.
    launches = len(wl.launch_names)
    start = Event(dev)
    evs = [[Event(dev) for _ in range(launches)] for _ in range(steps)]
    bound = [wl.bind_events(e) for e in evs]
    for _ in range(warmup):
        wl.run(stream)
    dev.sync()
    ctx = clocks if clocks is not None else _NullContext()
    with ctx:
        t0 = time.perf_counter()
        start.record(stream)
        for k in range(steps):
            wl.run(stream, bound[k])
        dev.sync()
        wall = time.perf_counter() - t0
    per_kernel = launch_durations(start, evs, wl)
    ends = [max(start.elapsed_ms(e) for e in row) for row in evs]
    step_ms = [ends[0]] + [ends[k] - ends[k - 1] for k in range(1, steps)]
    return {"wall_s": wall, "per_kernel": per_kernel, "step_ms": step_ms, "gpu_ms": ends[-1]}


class _NullContext:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


def graph_step_ms(dev, wl, stream, steps: int, warmup: int, per_graph: int) -> float:
    """GPU time per step with `per_graph` steps recorded into one HIP graph and
    replayed steps / per_graph times between two events (the launch-bound
    configurations' figure without the host's per-launch cost)."""
    from ferrum_gpu.hip import Capture, Event

    with Capture(dev, keep=[wl]) as cap:
        for _ in range(per_graph):
            wl.run(cap.stream)
    graph = cap.graph
    for _ in range(-(-warmup // per_graph)):
        graph.launch(stream)
    dev.sync()
    start, end = Event(dev), Event(dev)
    reps = max(1, steps // per_graph)
    start.record(stream)
    for _ in range(reps):
        graph.launch(stream)
    end.record(stream)
    dev.sync()
    ms = start.elapsed_ms(end) / (reps * per_graph)
    graph.destroy()
    return ms


def pass_table(np, wl, per_kernel: dict) -> list:
    """Each pass of the plan (launch key "i:kernel"): its launches' mean and
    median duration and the algorithmic bytes one launch moves over them."""
    rows = []
    for key in sorted(per_kernel, key=lambda k: int(k.split(":", 1)[0])):
        v = per_kernel[key]
        avg, med = float(np.mean(v)), float(np.median(v))
        gbs = wl.bytes_per_launch / (avg * 1e-3) / 1e9
        rows.append({"pass": int(key.split(":", 1)[0]), "kernel": key.split(":", 1)[1], "launches": len(v),
                     "avg_ms": round(avg, 5), "median_ms": round(med, 5), "bytes_per_launch": wl.bytes_per_launch,
                     "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)})
    return rows


def fp64_spot_check(np, wl, outs) -> float:
    """Relative L2 error of sampled bins of the first step's output (forward)
    against a direct DFT in fp64 (the reference's dft_naive_interleaved,
    layout_study.rs:5-21): 1D, bins of the first and last transform (16 up
    to 32768 points, 4 beyond: each bin costs O(N)); 2D, 8 bins (k1, k2) of
    the first and last image by a separable fp64 DFT."""
    from concurrent.futures import ThreadPoolExecutor

    import oracle  # test infrastructure: the checker only

    x, got = wl.x, outs[0]
    n, b = wl.elems, wl.batch
    rng = np.random.default_rng(wl.log_n)
    errs, refs = [], []
    for lane in sorted({0, b - 1}):
        xs, gs = x[lane * n:(lane + 1) * n], got[lane * n:(lane + 1) * n]
        if wl.dims == 1:
            # O(N) per bin with a cos and sin per term: 16 bins up to 32768
            # points, 4 beyond, one bin per thread (the C call drops the GIL)
            extra = 12 if n <= (1 << 15) else 1
            bins = np.unique(np.concatenate([[0, 1, n // 2, n - 1][:4 if extra > 1 else 3],
                                             rng.integers(0, n, extra)]))
            with ThreadPoolExecutor(max_workers=max(1, min(16, host_cores()))) as ex:
                exact = np.concatenate(list(ex.map(lambda k: oracle.dft_bins_f64(xs, [k]), bins.tolist())))
            sample = gs[bins]
        else:
            side = 1 << wl.log_n
            img = xs.reshape(side, side).astype(np.complex128)
            ks = rng.integers(0, side, (8, 2))
            ks[0] = (0, 0)
            idx = np.arange(side)
            exact = np.array([np.exp(-2j * np.pi * k1 * idx / side) @ (img @ np.exp(-2j * np.pi * k2 * idx / side))
                              for k1, k2 in ks])
            sample = gs.reshape(side, side)[ks[:, 0], ks[:, 1]]
        errs.append(sample.astype(np.complex128) - exact)
        refs.append(exact)
    e, r = np.concatenate(errs), np.concatenate(refs)
    return float(np.linalg.norm(e) / np.linalg.norm(r))


def config_record(np, N, dev, stream, name: str, steps: int, warmup: int, ramp_ms: float) -> tuple:
    """Times one BASELINE configuration on the GPU and returns (record, workload,
    outputs); the CPU checks are added by check_config afterwards."""
    wl = FftWorkload(name, np, dev)
    log(f"config {name}: {wl.desc}")
    clock_ramp(N, dev, wl, stream, ramp_ms)
    run = timed_steps(dev, wl, stream, steps, warmup)
    step_ms = run["step_ms"]
    med, mean = float(np.median(step_ms)), run["gpu_ms"] / steps
    d = wl.describe
    passes = pass_table(np, wl, run["per_kernel"])
    rec = {
        "workload": wl.desc,
        "kernels": wl.kernels,
        "plan": {k: d[k] for k in ("launches", "passes", "chunks", "units_per_chunk", "streams", "cache_resident")},
        "steps": steps, "warmup": warmup,
        "ms_per_step": round(med, 5),
        "ms_per_step_mean": round(mean, 5),
        "value": round(wl.algo_bytes / (med * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "pct_hbm_peak": round(100.0 * wl.algo_bytes / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
        "gflops": round(wl.flops / (med * 1e-3) / 1e9, 2),
        "algorithmic_bytes_per_step": wl.algo_bytes,
        "passes": passes,
        "timing": "GPU events stamped by every launch, steps back to back; ms_per_step is the median step "
                  "(the reference bench's statistic), value = algorithmic bytes / that median",
    }
    if d["passes"] > 1:
        phys = d["passes"] * wl.algo_bytes
        rec["physical_bytes_per_step"] = phys
        rec["physical_gbs"] = round(phys / (med * 1e-3) / 1e9, 1)
        rec["physical_pct_hbm_peak"] = round(100.0 * phys / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)
        rec["physical_note"] = ("each pass reads and writes every element once: passes x 16 bytes x elements per "
                                "step; intermediate passes are served partly by the Infinity Cache")
    if d["streams"] == 2:
        rec["passes_note"] = ("two chunks in flight on two streams: each launch's duration is its time while "
                              "sharing the GPU with the other stream's launch; passes_one_stream times the same "
                              "plan with its chunks on one stream (each pass alone on the GPU)")
        wl.set_streams(1)
        try:
            one = timed_steps(dev, wl, stream, steps, warmup)
        finally:
            wl.set_streams(2)
        rec["passes_one_stream"] = pass_table(np, wl, one["per_kernel"])
        rec["ms_per_step_one_stream"] = round(float(np.median(one["step_ms"])), 5)
    if wl.batch * wl.elems <= (1 << 22):
        # launch-bound sizes: the same steps as graph replays (no host cost per launch)
        g = graph_step_ms(dev, wl, stream, steps, warmup, GRAPH_STEPS_PER_REPLAY)
        rec["graph_ms_per_step"] = round(g, 5)
        rec["graph_value"] = round(wl.algo_bytes / (g * 1e-3) / 1e9, 2)
    if name in REFERENCE_US_PER_FFT:
        # per FFT as the reference's table counts it: one direction's launch / batch
        ffts = wl.batch * len(wl.steps)
        us = med * 1e3 / ffts
        ref_us, ref_kernel = REFERENCE_US_PER_FFT[name]
        rec["us_per_fft"] = round(us, 5)
        rec["reference_published"] = {"us_per_fft": ref_us, "kernel": ref_kernel, "note": REFERENCE_TABLE_NOTE}
        rec["reference_over_this"] = round(ref_us / us, 2)
        if "graph_ms_per_step" in rec:
            rec["graph_us_per_fft"] = round(rec["graph_ms_per_step"] * 1e3 / ffts, 5)
    wl.run(stream)
    dev.sync()
    outs = wl.step_outputs()
    wl.free()
    return rec, wl, outs


def check_config(np, rec: dict, wl, outs) -> None:
    """Adds the CPU oracle's verdict to a config record: relative L2 error of
    every step's output against the oracle's (computed outside the timed
    region), the round trip for forward + inverse chains, the fp64 spot
    check, and the oracle's own time on this host."""
    threads = max(1, min(16, host_cores(), wl.batch))
    t0 = time.perf_counter()
    wl.cpu(threads)
    secs = time.perf_counter() - t0
    refs = wl.cpu_outputs

    def rel(a, b):
        a = a.astype(np.complex128)
        b = b.astype(np.complex128)
        return float(np.linalg.norm(a - b) / np.linalg.norm(b))

    rec["rel_l2_vs_cpu"] = max(rel(o, r) for o, r in zip(outs, refs))
    rec["rel_l2_vs_cpu_per_step"] = [rel(o, r) for o, r in zip(outs, refs)]
    if len(wl.steps) == 2:
        rec["roundtrip_rel_l2"] = rel(outs[1], wl.x)
    rec["fp64_bins_rel_l2"] = fp64_spot_check(np, wl, outs)
    rec["cpu_oracle"] = {"seconds": round(secs, 4), "threads": threads,
                         "gbs": round(wl.algo_bytes / secs / 1e9, 4),
                         "note": "the C oracle (oracle/oracle.c -O3) on this host, one pass, as the checker"}
    rec["parity_ok"] = bool(rec["rel_l2_vs_cpu"] <= 1e-4 and rec["fp64_bins_rel_l2"] <= 1e-4 and
                            rec.get("roundtrip_rel_l2", 0.0) <= 1e-4)


def gate_check(result, min_frac):
    """The throughput gate of --min-frac: None without one, else whether the
    dominant kernel's roofline fraction reached it."""
    if min_frac is None:
        return None
    frac = result["roofline"]["frac"]
    return {"min_frac": min_frac, "frac": frac, "kernel": result["roofline"]["kernel"],
            "passed": bool(frac >= min_frac)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # The GPU reaches steady clocks after ~100 back-to-back launches of the
    # config-3 kernel (~20 ms); fewer warmup steps time the ramp, not the kernel.
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="cfg3", choices=WORKLOADS)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of single-thread CPU timing")
    ap.add_argument("--no-host-path", action="store_true",
                    help="skip timing the host-array entry points (PCIe-inclusive)")
    ap.add_argument("--ramp-ms", type=float, default=200.0,
                    help="before the warmup steps, run the plain copy kernel for this long (wall ms) so "
                         "that the shader clock leaves its idle level; reported as clock_ramp, 0 = off")
    ap.add_argument("--min-frac", type=float, default=None, metavar="F",
                    help="throughput gate: after printing the JSON line, exit with status 3 if the dominant "
                         "kernel's roofline fraction is below F (the reference's perf-gate, "
                         "crates/ferrum-gpu-bench/src/bin/perf-gate.rs, gates a ratio the same way)")
    ap.add_argument("--configs", default="auto", metavar="LIST",
                    help="comma-separated BASELINE configurations to time after the workload and report under "
                         "`configs` (" + ",".join(EXTRA_CONFIGS) + "); 'auto' (default): all of them when the "
                         "workload is cfg3, none otherwise; 'none': skip")
    ap.add_argument("--config-steps", type=int, default=CONFIG_STEPS,
                    help="timed steps per extra configuration (the reference bench: 100)")
    ap.add_argument("--config-warmup", type=int, default=CONFIG_WARMUP,
                    help="warmup steps per extra configuration (the reference bench: 10)")
    ap.add_argument("--graph", type=int, default=0, metavar="G",
                    help="record G steps into one HIP graph and time replays of it (for launch-bound "
                         "workloads); --steps must be a multiple of G.  0: one host launch per kernel")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "batched transforms shard by batch with no communication, so per-GPU work is the "
              "--gpus 1 workload", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2
    if args.graph < 0 or (args.graph and args.steps % args.graph):
        print("bench.py: --graph G needs G >= 1 dividing --steps", file=sys.stderr)
        return 2
    if args.configs == "auto":
        config_names = list(EXTRA_CONFIGS) if args.workload == "cfg3" else []
    elif args.configs == "none":
        config_names = []
    else:
        config_names = [c for c in args.configs.split(",") if c]
        bad = [c for c in config_names if c not in EXTRA_CONFIGS]
        if bad:
            print(f"bench.py: --configs takes {','.join(EXTRA_CONFIGS)}, 'auto' or 'none'; got {bad}",
                  file=sys.stderr)
            return 2
    if args.config_steps < 1 or args.config_warmup < 0:
        print("bench.py: --config-steps must be >= 1 and --config-warmup >= 0", file=sys.stderr)
        return 2

    import numpy as np

    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import Capture, Device, Event

    dev = Device(0)
    info = dev.info()
    log(f"device {info}")
    wl = (FftWorkload if args.workload in FFT_WORKLOADS else OpWorkload)(args.workload, np, dev)
    log(f"workload {args.workload}: {wl.desc}")
    stream = dev.default_stream
    log(f"plan {wl.describe} kernels {wl.kernels}")
    launches = len(wl.launch_names)

    per_kernel: dict[str, list[float]] = {}
    clocks = ClockSampler()
    ramp = clock_ramp(N, dev, wl, stream, args.ramp_ms)
    if ramp:
        log(f"clock ramp: {ramp['copies']} copy launches in {ramp['ms']} ms")
    if not args.graph:
        # One event stamped by every launch (plus one before the first): launch
        # i ran between consecutive events of its stream.
        run = timed_steps(dev, wl, stream, args.steps, args.warmup, clocks)
        wall = run["wall_s"]
        log(f"warmup {args.warmup} done; timed {args.steps} steps in {wall * 1e3:.3f} ms")
        per_kernel = run["per_kernel"]
    else:
        # G steps per graph, replayed steps / G times between two events: the
        # GPU time per launch is the replay time over all the launches in it
        # (for single-kernel steps: the kernel plus the in-graph dispatch gap).
        with Capture(dev, keep=[wl]) as cap:
            for _ in range(args.graph):
                wl.run(cap.stream)
        graph = cap.graph
        for _ in range(-(-args.warmup // args.graph)):
            graph.launch(stream)
        dev.sync()
        log(f"warmup {args.warmup} steps as graph replays done ({graph.node_count} nodes per graph)")
        start, end = Event(dev), Event(dev)
        dev.sync()
        with clocks:
            t0 = time.perf_counter()
            start.record(stream)
            for _ in range(args.steps // args.graph):
                graph.launch(stream)
            end.record(stream)
            dev.sync()
            wall = time.perf_counter() - t0
        per_launch = start.elapsed_ms(end) / (args.steps * launches)
        log(f"timed {args.steps} steps in {wall * 1e3:.3f} ms as {args.steps // args.graph} graph replays")
        for key in wl.launch_keys:
            per_kernel.setdefault(key, []).extend([per_launch] * args.steps)
        graph.destroy()
    steady = steady_state(np, per_kernel, dominant_key=max(per_kernel, key=lambda k: sum(per_kernel[k])),
                          graph=bool(args.graph))
    kernel_ms = {key: float(np.mean(v)) for key, v in per_kernel.items()}
    kernel_med = {key: float(np.median(v)) for key, v in per_kernel.items()}
    dominant = max(kernel_ms, key=lambda key: kernel_ms[key] * len(per_kernel[key]))
    dom_name = dominant.split(":", 1)[1]
    dom_avg = kernel_ms[dominant]
    achieved = wl.bytes_per_launch / (dom_avg * 1e-3) / 1e9

    ms_per_step = wall * 1e3 / args.steps
    value = wl.algo_bytes / (ms_per_step * 1e-3) / 1e9

    # HBM yardstick: the code object's plain copy kernel over the same bytes.
    src, dst, nbytes = wl.copy_bufs
    c0, c1 = Event(dev), Event(dev)
    copy_ms = []
    for _ in range(20):
        c0.record(stream)
        N.check(N.lib.fg_stream_copy(dev.handle, src._p, dst._p, nbytes, stream))
        c1.record(stream)
        c1.synchronize()
        copy_ms.append(c0.elapsed_ms(c1))
    copy_gbs = 2 * nbytes / (float(np.median(copy_ms)) * 1e-3) / 1e9

    # Output of one step (recomputed: the copy above overwrote an output).
    wl.run(stream)
    dev.sync()
    out = wl.output()

    # The other BASELINE configurations, timed on the GPU one after another
    # (their CPU checks come after the headline's CPU baseline below).
    extra = []
    # A configuration that raises records its error instead of costing the
    # headline line (a GPU fault ends the process either way).
    config_errors = {}
    for name in config_names:
        try:
            extra.append((name,) + config_record(np, N, dev, stream, name, args.config_steps, args.config_warmup,
                                                 args.ramp_ms))
            log(f"config {name}: {extra[-1][1]['ms_per_step']} ms per step (median of {args.config_steps})")
        except Exception as e:  # noqa: BLE001 -- reported in the JSON line
            config_errors[name] = f"{type(e).__name__}: {e}"
            log(f"config {name} failed: {config_errors[name]}")

    host = None
    if not args.no_host_path and isinstance(wl, FftWorkload) and wl.layout == "interleaved":
        host = host_path_rate(np, wl, dev)
        log(f"host path {host['value']} GB/s ({host['ms_per_step']} ms per step)")

    base = multi = err = None
    if not args.no_cpu:
        log("cpu baseline ...")
        base, multi, err = cpu_baseline(np, wl, out, args.cpu_budget)
        log(f"cpu baseline {base['value']} GB/s (1 core), {multi['value']} GB/s ({multi['cores']} cores); "
            f"gpu-vs-cpu {'max abs diff' if wl.exact else 'rel_l2'} {err:.3e}")

    configs = None
    if config_names:
        configs = {}
        for name, rec, cwl, outs in extra:
            try:
                check_config(np, rec, cwl, outs)
                log(f"config {name}: rel_l2 {rec['rel_l2_vs_cpu']:.3e}, fp64 bins {rec['fp64_bins_rel_l2']:.3e}")
            except Exception as e:  # noqa: BLE001 -- reported in the JSON line
                rec["check_error"] = f"{type(e).__name__}: {e}"
                rec["parity_ok"] = False
            configs[name] = rec
        for name, err in config_errors.items():
            configs[name] = {"error": err, "parity_ok": False}
        del extra

    config = {"workload": wl.desc, "name": args.workload}
    config.update(wl.config())
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
        "config": config,
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "gflops": round(wl.flops / (ms_per_step * 1e-3) / 1e9, 2),
        "kernels_avg_ms": {key: round(v, 5) for key, v in kernel_ms.items()},
        "kernels_median_ms": {key: round(v, 5) for key, v in kernel_med.items()},
        "stream_copy_gbs": round(copy_gbs, 1),
        "stream_copy_bytes": nbytes,
        "roofline": {
            "bound": "hbm",
            "kernel": dom_name,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_for(dom_name, args.workload),
            "bytes_per_launch": wl.bytes_per_launch,
            "avg_launch_ms": round(dom_avg, 5),
        },
        "cpu_baseline": base,
        "cpu_baseline_all_cores": multi,
        "host_path": host,
        ("max_abs_diff_vs_cpu" if wl.exact else "rel_l2_vs_cpu"): err,
        "device": info,
        "gpu_clocks": clocks.report(),
        "clock_ramp": ramp,
        "steady_state": steady,
    }
    if configs is not None:
        result["configs"] = configs
    if args.graph:
        result["launch_mode"] = f"HIP graph of {args.graph} steps per replay"
    else:
        result["launch_mode"] = "one host launch per kernel, one event after each" + (
            "; odd chunks on the plan's second stream" if wl.streams == 2 else "")

    gate = gate_check(result, args.min_frac)
    if gate is not None:
        result["gate"] = gate
    print(json.dumps(result), flush=True)
    if gate is not None and not gate["passed"]:
        print(f"bench.py: gate failed: roofline frac {gate['frac']} < {gate['min_frac']}", file=sys.stderr)
        return 3
    return 0


if __name__ == "__main__":
    sys.exit(main())

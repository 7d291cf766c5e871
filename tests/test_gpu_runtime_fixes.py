"""GPU tests of runtime behaviour at the C ABI's edges.

* An event recorded with stream NULL (Python ``Event.record()``) lands on the
  device's default stream, the one ``Plan.execute()`` and the copies use
  for NULL, so it brackets a default-stream execution.
* Kernel handles of the transpose and the streaming copy belong to the device
  whose module they came from: a device opened after another was closed
  (whose module, and so its handles, are gone) launches its own.
* The first split-layout execution of a multi-launch plan allocates its
  staging buffer synchronously, which a stream capture cannot record: on a
  capturing stream it is refused before any allocation, and the capture ends
  cleanly with what was recorded before it.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from conftest import normal_c64, rel_l2, uniform_c64

pytestmark = pytest.mark.gpu

TOL = 1e-4


def test_null_stream_events_bracket_default_stream_work(gpu_device):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer, Event

    log_n, batch = 10, 65536  # config 3: ~0.18 ms per execution
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    a, b = DeviceBuffer(gpu_device, plan.nbytes), DeviceBuffer(gpu_device, plan.nbytes)
    ferrum_gpu.synthetic.normal(gpu_device, a, batch << log_n, 3)
    gpu_device.sync()
    start, end = Event(gpu_device), Event(gpu_device)
    reps = 10
    start.record()                       # stream 0: the device default stream
    for _ in range(reps):
        plan.execute(a, b)               # stream 0: the device default stream
    end.record()
    end.synchronize()
    ms = start.elapsed_ms(end)
    # ten executions of a 1 GiB pass cannot take under 0.1 ms each (10 TB/s);
    # events on another stream would bracket nothing (~0 ms)
    assert ms >= 0.1 * reps, f"events bracket {ms} ms for {reps} executions"
    # and end.synchronize() waited for the work: the output is complete now,
    # read back without any further device synchronisation
    out = np.empty(batch << log_n, np.complex64)
    ferrum_gpu._native.check(ferrum_gpu._native.lib.fg_copy_d2h(
        gpu_device.handle, out.ctypes.data, b._p, out.nbytes))
    x = np.empty_like(out)
    a.copy_to_host(x)
    lanes = slice(0, 64 << log_n)
    assert rel_l2(out[lanes], oracle.fft_1d(x[lanes], log_n)) <= TOL
    plan.destroy()


def test_transpose_and_copy_on_a_reopened_device(gpu_device):
    import ferrum_gpu
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import Device, DeviceBuffer

    rows, cols = 96, 200
    x = uniform_c64(np.random.default_rng(11), rows * cols)
    for round_ in range(3):
        print(f"[case] reopen round {round_}", flush=True)
        dev = Device(0)
        a, b, c = (DeviceBuffer(dev, x.nbytes + 64) for _ in range(3))
        a.copy_from_host(x)
        ferrum_gpu.fft.transpose(dev, a, b, rows, cols)
        N.check(N.lib.fg_stream_copy(dev.handle, b._p, c._p, (x.nbytes // 16) * 16, None))
        dev.sync()
        t = np.empty_like(x)
        b.copy_to_host(t)
        assert np.array_equal(t, x.reshape(rows, cols).T.reshape(-1))
        cp = np.empty(x.nbytes // 16 * 2, np.complex64)
        c.copy_to_host(cp)
        assert np.array_equal(cp, t[:cp.size])
        for buf in (a, b, c):
            buf.free()
        dev.close()


@pytest.mark.parametrize("dims,log_n,batch", [(1, 16, 3), (2, 12, 1)])
def test_first_split_call_refused_under_capture(gpu_device, dims, log_n, batch):
    import ferrum_gpu
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import Capture, DeviceBuffer

    print(f"[case] split under capture dims={dims} log_n={log_n}", flush=True)
    elems = 1 << (log_n * dims)
    n = batch * elems
    x = normal_c64(np.random.default_rng(log_n), n)
    re, im = np.ascontiguousarray(x.real), np.ascontiguousarray(x.imag)
    plan = (ferrum_gpu.fft.Plan1D if dims == 1 else ferrum_gpu.fft.Plan2D)(log_n, batch, gpu_device)
    assert plan.describe()["launches"] > 1
    small = ferrum_gpu.fft.Plan1D(8, 4, gpu_device)  # a single-pass plan recorded beside it
    s_buf = DeviceBuffer(gpu_device, small.nbytes)
    y = uniform_c64(np.random.default_rng(1), 4 << 8)
    s_buf.copy_from_host(y)
    parts = [DeviceBuffer(gpu_device, 4 * n) for _ in range(4)]
    parts[0].copy_from_host(re)
    parts[1].copy_from_host(im)

    with Capture(gpu_device, keep=[small]) as cap:
        small.execute(s_buf, s_buf, stream=cap.stream)
        with pytest.raises(N.FerrumGpuError) as e:
            plan.execute_split(parts[0], parts[1], parts[2], parts[3], stream=cap.stream)
        assert e.value.code == N.FG_ERR_INVALID_ARGUMENT and "capture" in str(e.value)
    graph = cap.graph                     # the capture ended cleanly with the one node
    assert graph.node_count == 1
    graph.launch()
    gpu_device.sync()
    got = s_buf.copy_to_host(np.empty_like(y))
    assert rel_l2(got, oracle.fft_1d(y, 8)) <= TOL
    graph.destroy()

    # Eager, the first call allocates and runs; after it the split path can be captured.
    plan.execute_split(parts[0], parts[1], parts[2], parts[3])
    gpu_device.sync()
    out_re, out_im = parts[2].copy_to_host(np.empty_like(re)), parts[3].copy_to_host(np.empty_like(im))
    eager = (out_re + 1j * out_im).astype(np.complex64)
    ref = oracle.fft_1d(x, log_n) if dims == 1 else oracle.fft_2d(x, log_n)
    assert rel_l2(eager, ref) <= TOL
    with Capture(gpu_device, keep=[plan]) as cap:
        plan.execute_split(parts[0], parts[1], parts[2], parts[3], stream=cap.stream)
    graph = cap.graph
    assert graph.node_count == plan.describe()["launches"] + 2
    for replay in range(2):
        parts[2].copy_from_host(np.zeros_like(re))
        gpu_device.sync()
        graph.launch()
        gpu_device.sync()
        again = parts[2].copy_to_host(np.empty_like(re))
        assert np.array_equal(again, out_re), f"replay {replay}"
    graph.destroy()
    plan.destroy()
    small.destroy()


def test_batches_beyond_one_launch_run_in_chunks(gpu_device):
    # A single-pass plan whose batch exceeds one launch's 2^32 - 1 work-items
    # runs as several launches (never a truncated grid): N = 4 at 2^32
    # transforms is 64 work-items per 64 transforms, so 2^32 - 64 transforms
    # per launch and two launches.  Created, described, never executed here.
    import ferrum_gpu

    print("[case] Plan1D(2, 2**32) and Plan1D(2, 2**32 - 64): chunking only", flush=True)
    p = ferrum_gpu.fft.Plan1D(2, 2**32, gpu_device)
    d = p.describe()
    assert d["launches"] == 2 and d["chunks"] == 2 and d["units_per_chunk"] == 2**32 - 64
    assert p.kernel_names() == ["fg_fft_n2", "fg_fft_n2"]
    p.destroy()
    q = ferrum_gpu.fft.Plan1D(2, 2**32 - 64, gpu_device)
    assert q.describe()["launches"] == 1
    q.destroy()


def test_in_place_kernel_names(gpu_device):
    # 4096 x 4096 (config 5): out of place the row pairs and 2048-row column
    # tiles, in place the 4096-point rows and 4096-row column tiles, as many
    # launches; every other plan names the same kernels both ways
    import ferrum_gpu

    p = ferrum_gpu.fft.Plan2D(12, 2, gpu_device)
    assert p.kernel_names() == ["fg_fft2d_rowpair_n12", "fg_tile_l11_g8_h_cc"]
    assert p.kernel_names(in_place=True) == ["fg_fft_n12_sc", "fg_tile_l12_g8_h_cc"]
    p.destroy()
    # 1024 x 2048: 512-row column tiles after the row pairs, 1024-row ones in place
    p = ferrum_gpu.fft.Plan2D(10, 2, gpu_device, log_cols=11)
    assert p.kernel_names() == ["fg_fft2d_rowpair_n11", "fg_tile_l9_g16_h_cs"]
    assert p.kernel_names(in_place=True) == ["fg_fft_n11_sc", "fg_tile_l10_g16_h_cs"]
    p.destroy()
    for plan in (ferrum_gpu.fft.Plan1D(24, 4, gpu_device), ferrum_gpu.fft.Plan2D(10, 4, gpu_device),
                 ferrum_gpu.fft.Plan1D(10, 4096, gpu_device)):
        assert plan.kernel_names(in_place=True) == plan.kernel_names()
        plan.destroy()


def test_batch_beyond_one_launch_executes_in_chunks(gpu_device):
    # 2^32 transforms of N = 4 (128 GiB, in place): two launches, the second
    # of 64 transforms at byte offset 32 * (2^32 - 64).  The transforms on
    # both sides of the launch boundary, and the first and last, equal the
    # same plan kernel on a small batch bit for bit and the oracle to 1e-6.
    import ferrum_gpu
    from ferrum_gpu import _native as N
    from ferrum_gpu import synthetic
    from ferrum_gpu.hip import DeviceBuffer

    if gpu_device.info()["total_mem"] < (200 << 30):
        pytest.skip("needs a GPU with 200 GiB or more")
    batch = 2**32
    n = 4 * batch
    print("[case] Plan1D(2, 2**32) in place over 128 GiB, two launches", flush=True)
    try:
        buf = DeviceBuffer(gpu_device, 8 * n)
    except N.FerrumGpuError as e:
        pytest.skip(f"128 GiB not available: {e}")
    try:
        synthetic.uniform(gpu_device, buf, n, 77)
        gpu_device.sync()
        lanes = [0, 1, 2**32 - 66, 2**32 - 65, 2**32 - 64, 2**32 - 63, 2**32 - 2, 2**32 - 1]

        def read(lane):
            h = np.empty(4, np.complex64)
            N.check(N.lib.fg_copy_d2h(gpu_device.handle, h.ctypes.data, buf.ptr + 32 * lane, 32))
            return h

        x = np.concatenate([read(lane) for lane in lanes])
        plan = ferrum_gpu.fft.Plan1D(2, batch, gpu_device)
        assert plan.describe()["launches"] == 2
        plan.execute(buf, buf, "forward", False)
        gpu_device.sync()
        got = np.concatenate([read(lane) for lane in lanes])
        plan.destroy()
    finally:
        buf.free()
    small = ferrum_gpu.fft.Plan1D(2, len(lanes), gpu_device)
    a, b = DeviceBuffer(gpu_device, small.nbytes), DeviceBuffer(gpu_device, small.nbytes)
    a.copy_from_host(x)
    small.execute(a, b, "forward", False)
    gpu_device.sync()
    want = np.empty_like(x)
    b.copy_to_host(want)
    small.destroy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert rel_l2(got, oracle.fft_1d(x, 2)) <= 1e-6


@pytest.mark.parametrize("kind,log_n,batch", [("1d", 15, 600), ("1d", 14, 1100), ("2d", 7, 1100)])
def test_staggered_start_keeps_the_bits(gpu_device, kind, log_n, batch):
    # The kernels with one or two workgroups per CU delay their first round's
    # workgroups when the grid spans two or more rounds (fg_fft_n15 from 512
    # transforms, fg_fft_n14 and 16384-point images from 1024).  The delay
    # changes no arithmetic: transforms at both ends of such a batch equal,
    # bit for bit, the same transforms run as a batch of 8 (no delay), and
    # the oracle within 1e-4, forward and normalised inverse.
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    elems = 1 << (log_n if kind == "1d" else 2 * log_n)
    x = normal_c64(np.random.default_rng(log_n * 7 + batch), batch * elems)
    lanes = [0, 1, 2, 3, batch - 4, batch - 3, batch - 2, batch - 1]
    sub = np.concatenate([x[i * elems:(i + 1) * elems] for i in lanes])
    print(f"[case] stagger {kind} log_n={log_n} batch={batch}", flush=True)
    mk = ferrum_gpu.fft.Plan1D if kind == "1d" else ferrum_gpu.fft.Plan2D
    for direction, normalize in (("forward", False), ("inverse", True)):
        outs = []
        for data, b in ((x, batch), (sub, len(lanes))):
            plan = mk(log_n, b, gpu_device)
            a, o = DeviceBuffer(gpu_device, plan.nbytes), DeviceBuffer(gpu_device, plan.nbytes)
            a.copy_from_host(data)
            plan.execute(a, o, direction, normalize)
            gpu_device.sync()
            y = np.empty_like(data)
            o.copy_to_host(y)
            outs.append(y)
            plan.destroy()
            a.free()
            o.free()
        big = np.concatenate([outs[0][i * elems:(i + 1) * elems] for i in lanes])
        assert np.array_equal(big.view(np.uint32), outs[1].view(np.uint32))
        ref = (oracle.fft_1d(sub, log_n, direction, normalize, threads=8) if kind == "1d"
               else oracle.fft_2d(sub, log_n, direction, normalize))
        assert rel_l2(outs[1], ref) <= 1e-4

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

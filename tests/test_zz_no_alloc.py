"""fg_fft_exec_split_noalloc, the allocation-free variant of fg_fft_exec_split.

No counterpart in the reference.  Multi-launch plans stage through the
library's fixed 64 MiB device scratch area instead of a lazily allocated
buffer of their own.  Bar: bit for bit what fg_fft_exec_split gives (same
kernels on the same data), and relative L2 <= 1e-4 against the CPU oracle.
Calls are made through the C ABI, two in a row with the second smaller than
the first (the area keeps the previous call's contents).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from conftest import normal_c64, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4
SCRATCH_BYTES = 64 << 20


def _parts(dev, x):
    from ferrum_gpu.hip import DeviceBuffer

    ins = []
    for h in (np.ascontiguousarray(x.real), np.ascontiguousarray(x.imag)):
        b = DeviceBuffer(dev, h.nbytes)
        b.copy_from_host(h)
        ins.append(b)
    outs = [DeviceBuffer(dev, 4 * x.size) for _ in range(2)]
    return ins, outs


def _read(dev, outs, n):
    dev.sync()
    re, im = np.empty(n, np.float32), np.empty(n, np.float32)
    outs[0].copy_to_host(re)
    outs[1].copy_to_host(im)
    return (re + 1j * im).astype(np.complex64)


def _call(fn, plan, ins, outs, direction, normalize, stream=None):
    from ferrum_gpu import _native as N

    d = N.FG_FORWARD if direction == "forward" else N.FG_INVERSE
    return fn(plan._p, ins[0]._p, ins[1]._p, outs[0]._p, outs[1]._p, d, int(normalize), ctypes.c_void_p(stream))


def _plan(dev, dims, log_n, batch):
    import ferrum_gpu

    return (ferrum_gpu.fft.Plan1D if dims == 1 else ferrum_gpu.fft.Plan2D)(log_n, batch, dev)


# Two multi-launch calls in a row, the second smaller than the first (the
# first fills the 64 MiB area exactly), then a single-pass plan (no staging).
CALLS = [(1, 20, 8, "forward", False), (2, 8, 3, "inverse", True), (1, 10, 5, "forward", False)]


def test_noalloc_equals_split_on_consecutive_calls(gpu_device):
    from ferrum_gpu import _native as N

    for i, (dims, log_n, batch, direction, normalize) in enumerate(CALLS):
        print(f"[case] noalloc call {i}: dims={dims} log_n={log_n} batch={batch} {direction}", flush=True)
        plan = _plan(gpu_device, dims, log_n, batch)
        n = batch << (log_n * dims)
        assert 8 * n <= SCRATCH_BYTES
        x = normal_c64(np.random.default_rng(100 + i), n)
        ins, outs = _parts(gpu_device, x)
        N.check(_call(N.lib.fg_fft_exec_split_noalloc, plan, ins, outs, direction, normalize))
        got = _read(gpu_device, outs, n)
        outs2 = _parts(gpu_device, x)[1]
        N.check(_call(N.lib.fg_fft_exec_split, plan, ins, outs2, direction, normalize))
        ref_split = _read(gpu_device, outs2, n)
        assert np.array_equal(got.view(np.uint32), ref_split.view(np.uint32)), f"call {i}: differs from exec_split"
        ref = (oracle.fft_1d(x, log_n, direction, normalize, threads=8) if dims == 1
               else oracle.fft_2d(x, log_n, direction, normalize))
        assert rel_l2(got, ref) <= TOL
        # in place (out == in) as well
        N.check(_call(N.lib.fg_fft_exec_split_noalloc, plan, ins, ins, direction, normalize))
        assert np.array_equal(_read(gpu_device, ins, n).view(np.uint32), ref_split.view(np.uint32))
        plan.destroy()


def test_noalloc_refuses_plans_beyond_the_scratch_area(gpu_device):
    from ferrum_gpu import _native as N

    plan = _plan(gpu_device, 1, 20, 9)          # 72 MiB of staging
    n = 9 << 20
    x = normal_c64(np.random.default_rng(5), n)
    ins, outs = _parts(gpu_device, x)
    sentinel = np.full(n, 3.25, np.float32)
    outs[0].copy_from_host(sentinel)
    rc = _call(N.lib.fg_fft_exec_split_noalloc, plan, ins, outs, "forward", False)
    assert rc == N.FG_ERR_INVALID_ARGUMENT
    assert "beyond the 67108864-byte device scratch area" in N.last_error()
    gpu_device.sync()
    after = np.empty(n, np.float32)
    outs[0].copy_to_host(after)
    assert np.array_equal(after, sentinel)      # nothing was launched
    plan.destroy()


def test_noalloc_call_captured_on_a_fresh_plan(gpu_device):
    """A multi-launch plan that never ran a split call: the allocating entry
    point is refused on a capturing stream, the allocation-free one records
    and replays."""
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import Capture

    log_n, batch = 16, 3
    n = batch << log_n
    x = normal_c64(np.random.default_rng(6), n)
    eager_plan = _plan(gpu_device, 1, log_n, batch)
    ins, outs = _parts(gpu_device, x)
    N.check(_call(N.lib.fg_fft_exec_split_noalloc, eager_plan, ins, outs, "inverse", True))
    eager = _read(gpu_device, outs, n)
    assert rel_l2(eager, oracle.fft_1d(x, log_n, "inverse", True)) <= TOL

    plan = _plan(gpu_device, 1, log_n, batch)
    outs3 = _parts(gpu_device, x)[1]
    with Capture(gpu_device, keep=[plan]) as cap:
        rc = _call(N.lib.fg_fft_exec_split, plan, ins, outs3, "inverse", True, cap.stream)
        assert rc == N.FG_ERR_INVALID_ARGUMENT and "capture" in N.last_error()
        N.check(_call(N.lib.fg_fft_exec_split_noalloc, plan, ins, outs3, "inverse", True, cap.stream))
    graph = cap.graph
    assert graph.node_count == plan.describe()["launches"] + 2
    for replay in range(3):
        outs3[0].copy_from_host(np.zeros(n, np.float32))
        outs3[1].copy_from_host(np.zeros(n, np.float32))
        gpu_device.sync()
        graph.launch()
        got = _read(gpu_device, outs3, n)
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {replay}"
    graph.destroy()
    plan.destroy()
    eager_plan.destroy()


def test_noalloc_two_stream_plan(gpu_device):
    # a multi-pass plan with two chunks in flight (chunk limit lowered to
    # 16 MiB: 8 MiB chunks, describe()["streams"] == 2) staged through the
    # scratch area: its odd chunks run on the device's chunk stream, the
    # join brings them back before the deinterleave
    import ferrum_gpu
    from ferrum_gpu import _native as N

    saved = ferrum_gpu.fft.get_chunk_bytes()
    ferrum_gpu.fft.set_chunk_bytes(16 << 20)
    try:
        log_n, batch = 20, 8
        plan = _plan(gpu_device, 1, log_n, batch)
    finally:
        ferrum_gpu.fft.set_chunk_bytes(saved)
    d = plan.describe()
    print(f"[case] noalloc two-stream plan {d}", flush=True)
    assert d["streams"] == 2 and d["chunks"] == 8
    n = batch << log_n
    x = normal_c64(np.random.default_rng(8), n)
    ins, outs = _parts(gpu_device, x)
    for direction, normalize in (("forward", False), ("inverse", True)):
        N.check(_call(N.lib.fg_fft_exec_split_noalloc, plan, ins, outs, direction, normalize))
        got = _read(gpu_device, outs, n)
        outs2 = _parts(gpu_device, x)[1]
        N.check(_call(N.lib.fg_fft_exec_split, plan, ins, outs2, direction, normalize))
        assert np.array_equal(got.view(np.uint32), _read(gpu_device, outs2, n).view(np.uint32))
        assert rel_l2(got, oracle.fft_1d(x, log_n, direction, normalize, threads=8)) <= TOL
    plan.destroy()


def test_noalloc_calls_on_two_streams_take_turns(gpu_device):
    # two staging calls made back to back on two streams, no host
    # synchronisation between them: the second waits on its stream for the
    # first's last launch, so neither overwrites the other's staged data
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import Stream

    shapes = [(1, 20, 8), (1, 17, 16)]
    plans, data = [], []
    for i, (dims, log_n, batch) in enumerate(shapes):
        n = batch << log_n
        x = normal_c64(np.random.default_rng(60 + i), n)
        plans.append(_plan(gpu_device, dims, log_n, batch))
        data.append((x, n, log_n) + _parts(gpu_device, x))
    streams = [Stream(gpu_device), Stream(gpu_device)]
    print("[case] noalloc calls on two streams", flush=True)
    for rep in range(3):
        for (x, n, log_n, ins, outs), plan, s in zip(data, plans, streams):
            N.check(_call(N.lib.fg_fft_exec_split_noalloc, plan, ins, outs, "forward", False, s.handle))
        for s in streams:
            s.sync()
        for (x, n, log_n, ins, outs), plan in zip(data, plans):
            got = _read(gpu_device, outs, n)
            ref2 = _parts(gpu_device, x)[1]
            N.check(_call(N.lib.fg_fft_exec_split, plan, ins, ref2, "forward", False))
            assert np.array_equal(got.view(np.uint32), _read(gpu_device, ref2, n).view(np.uint32)), rep
    for s in streams:
        s.destroy()
    for p in plans:
        p.destroy()

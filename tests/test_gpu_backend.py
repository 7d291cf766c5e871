"""GPU checks of the substrate: the Backend contract over HIP.

Re-creates the reference's substrate smoke path (hand-written vector_add
loaded and launched through `Backend`, examples/vector-add/src/main.rs:62-135,
crates/ferrum-gpu-cuda/tests/load_launch.rs:68-138) plus the error variants of
crates/ferrum-gpu-cuda/src/error.rs:9-34.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_device_info(gpu_device):
    info = gpu_device.info()
    assert info["arch"] == "gfx950"
    assert info["cu_count"] >= 64


def test_alloc_zeros_and_round_trip(gpu_device):
    from ferrum_gpu.hip import DeviceBuffer

    buf = DeviceBuffer(gpu_device, 4096)
    out = np.ones(1024, np.float32)
    buf.copy_to_host(out)
    assert not out.any()                      # alloc_zeros
    src = np.arange(1024, dtype=np.float32)
    buf.copy_from_host(src)
    buf.copy_to_host(out)
    assert np.array_equal(out, src)
    buf.free()


def test_vector_add_through_backend(gpu_device):
    from ferrum_gpu.hip import DeviceBuffer, Module

    n = 100_003
    a = np.random.default_rng(0).random(n, dtype=np.float32)
    b = np.random.default_rng(1).random(n, dtype=np.float32)
    da, db, dc = (DeviceBuffer(gpu_device, 4 * n) for _ in range(3))
    da.copy_from_host(a)
    db.copy_from_host(b)
    k = Module(gpu_device).kernel("fg_vector_add")
    k.launch(((n + 255) // 256,), (256,),
             [ctypes.c_void_p(da.ptr), ctypes.c_void_p(db.ptr), ctypes.c_void_p(dc.ptr), ctypes.c_uint32(n)])
    gpu_device.sync()
    c = np.empty(n, np.float32)
    dc.copy_to_host(c)
    assert np.array_equal(c, a + b)


def test_backend_errors(gpu_device):
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import Module

    with pytest.raises(N.FerrumGpuError) as e:
        Module(gpu_device, image=b"\x7fELF-not-really", backend_id=N.FG_BACKEND_CUDA)
    assert e.value.code == N.FG_ERR_BACKEND_MISMATCH
    with pytest.raises(N.FerrumGpuError) as e:
        Module(gpu_device).kernel("no_such_kernel")
    assert e.value.code == N.FG_ERR_KERNEL_NOT_FOUND


def test_events_and_stream_copy(gpu_device):
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import DeviceBuffer, Event

    nbytes = 64 << 20
    src = np.random.default_rng(2).random(nbytes // 4, dtype=np.float32)
    a, b = DeviceBuffer(gpu_device, nbytes), DeviceBuffer(gpu_device, nbytes)
    a.copy_from_host(src)
    s = gpu_device.default_stream
    e0, e1 = Event(gpu_device), Event(gpu_device)
    e0.record(s)
    N.check(N.lib.fg_stream_copy(gpu_device.handle, ctypes.c_void_p(a.ptr), ctypes.c_void_p(b.ptr), nbytes,
                                 ctypes.c_void_p(s)))
    e1.record(s)
    e1.synchronize()
    assert e0.elapsed_ms(e1) > 0
    out = np.empty_like(src)
    b.copy_to_host(out)
    assert np.array_equal(out, src)
    # the copy kernel moves 16-byte vectors: misaligned pointers and odd sizes
    # are refused on the host, nothing is launched
    for p_in, p_out, n in ((a.ptr + 8, b.ptr, 1 << 20), (a.ptr, b.ptr + 4, 1 << 20), (a.ptr, b.ptr, 24)):
        rc = N.lib.fg_stream_copy(gpu_device.handle, ctypes.c_void_p(p_in), ctypes.c_void_p(p_out), n,
                                  ctypes.c_void_p(s))
        assert rc == N.FG_ERR_INVALID_ARGUMENT, (p_in - a.ptr, p_out - b.ptr, n)
        assert "16" in N.last_error()


def test_device_close_waits_for_its_plans_and_graphs(gpu_device):
    # A device cannot be closed while plans or captured graphs made on it
    # live (they refer to it); after they are destroyed it closes.
    import ferrum_gpu
    from ferrum_gpu._native import FerrumGpuError
    from ferrum_gpu.hip import Capture, Device, DeviceBuffer

    dev = Device(0)
    plan = ferrum_gpu.fft.Plan1D(8, 4, dev)
    buf = DeviceBuffer(dev, plan.nbytes)
    with Capture(dev) as cap:
        plan.execute(buf, buf, "forward", stream=cap.stream)
    graph = cap.graph
    with pytest.raises(FerrumGpuError, match="plan\\(s\\) or graph\\(s\\)"):
        dev.close()
    plan.destroy()
    with pytest.raises(FerrumGpuError):
        dev.close()          # the captured graph still refers to the device
    graph.destroy()
    buf.free()
    dev.close()


def test_c_program_over_the_c_abi(gpu_device, capfd):
    # examples/fft_c_abi.c drives the library from plain C (device, host and
    # device-resident FFTs, the generator, plans, copies) and checks closed
    # forms; its library build runs the same code in this process.
    import os

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    lib = ctypes.CDLL(os.path.join(root, "ferrum-gpu_amd", "examples", "libfft_c_abi.so"))
    lib.fft_c_abi_example.restype = ctypes.c_int
    rc = lib.fft_c_abi_example()
    out = capfd.readouterr().out
    print(out)
    assert rc == 0 and out.strip().endswith("OK"), out

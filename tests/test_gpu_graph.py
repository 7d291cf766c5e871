"""HIP graphs of plan executions (fg_fft_graph_create / fg_graph_launch).

No reference counterpart: the reference submits every launch from the host
(crates/ferrum-gpu-py/src/lib.rs:142-233).  A graph replays exactly the
kernels of fg_fft_exec, so every replay must equal the eager result bit for
bit, and match the CPU oracle within the 1e-4 relative-L2 gate.  Each replay
is separated from the next by eager work and synchronisations of the
program's own, and each is checked.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import normal_c64, rel_l2, uniform_c64

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint32)


CASES = [
    # (dims, log_n, batch, direction, normalize): single-pass, multi-pass 1D, 2D
    (1, 10, 64, "forward", False),
    (1, 8, 256, "inverse", True),
    (1, 16, 4, "inverse", True),
    (1, 22, 1, "forward", False),
    (2, 11, 1, "forward", False),
    (2, 12, 1, "inverse", True),
]


@pytest.mark.parametrize("dims,log_n,batch,direction,normalize", CASES)
def test_graph_replays_equal_eager(gpu_device, dims, log_n, batch, direction, normalize):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    elems = 1 << (log_n * dims)
    print(f"[case] graph dims={dims} log_n={log_n} batch={batch} {direction}", flush=True)
    x = uniform_c64(np.random.default_rng(log_n * 10 + dims), batch * elems)
    plan = (ferrum_gpu.fft.Plan1D if dims == 1 else ferrum_gpu.fft.Plan2D)(log_n, batch, gpu_device)
    d_in, d_out, d_eager, d_other = (DeviceBuffer(gpu_device, x.nbytes) for _ in range(4))
    d_in.copy_from_host(x)
    d_other.copy_from_host(x)
    plan.execute(d_in, d_eager, direction, normalize)
    gpu_device.sync()
    eager = d_eager.copy_to_host(np.empty_like(x))
    if dims == 1:
        ref = oracle.fft_1d(x, log_n, direction, normalize)
    else:
        ref = oracle.fft_2d(x, log_n, direction, normalize)
    assert rel_l2(eager, ref) <= TOL

    graph = plan.capture_graph(d_in, d_out, direction, normalize)
    assert graph.node_count == len(plan.kernel_names())
    zeros = np.zeros_like(x)
    for replay in range(3):
        d_out.copy_from_host(zeros)                         # eager copy between replays
        plan.execute(d_other, d_other, direction, normalize)  # eager kernels on another buffer
        gpu_device.sync()
        graph.launch()
        gpu_device.sync()
        got = d_out.copy_to_host(np.empty_like(x))
        assert np.array_equal(_bits(got), _bits(eager)), f"replay {replay} differs from the eager result"
    graph.destroy()
    plan.destroy()


def test_graph_reps_in_place_on_a_stream(gpu_device):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer, Stream

    log_n, batch, reps = 10, 32, 3
    x = normal_c64(np.random.default_rng(5), batch << log_n)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    d = DeviceBuffer(gpu_device, x.nbytes)
    d.copy_from_host(x)
    for _ in range(reps):
        plan.execute(d, d)
    gpu_device.sync()
    eager = d.copy_to_host(np.empty_like(x))
    ref = x
    for _ in range(reps):
        ref = oracle.fft_1d(ref, log_n)
    assert rel_l2(eager, ref) <= TOL

    stream = Stream(gpu_device)
    graph = plan.capture_graph(d, d, reps=reps)
    assert graph.node_count == reps
    for replay in range(2):
        d.copy_from_host(x)
        graph.launch(stream.handle)
        stream.sync()
        got = d.copy_to_host(np.empty_like(x))
        assert np.array_equal(_bits(got), _bits(eager)), f"replay {replay}"
    graph.destroy()
    stream.destroy()


def test_graph_argument_errors_and_plan_lifetime(gpu_device):
    import ferrum_gpu
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import DeviceBuffer

    plan = ferrum_gpu.fft.Plan1D(16, 2, gpu_device)  # two launches per execution
    d = DeviceBuffer(gpu_device, (2 << 16) * 8)
    for bad in (0, -1, 32769):
        with pytest.raises(N.FerrumGpuError) as e:
            plan.capture_graph(d, d, reps=bad)
        assert e.value.code == N.FG_ERR_INVALID_ARGUMENT
    with pytest.raises(ValueError):
        plan.capture_graph(d, d, direction="sideways")
    g = plan.capture_graph(d, d, reps=2)
    assert g.node_count == 4
    with pytest.raises(N.FerrumGpuError) as e:
        plan.destroy()                      # a graph still replays this plan
    assert e.value.code == N.FG_ERR_INVALID_ARGUMENT and "graph" in str(e.value)
    g.destroy()
    plan.destroy()


def test_general_capture_of_a_forward_inverse_step(gpu_device):
    """Config 2's step (forward, then normalised inverse) plus an elementwise
    product, recorded with Capture and replayed."""
    import ferrum_gpu
    from ferrum_gpu.hip import Capture, DeviceBuffer

    log_n, batch = 8, 256
    n = batch << log_n
    rng = np.random.default_rng(2)
    x, w = uniform_c64(rng, n), uniform_c64(rng, n)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    b0, b1, b2, bw, b3 = (DeviceBuffer(gpu_device, x.nbytes) for _ in range(5))
    b0.copy_from_host(x)
    bw.copy_from_host(w)

    def step(stream):
        plan.execute(b0, b1, "forward", stream=stream)
        plan.execute(b1, b2, "inverse", True, stream=stream)
        ferrum_gpu.pointwise.cmul(gpu_device, b2, bw, b3, n, stream=stream)

    step(0)
    gpu_device.sync()
    eager = b3.copy_to_host(np.empty_like(x))
    fwd = oracle.fft_1d(x, log_n)
    inv = oracle.fft_1d(fwd, log_n, "inverse", True)
    assert rel_l2(eager, oracle.cmul_interleaved(inv, w)) <= TOL

    with Capture(gpu_device, keep=[plan]) as cap:
        step(cap.stream)
    graph = cap.graph
    assert graph.node_count == 3
    for replay in range(3):
        b3.copy_from_host(np.zeros_like(x))
        plan.execute(b3, b3)          # eager work between replays
        gpu_device.sync()
        graph.launch()
        gpu_device.sync()
        got = b3.copy_to_host(np.empty_like(x))
        assert np.array_equal(_bits(got), _bits(eager)), f"replay {replay}"
    graph.destroy()


def test_capture_block_error_ends_capture(gpu_device):
    import ferrum_gpu
    from ferrum_gpu.hip import Capture, DeviceBuffer

    plan = ferrum_gpu.fft.Plan1D(10, 4, gpu_device)
    d = DeviceBuffer(gpu_device, (4 << 10) * 8)
    with pytest.raises(RuntimeError, match="planted"):
        with Capture(gpu_device) as cap:
            plan.execute(d, d, stream=cap.stream)
            raise RuntimeError("planted")
    assert cap.graph is None
    # the device and the thread are out of capture mode: eager work runs
    x = uniform_c64(np.random.default_rng(9), 4 << 10)
    d.copy_from_host(x)
    plan.execute(d, d)
    gpu_device.sync()
    assert rel_l2(d.copy_to_host(np.empty_like(x)), oracle.fft_1d(x, 10)) <= TOL

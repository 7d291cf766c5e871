"""Single-pass plans too small to fill the GPU run the latency geometry
(fg_fft_n<L>_lat: one transform per workgroup, fewer elements per thread);
larger batches run the throughput geometry.  Both must match the oracle, and
a latency plan's split-layout execution (its _split twin) must give the
interleaved result bit for bit."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import normal_c64, rel_l2, uniform_c64
from test_stockham_model import LATENCY_GEOM

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _exec(dev, plan, x, direction="forward", normalize=False):
    from ferrum_gpu.hip import DeviceBuffer

    a, b = DeviceBuffer(dev, plan.nbytes), DeviceBuffer(dev, plan.nbytes)
    a.copy_from_host(x)
    plan.execute(a, b, direction, normalize)
    dev.sync()
    out = np.empty_like(x)
    b.copy_to_host(out)
    return out


@pytest.mark.parametrize("log_n", sorted(LATENCY_GEOM))
def test_small_batches_pick_the_latency_kernel(gpu_device, log_n):
    import ferrum_gpu

    cus = gpu_device.info()["cu_count"]
    small = ferrum_gpu.fft.Plan1D(log_n, 256, gpu_device)
    assert small.kernel_names() == [f"fg_fft_n{log_n}_lat"]
    # enough transforms for two throughput workgroups per CU
    big = ferrum_gpu.fft.Plan1D(log_n, 2 * cus * 64, gpu_device)
    assert big.kernel_names() == [f"fg_fft_n{log_n}"]
    rng = np.random.default_rng(600 + log_n)
    for plan, batch in ((small, 256), (big, 2 * cus * 64)):
        x = uniform_c64(rng, batch << log_n)
        print(f"[case] log_n={log_n} batch={batch} kernel={plan.kernel_names()[0]}", flush=True)
        assert rel_l2(_exec(gpu_device, plan, x), oracle.fft_1d(x, log_n, threads=8)) <= TOL
        plan.destroy()


@pytest.mark.parametrize("log_n", sorted(LATENCY_GEOM))
@pytest.mark.parametrize("batch", [1, 3, 100])
@pytest.mark.parametrize("normalize", [False, True])
def test_latency_kernel_inverse(gpu_device, log_n, batch, normalize):
    import ferrum_gpu

    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    assert plan.kernel_names()[0].endswith("_lat")
    rng = np.random.default_rng(700 + log_n + batch)
    x = normal_c64(rng, batch << log_n)
    got = _exec(gpu_device, plan, x, "inverse", normalize)
    assert rel_l2(got, oracle.fft_1d(x, log_n, "inverse", normalize)) <= TOL
    plan.destroy()


@pytest.mark.parametrize("log_n", sorted(LATENCY_GEOM))
def test_latency_plan_split_layout(gpu_device, log_n):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    batch = 37
    n = batch << log_n
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    assert plan.kernel_names()[0].endswith("_lat")
    rng = np.random.default_rng(800 + log_n)
    x = uniform_c64(rng, n)
    parts = [DeviceBuffer(gpu_device, 4 * n) for _ in range(4)]
    parts[0].copy_from_host(np.ascontiguousarray(x.real))
    parts[1].copy_from_host(np.ascontiguousarray(x.imag))
    plan.execute_split(parts[0], parts[1], parts[2], parts[3], "inverse", True)
    gpu_device.sync()
    re, im = np.empty(n, np.float32), np.empty(n, np.float32)
    parts[2].copy_to_host(re)
    parts[3].copy_to_host(im)
    assert rel_l2(re + 1j * im, oracle.fft_1d(x, log_n, "inverse", True)) <= TOL
    inter = _exec(gpu_device, plan, x, "inverse", True)
    assert np.array_equal(inter.real, re) and np.array_equal(inter.imag, im)
    plan.destroy()

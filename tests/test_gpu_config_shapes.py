"""GPU parity at the shapes the benchmark measures, on the benchmark's own data.

* The single-pass throughput kernels with a partly filled last workgroup:
  fg_fft_n10 holds two transforms per workgroup and fg_fft_n8 four, and they
  only run when the batch fills at least two workgroups per CU (smaller
  batches take the _lat kernels), so batches 1025 and 2051 are the smallest
  ragged cases that reach them.  Every byte past the batch must stay
  untouched.
* An fp64 direct-DFT spot check (crates/ferrum-gpu-fft/src/layout_study.rs:5-21)
  at each BASELINE configuration's own shape and kernel, on the inputs the
  benchmark generates (the library's seeded generator, seed = configuration
  index), with the sampled lanes including the first and the last transform.

Bar: relative L2 <= 1e-4 against the CPU oracle (the reference's Stockham
path) and against the fp64 bins.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4
GUARD = 1 << 16  # bytes after the output that no launch may write
SENTINEL = np.complex64(complex(1234.5, -6789.25))


def _seeded(dev, n, seed, dist):
    """n complex64 values from the library's generator (what bench.py measures)."""
    from ferrum_gpu import synthetic
    from ferrum_gpu.hip import DeviceBuffer

    buf = DeviceBuffer(dev, 8 * n)
    (synthetic.normal if dist == "normal" else synthetic.uniform)(dev, buf, n, seed)
    dev.sync()
    x = np.empty(n, np.complex64)
    buf.copy_to_host(x)
    buf.free()
    return x


def _exec_guarded(dev, plan, x, direction, normalize, in_place):
    """plan.execute on x with GUARD sentinel bytes after the output buffer;
    returns (output, guard contents)."""
    from ferrum_gpu.hip import DeviceBuffer

    n = x.size
    a = DeviceBuffer(dev, plan.nbytes + GUARD)
    host = np.full((plan.nbytes + GUARD) // 8, SENTINEL, np.complex64)
    host[:n] = x
    a.copy_from_host(host)
    if in_place:
        b = a
    else:
        b = DeviceBuffer(dev, plan.nbytes + GUARD)
        b.copy_from_host(np.full((plan.nbytes + GUARD) // 8, SENTINEL, np.complex64))
    plan.execute(a, b, direction, normalize)
    dev.sync()
    out = np.empty((plan.nbytes + GUARD) // 8, np.complex64)
    b.copy_to_host(out)
    return out[:n], out[n:]


@pytest.mark.parametrize("log_n,batch,kernel", [(10, 1025, "fg_fft_n10"), (8, 2051, "fg_fft_n8"),
                                                (10, 4097, "fg_fft_n10"), (8, 8193, "fg_fft_n8")])
@pytest.mark.parametrize("direction,normalize", [("forward", False), ("inverse", True)])
@pytest.mark.parametrize("in_place", [False, True])
def test_throughput_kernel_ragged_last_workgroup(gpu_device, log_n, batch, kernel, direction, normalize, in_place):
    import ferrum_gpu

    print(f"[case] ragged {kernel} batch={batch} {direction} in_place={in_place}", flush=True)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    assert plan.kernel_names() == [kernel]  # the throughput kernel, not the latency one
    x = _seeded(gpu_device, batch << log_n, 100 + log_n, "uniform")
    got, guard = _exec_guarded(gpu_device, plan, x, direction, normalize, in_place)
    assert np.all(guard == SENTINEL), "a launch wrote past the last transform"
    ref = oracle.fft_1d(x, log_n, direction, normalize, threads=8)
    assert rel_l2(got, ref) <= TOL
    # the transforms of the partly filled last workgroup, on their own
    n = 1 << log_n
    tail = slice((batch - 3) * n, batch * n)
    assert rel_l2(got[tail], ref[tail]) <= TOL
    plan.destroy()


@pytest.mark.parametrize("log_n,batch,kernel", [(10, 1025, "fg_fft_n10_split"), (8, 2051, "fg_fft_n8_split")])
def test_split_twin_ragged_last_workgroup(gpu_device, log_n, batch, kernel):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    print(f"[case] ragged {kernel} batch={batch}", flush=True)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    assert plan.kernel_names() == [kernel[:-len("_split")]]
    n = batch << log_n
    x = _seeded(gpu_device, n, 200 + log_n, "normal")
    half = plan.nbytes // 2
    parts = []
    for host in (np.ascontiguousarray(x.real), np.ascontiguousarray(x.imag)):
        b = DeviceBuffer(gpu_device, half + GUARD)
        b.copy_from_host(np.concatenate([host, np.full(GUARD // 4, 7.5, np.float32)]))
        parts.append(b)
    outs = []
    for _ in range(2):
        b = DeviceBuffer(gpu_device, half + GUARD)
        b.copy_from_host(np.full((half + GUARD) // 4, 7.5, np.float32))
        outs.append(b)
    plan.execute_split(parts[0], parts[1], outs[0], outs[1], "inverse", True)
    gpu_device.sync()
    res = []
    for b in outs:
        h = np.empty((half + GUARD) // 4, np.float32)
        b.copy_to_host(h)
        assert np.all(h[n:] == 7.5), "a launch wrote past the last transform"
        res.append(h[:n])
    got = res[0] + 1j * res[1]
    # bit for bit what the interleaved kernel gives
    inter, _ = _exec_guarded(gpu_device, plan, x, "inverse", True, False)
    assert np.array_equal(got.astype(np.complex64), inter)
    assert rel_l2(got, oracle.fft_1d(x, log_n, "inverse", True, threads=8)) <= TOL
    plan.destroy()


# (name, log_n, batch, seed, distribution, expected kernel)
CONFIGS_1D = [
    ("cfg1", 10, 256, 1, "uniform", "fg_fft_n10_lat"),
    ("cfg2_256", 8, 256, 2, "uniform", "fg_fft_n8_lat"),
    ("cfg2_4096", 12, 256, 2, "uniform", "fg_fft_n12_lat"),
    ("cfg3", 10, 65536, 3, "normal", "fg_fft_n10"),
]


@pytest.mark.parametrize("name,log_n,batch,seed,dist,kernel", CONFIGS_1D)
def test_fp64_spot_check_at_config_shape(gpu_device, name, log_n, batch, seed, dist, kernel):
    import ferrum_gpu

    print(f"[case] fp64 spot check {name} ({kernel})", flush=True)
    n = 1 << log_n
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    assert plan.kernel_names() == [kernel]
    x = _seeded(gpu_device, batch * n, seed, dist)
    fwd, _ = _exec_guarded(gpu_device, plan, x, "forward", False, False)
    assert rel_l2(fwd, oracle.fft_1d(x, log_n, threads=8)) <= TOL
    rng = np.random.default_rng(seed)
    lanes = sorted({0, 1, batch // 2, batch - 2, batch - 1} | set(rng.integers(0, batch, 6).tolist()))
    bins = np.unique(np.concatenate([[0, 1, n // 2, n - 1], rng.integers(0, n, 60)]))
    fwd2 = fwd.reshape(batch, n)
    for lane in lanes:
        exact = oracle.dft_bins_f64(x[lane * n:(lane + 1) * n], bins)
        assert rel_l2(fwd2[lane, bins], exact) <= TOL, f"lane {lane}"
    if name.startswith("cfg2"):
        # config 2 is forward + normalised inverse: the inverse's bins are
        # (1/N) sum_k X_k W^{-nk}, the fp64 DFT with the opposite sign
        inv, _ = _exec_guarded(gpu_device, plan, fwd, "inverse", True, False)
        assert rel_l2(inv, oracle.fft_1d(fwd, log_n, "inverse", True)) <= TOL
        assert rel_l2(inv, x) <= TOL
        inv2 = inv.reshape(batch, n)
        for lane in lanes:
            exact = oracle.dft_bins_f64(fwd[lane * n:(lane + 1) * n], bins, sign=+1) / n
            assert rel_l2(inv2[lane, bins], exact) <= TOL, f"inverse lane {lane}"
    plan.destroy()

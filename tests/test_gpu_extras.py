"""GPU checks beyond the reference's square API: rectangular 2D, the tiled
transpose, in-place multi-pass plans, and concurrent host-path calls.

Rectangular 2D has no reference counterpart (Plan2D is square,
crates/ferrum-gpu-fft/src/plan.rs:98-135); its oracle is the reference's own
1D Stockham (oracle.fft_1d) applied along rows and then along columns, the
separable construction cpu_2d.rs:9-64 uses, plus numpy.fft.fft2.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest

import oracle
from conftest import normal_c64, rel_l2, uniform_c64

pytestmark = pytest.mark.gpu

TOL = 1e-4


def oracle_2d_rect(x, lr, lc, direction="forward", normalize=False):
    b = x.reshape(-1, 1 << lr, 1 << lc)
    rows = oracle.fft_1d(b.reshape(-1), lc, direction).reshape(b.shape)
    cols = oracle.fft_1d(np.ascontiguousarray(rows.transpose(0, 2, 1)).reshape(-1), lr, direction)
    out = np.ascontiguousarray(cols.reshape(b.shape[0], 1 << lc, 1 << lr).transpose(0, 2, 1))
    if direction == "inverse" and normalize:
        out = out * np.float32(1.0 / ((1 << lr) * (1 << lc)))
    return out.reshape(x.shape)


@pytest.mark.parametrize("lr,lc", [(4, 12), (12, 4), (5, 9), (9, 5), (11, 6), (6, 11), (10, 12), (12, 10)])
def test_rect_2d_forward(gpu_device, lr, lc):
    import ferrum_gpu

    rng = np.random.default_rng(lr * 100 + lc)
    batch = 2
    x = uniform_c64(rng, batch << (lr + lc)).reshape(batch, 1 << lr, 1 << lc)
    print(f"[case] rect 2d {1 << lr}x{1 << lc}", flush=True)
    got = ferrum_gpu.fft.fft2_c2c_pow2(x, device=gpu_device)
    assert got.shape == x.shape
    assert rel_l2(got, oracle_2d_rect(x, lr, lc)) <= TOL
    assert rel_l2(got, np.fft.fft2(x.astype(np.complex128))) <= TOL


@pytest.mark.parametrize("lr,lc", [(4, 8), (12, 5)])
def test_rect_2d_inverse_roundtrip(gpu_device, lr, lc):
    import ferrum_gpu

    rng = np.random.default_rng(lr + 7 * lc)
    x = normal_c64(rng, 1 << (lr + lc)).reshape(1 << lr, 1 << lc)
    inv = ferrum_gpu.fft.fft2_c2c_pow2(x, "inverse", True, device=gpu_device)
    assert rel_l2(inv, oracle_2d_rect(x, lr, lc, "inverse", True)) <= TOL
    back = ferrum_gpu.fft.fft2_c2c_pow2(inv, device=gpu_device)
    assert rel_l2(back, x) <= TOL


SMALL_2D = [(lr, lc) for lr in range(4, 11) for lc in range(4, 11) if lr + lc <= 14]


@pytest.mark.parametrize("lr,lc", SMALL_2D)
def test_one_pass_small_2d_every_shape(gpu_device, lr, lc):
    """The one-kernel plans (images of up to 16384 points): forward and
    normalised inverse, a batch that leaves the last workgroup partly empty,
    out of place and in place."""
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    n = 1 << (lr + lc)
    per_group = max(1, 256 * (16 if lr + lc >= 14 else 8) // n)   # images per workgroup
    batch = 2 * per_group + 1
    rng = np.random.default_rng(900 + 16 * lr + lc)
    x = uniform_c64(rng, batch * n).reshape(batch, 1 << lr, 1 << lc)
    print(f"[case] one-pass 2d {1 << lr}x{1 << lc} batch={batch}", flush=True)
    plan = ferrum_gpu.fft.Plan2D(lr, batch, gpu_device, log_cols=lc)
    assert plan.kernel_names() == [f"fg_fft2d_l{lr}_{lc}"]
    a, b = DeviceBuffer(gpu_device, plan.nbytes), DeviceBuffer(gpu_device, plan.nbytes)
    a.copy_from_host(x)
    plan.execute(a, b, "forward")
    gpu_device.sync()
    fwd = np.empty_like(x)
    b.copy_to_host(fwd)
    assert rel_l2(fwd, oracle_2d_rect(x, lr, lc)) <= TOL
    assert rel_l2(fwd, np.fft.fft2(x.astype(np.complex128))) <= TOL
    plan.execute(b, b, "inverse", True)       # in place
    gpu_device.sync()
    inv = np.empty_like(x)
    b.copy_to_host(inv)
    assert rel_l2(inv, oracle_2d_rect(fwd, lr, lc, "inverse", True)) <= TOL
    assert rel_l2(inv, x) <= TOL
    plan.destroy()


def test_square_api_equals_rect_api(gpu_device):
    import ferrum_gpu

    x = uniform_c64(np.random.default_rng(3), 256 * 256).reshape(256, 256)
    a = ferrum_gpu.fft.fft_2d_c2c_pow2(x, 8, device=gpu_device)
    b = ferrum_gpu.fft.fft2_c2c_pow2(x, device=gpu_device)
    assert np.array_equal(a, b)


# 64 x 64 tiles below 128 rows or columns; 128 x 128 tiles in super-tiles of
# up to 8 x 8 above (full and partial super-tiles, ragged edge tiles, batches)
@pytest.mark.parametrize("rows,cols,batch", [(64, 64, 1), (4096, 4096, 1), (1000, 37, 3), (1, 5000, 2),
                                             (513, 1, 1), (128, 4096, 2), (1100, 1300, 2), (129, 200, 3),
                                             (8192, 136, 1), (300, 8192, 1), (127, 4096, 1)])
def test_transpose_exact(gpu_device, rows, cols, batch):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    x = uniform_c64(np.random.default_rng(rows + cols), batch * rows * cols)
    a, b = DeviceBuffer(gpu_device, x.nbytes), DeviceBuffer(gpu_device, x.nbytes)
    a.copy_from_host(x)
    ferrum_gpu.fft.transpose(gpu_device, a, b, rows, cols, batch)
    gpu_device.sync()
    out = np.empty_like(x)
    b.copy_to_host(out)
    exp = x.reshape(batch, rows, cols).transpose(0, 2, 1).reshape(-1)
    assert np.array_equal(out, exp)


def test_transpose_rejects_alias(gpu_device):
    import ferrum_gpu
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import DeviceBuffer

    a = DeviceBuffer(gpu_device, 64 * 64 * 8)
    with pytest.raises(N.FerrumGpuError):
        ferrum_gpu.fft.transpose(gpu_device, a, a, 64, 64)


@pytest.mark.parametrize("log_n", [10, 14, 22])
def test_in_place_execution_matches_out_of_place(gpu_device, log_n):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    batch = max(1, (1 << 20) >> log_n)
    x = uniform_c64(np.random.default_rng(log_n), batch << log_n)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    a, b = DeviceBuffer(gpu_device, x.nbytes), DeviceBuffer(gpu_device, x.nbytes)
    a.copy_from_host(x)
    plan.execute(a, b)
    plan.execute(a, a)          # in place
    gpu_device.sync()
    oa, ob = np.empty_like(x), np.empty_like(x)
    a.copy_to_host(oa)
    b.copy_to_host(ob)
    assert np.array_equal(oa, ob)
    assert rel_l2(oa, oracle.fft_1d(x, log_n, threads=8)) <= TOL


def test_concurrent_host_calls(gpu_device):
    # The host path releases the GIL (ctypes) and serialises on the device's
    # lock; results from concurrent threads must equal sequential ones.
    import ferrum_gpu

    rng = np.random.default_rng(12)
    jobs = [(uniform_c64(rng, 8 << l), l) for l in (6, 9, 10, 12, 14, 10, 9, 6)]
    expected = [ferrum_gpu.fft.fft_1d_c2c_pow2(x, l, device=gpu_device) for x, l in jobs]
    results = [None] * len(jobs)
    errors = []

    def work(i):
        try:
            x, l = jobs[i]
            for _ in range(3):
                results[i] = ferrum_gpu.fft.fft_1d_c2c_pow2(x, l, device=gpu_device)
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    ts = [threading.Thread(target=work, args=(i,)) for i in range(len(jobs))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
    for r, e in zip(results, expected):
        assert np.array_equal(r, e)


def test_device_streams_are_independent(gpu_device):
    # A plan executed on a caller-created stream orders correctly with a sync
    # of that stream only.
    import ctypes

    import ferrum_gpu
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import DeviceBuffer

    s = ctypes.c_void_p()
    N.check(N.lib.fg_stream_create(gpu_device.handle, ctypes.byref(s)))
    try:
        x = uniform_c64(np.random.default_rng(4), 64 * 1024)
        plan = ferrum_gpu.fft.Plan1D(10, 64, gpu_device)
        a, b = DeviceBuffer(gpu_device, x.nbytes), DeviceBuffer(gpu_device, x.nbytes)
        a.copy_from_host(x)
        plan.execute(a, b, stream=s.value)
        N.check(N.lib.fg_stream_sync(gpu_device.handle, s))
        out = np.empty_like(x)
        b.copy_to_host(out)
        assert rel_l2(out, oracle.fft_1d(x, 10)) <= TOL
    finally:
        N.check(N.lib.fg_stream_destroy(gpu_device.handle, s))


@pytest.mark.parametrize("kind,log_n,batch", [("1d", 12, 1000), ("1d", 14, 300), ("2d", 6, 3001), ("1d", 10, 8191),
                                              ("2d", 12, 2), ("2d", 11, 3)])
def test_host_path_matches_the_device_plan(gpu_device, kind, log_n, batch):
    """The host-array entry points (pinned pieces, parallel host copies) give
    the device-resident plan's out-of-place output bit for bit, forward and
    normalised inverse, for 1D single- and multi-pass lengths and 2D images
    -- including config 5's 4096 x 4096 images and 2048-row ones, whose
    in-place execution runs other kernels (the host path runs them out of
    place, so it takes the row pairs)."""
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    n = 1 << (2 * log_n if kind == "2d" else log_n)
    rng = np.random.default_rng(4000 + log_n)
    x = uniform_c64(rng, batch * n)
    print(f"[case] host path {kind} log_n={log_n} batch={batch}", flush=True)
    for direction, normalize in (("forward", False), ("inverse", True)):
        if kind == "2d":
            got = ferrum_gpu.fft.fft_2d_c2c_pow2(x.reshape(batch, 1 << log_n, 1 << log_n), log_n, direction,
                                                 normalize, device=gpu_device).reshape(-1)
            plan = ferrum_gpu.fft.Plan2D(log_n, batch, gpu_device)
        else:
            got = ferrum_gpu.fft.fft_1d_c2c_pow2(x, log_n, direction, normalize, device=gpu_device)
            plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
        a, b = DeviceBuffer(gpu_device, plan.nbytes), DeviceBuffer(gpu_device, plan.nbytes)
        a.copy_from_host(x)
        plan.execute(a, b, direction, normalize)
        gpu_device.sync()
        want = np.empty_like(x)
        b.copy_to_host(want)
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64))
        if plan.kernel_names(in_place=True) != plan.kernel_names():
            # the in-place form rounds differently, so bit-identity above
            # shows the host path ran the out-of-place kernels
            plan.execute(a, a, direction, normalize)
            gpu_device.sync()
            inplace = np.empty_like(x)
            a.copy_to_host(inplace)
            assert not np.array_equal(inplace.view(np.uint64), want.view(np.uint64))
            assert rel_l2(inplace, want) <= 1e-5
        a.free()
        b.free()
        plan.destroy()

"""GPU parity of the multi-pass paths: 1D lengths 2^13 .. 2^24 (one pass up to 2^14) and 2D images.

Bar: relative L2 <= 1e-4 against the CPU oracle (the reference's radix-2
Stockham, crates/ferrum-gpu-fft/src/cpu.rs and cpu_2d.rs) on identical seeded
inputs, plus fp64 direct-DFT spot checks; the reference's own 2D pytest matrix
(crates/ferrum-gpu-py/python/tests/test_fft_2d_vs_numpy.py) is re-created.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import normal_c64, rel_l2, uniform_c64

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _plan_run(dev, x, log_n, batch, direction="forward", normalize=False, two_d=False):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    plan = (ferrum_gpu.fft.Plan2D if two_d else ferrum_gpu.fft.Plan1D)(log_n, batch, dev)
    a, b = DeviceBuffer(dev, plan.nbytes), DeviceBuffer(dev, plan.nbytes)
    a.copy_from_host(x)
    plan.execute(a, b, direction, normalize)
    dev.sync()
    out = np.empty_like(x)
    b.copy_to_host(out)
    # the input buffer is left untouched
    back = np.empty_like(x)
    a.copy_to_host(back)
    assert np.array_equal(back, x)
    plan.destroy()
    return out


@pytest.mark.parametrize("log_n", list(range(13, 25)))
def test_1d_multipass_forward(gpu_device, log_n):
    batch = max(1, (1 << 21) >> log_n)
    rng = np.random.default_rng(300 + log_n)
    x = uniform_c64(rng, batch << log_n)
    print(f"[case] 1d log_n={log_n} batch={batch}", flush=True)
    got = _plan_run(gpu_device, x, log_n, batch)
    assert rel_l2(got, oracle.fft_1d(x, log_n, threads=8)) <= TOL


# every last-pass / middle-pass tile shape of the chunked plans (64..1024-point
# row passes, 8-column middle passes) runs the inverse's conjugations once
@pytest.mark.parametrize("log_n", [13, 14, 16, 17, 18, 19, 20, 21, 22, 23, 24])
@pytest.mark.parametrize("normalize", [False, True])
def test_1d_multipass_inverse(gpu_device, log_n, normalize):
    rng = np.random.default_rng(400 + log_n)
    x = normal_c64(rng, 1 << log_n)
    got = _plan_run(gpu_device, x, log_n, 1, "inverse", normalize)
    assert rel_l2(got, oracle.fft_1d(x, log_n, "inverse", normalize)) <= TOL


def test_1d_host_api_large(gpu_device):
    import ferrum_gpu

    rng = np.random.default_rng(7)
    x = uniform_c64(rng, 3 << 15)
    y = ferrum_gpu.fft.fft_1d_c2c_pow2(x, 15, device=gpu_device)
    assert rel_l2(y, oracle.fft_1d(x, 15)) <= TOL
    z = ferrum_gpu.fft.fft_1d_c2c_pow2(y, 15, direction="inverse", normalize=True, device=gpu_device)
    assert rel_l2(z, x) <= TOL


def test_config4_n2p24_b4(gpu_device):
    rng = np.random.default_rng(4)
    log_n, batch = 24, 4
    x = normal_c64(rng, batch << log_n)
    print("[case] config4 N=2^24 batch=4", flush=True)
    got = _plan_run(gpu_device, x, log_n, batch)
    ref = oracle.fft_1d(x, log_n, threads=4)
    assert rel_l2(got, ref) <= TOL
    n = 1 << log_n
    bins = [0, 1, 4097, 1 << 23, n - 1]
    exact = oracle.dft_bins_f64(x[:n], bins)
    assert rel_l2(got[:n][bins], exact) <= TOL


# ------------------------------------------------------------------------ 2D


@pytest.mark.parametrize("log_n", list(range(4, 13)))
def test_2d_forward(gpu_device, log_n):
    n = 1 << log_n
    batch = 3 if log_n <= 9 else 1
    rng = np.random.default_rng(500 + log_n)
    x = uniform_c64(rng, batch * n * n).reshape(batch, n, n)
    print(f"[case] 2d log_n={log_n} batch={batch}", flush=True)
    got = _plan_run(gpu_device, x, log_n, batch, two_d=True)
    assert rel_l2(got, oracle.fft_2d(x, log_n)) <= TOL


@pytest.mark.parametrize("log_n", [4, 7, 10, 11, 12])
@pytest.mark.parametrize("normalize", [False, True])
def test_2d_inverse(gpu_device, log_n, normalize):
    n = 1 << log_n
    rng = np.random.default_rng(600 + log_n)
    x = normal_c64(rng, n * n).reshape(1, n, n)
    got = _plan_run(gpu_device, x, log_n, 1, "inverse", normalize, two_d=True)
    assert rel_l2(got, oracle.fft_2d(x, log_n, "inverse", normalize)) <= TOL


def _input_2d(n):
    base = np.arange(n * n, dtype=np.float32).reshape(n, n)
    return (np.sin(base * np.float32(0.1)) + 1j * np.cos(base * np.float32(0.07))).astype(np.complex64)


@pytest.mark.parametrize("log_n", [4, 5, 6, 8, 10])
@pytest.mark.parametrize("use_device", [False, True])
def test_reference_2d_cases_match_numpy(gpu_device, log_n, use_device):
    # test_fft_2d_vs_numpy.py:19-41 (the reference gated at 1e-3)
    import ferrum_gpu

    n = 1 << log_n
    arr = _input_2d(n)
    exp = np.fft.fft2(arr.astype(np.complex128))
    out = ferrum_gpu.fft.fft_2d_c2c_pow2(arr, log_n, device=gpu_device if use_device else None)
    assert out.shape == arr.shape and out.dtype == np.complex64
    assert float(np.max(np.abs(out - exp))) / float(np.max(np.abs(exp))) < 1e-4
    assert rel_l2(out, oracle.fft_2d(arr, log_n)) <= TOL


@pytest.mark.parametrize("log_n", [4, 6, 8, 12])
def test_reference_2d_roundtrip(gpu_device, log_n):
    # test_fft_2d_vs_numpy.py:44-60
    import ferrum_gpu

    n = 1 << log_n
    arr = _input_2d(n)
    fwd = ferrum_gpu.fft.fft_2d_c2c_pow2(arr, log_n, direction="forward", device=gpu_device)
    inv = ferrum_gpu.fft.fft_2d_c2c_pow2(fwd, log_n, direction="inverse", normalize=True, device=gpu_device)
    assert float(np.max(np.abs(arr - inv))) / float(np.max(np.abs(arr))) < 1e-4


def test_2d_stack_host_api(gpu_device):
    import ferrum_gpu

    rng = np.random.default_rng(8)
    x = uniform_c64(rng, 4 * 64 * 64).reshape(4, 64, 64)
    y = ferrum_gpu.fft.fft_2d_c2c_pow2(x, 6, device=gpu_device)
    assert y.shape == x.shape
    assert rel_l2(y, oracle.fft_2d(x, 6)) <= TOL


def test_config5_4096sq_b2(gpu_device):
    rng = np.random.default_rng(5)
    log_n, batch = 12, 2
    n = 1 << log_n
    x = uniform_c64(rng, batch * n * n).reshape(batch, n, n)
    print("[case] config5 4096x4096 batch=2", flush=True)
    got = _plan_run(gpu_device, x, log_n, batch, two_d=True)
    ref = oracle.fft_2d(x, log_n)
    assert rel_l2(got, ref) <= TOL
    # separable fp64 DFT at sampled (k1, k2) of image 1
    idx = np.arange(n)
    img = x[1].astype(np.complex128)
    for k1, k2 in [(0, 0), (1, 4095), (2048, 7), (777, 3001)]:
        v = np.exp(-2j * np.pi * k1 * idx / n) @ img @ np.exp(-2j * np.pi * k2 * idx / n)
        assert abs(got[1, k1, k2] - v) <= 1e-4 * np.linalg.norm(img)


def test_host_path_plan_cache_eviction(gpu_device):
    # The host entry points keep the 8 most recently used plans per device:
    # more distinct batches than that evict and re-create plans, every result
    # stays correct (multi-pass plans, whose workspaces the bound protects).
    import ferrum_gpu

    rng = np.random.default_rng(77)
    log_n = 16
    batches = list(range(1, 12)) + [3, 1, 11]
    for batch in batches:
        x = uniform_c64(rng, batch << log_n)
        y = ferrum_gpu.fft.fft_1d_c2c_pow2(x, log_n, device=gpu_device)
        assert rel_l2(y, oracle.fft_1d(x, log_n)) <= TOL, batch

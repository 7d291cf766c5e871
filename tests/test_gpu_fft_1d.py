"""GPU parity of the batched 1D C2C FFT against the CPU oracle.

Bar (north star): relative L2 <= 1e-4 against the CPU Stockham reference on
identical seeded inputs, plus an fp64 direct-DFT spot check.  The reference's
own GPU gates are re-created alongside: the 8 CASES x {one-shot, persistent
device} of crates/ferrum-gpu-py/python/tests/test_fft_vs_numpy.py:37-63 and
the large-batch cases of :71-107.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import normal_c64, rel_l2, uniform_c64

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _fft(x, log_n, direction="forward", normalize=False, device=None):
    import ferrum_gpu

    return ferrum_gpu.fft.fft_1d_c2c_pow2(x, log_n, direction=direction, normalize=normalize, device=device)


@pytest.mark.parametrize("log_n", list(range(2, 16)))
@pytest.mark.parametrize("batch", [1, 7, 257])
def test_forward_matches_oracle(gpu_device, log_n, batch):
    rng = np.random.default_rng(1000 * log_n + batch)
    x = uniform_c64(rng, batch << log_n)
    print(f"[case] fwd log_n={log_n} batch={batch}", flush=True)
    got = _fft(x, log_n, device=gpu_device)
    assert got.dtype == np.complex64 and got.shape == x.shape
    assert rel_l2(got, oracle.fft_1d(x, log_n)) <= TOL


@pytest.mark.parametrize("log_n", list(range(2, 16)))
@pytest.mark.parametrize("normalize", [False, True])
def test_inverse_matches_oracle(gpu_device, log_n, normalize):
    rng = np.random.default_rng(77 + log_n)
    x = normal_c64(rng, 5 << log_n)
    print(f"[case] inv log_n={log_n} normalize={normalize}", flush=True)
    got = _fft(x, log_n, "inverse", normalize, device=gpu_device)
    assert rel_l2(got, oracle.fft_1d(x, log_n, "inverse", normalize)) <= TOL


@pytest.mark.parametrize("log_n", [2, 6, 10, 12])
def test_roundtrip(gpu_device, log_n):
    rng = np.random.default_rng(5 + log_n)
    x = uniform_c64(rng, 33 << log_n)
    y = _fft(_fft(x, log_n, device=gpu_device), log_n, "inverse", True, device=gpu_device)
    assert rel_l2(y, x) <= TOL


def test_fp64_direct_dft_spot_check(gpu_device):
    rng = np.random.default_rng(64)
    for log_n in (4, 8, 10, 12, 13, 14, 15):
        n = 1 << log_n
        x = normal_c64(rng, 6 * n)
        got = _fft(x, log_n, device=gpu_device).reshape(6, n)
        bins = rng.integers(0, n, 64)
        for lane in (0, 3, 5):
            exact = oracle.dft_bins_f64(x[lane * n:(lane + 1) * n], bins)
            assert rel_l2(got[lane, bins], exact) <= TOL


# ---- the reference's pytest matrix (test_fft_vs_numpy.py) -------------------

CASES = [
    (2, 1, "forward", False, "N=4 fwd"),
    (3, 1, "forward", False, "N=8 fwd"),
    (6, 1, "forward", False, "N=64 fwd"),
    (8, 1, "forward", False, "N=256 fwd"),
    (10, 1, "forward", False, "N=1024 fwd"),
    (12, 1, "forward", False, "N=4096 fwd"),
    (8, 8, "forward", False, "N=256 fwd batch=8"),
    (8, 1, "inverse", True, "N=256 inv normalize"),
]


def _sin_cos_lanes(n, batch):
    i = np.arange(n, dtype=np.float32)
    return np.tile((np.sin(i) + 1j * np.cos(i)).astype(np.complex64), batch)


def _numpy_ref(x, n, direction, normalize):
    lanes = x.astype(np.complex128).reshape(-1, n)
    if direction == "forward":
        return np.fft.fft(lanes, axis=1).reshape(-1)
    r = np.fft.ifft(lanes, axis=1)
    return (r if normalize else r * n).reshape(-1)


@pytest.mark.parametrize("log_n,batch,direction,normalize,label", CASES)
@pytest.mark.parametrize("use_device", [False, True])
def test_reference_cases_match_numpy(gpu_device, log_n, batch, direction, normalize, label, use_device):
    n = 1 << log_n
    x = _sin_cos_lanes(n, batch)
    exp = _numpy_ref(x, n, direction, normalize).astype(np.complex64)
    out = _fft(x, log_n, direction, normalize, device=gpu_device if use_device else None)
    assert out.shape == x.shape
    err = float(np.max(np.abs(out - exp))) / max(1e-9, float(np.max(np.abs(exp))))
    assert err < 1e-4, f"{label} use_device={use_device}: {err}"
    assert rel_l2(out, oracle.fft_1d(x, log_n, direction, normalize)) <= TOL


@pytest.mark.parametrize("log_n,direction,normalize", [(8, "forward", False), (8, "inverse", True),
                                                       (12, "forward", False)])
def test_reference_large_batch_cases(gpu_device, log_n, direction, normalize):
    # test_fft_vs_numpy.py:71-107 (batch 4096; the reference allowed 1e-3).
    n = 1 << log_n
    x = _sin_cos_lanes(n, 4096)
    out = _fft(x, log_n, direction, normalize, device=gpu_device)
    exp = _numpy_ref(x, n, direction, normalize)
    assert float(np.max(np.abs(out - exp))) / float(np.max(np.abs(exp))) < 1e-4
    assert rel_l2(out, oracle.fft_1d(x, log_n, direction, normalize, threads=8)) <= TOL


# ---- device-resident plans and the BASELINE configurations -------------------


def _run_plan(dev, log_n, batch, x, direction="forward", normalize=False, in_place=False):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    plan = ferrum_gpu.fft.Plan1D(log_n, batch, dev)
    a = DeviceBuffer(dev, plan.nbytes)
    a.copy_from_host(x)
    b = a if in_place else DeviceBuffer(dev, plan.nbytes)
    plan.execute(a, b, direction, normalize)
    dev.sync()
    out = np.empty_like(x)
    b.copy_to_host(out)
    plan.destroy()
    return out


def test_config1_n1024_b256(gpu_device):
    rng = np.random.default_rng(1)
    x = uniform_c64(rng, 256 * 1024)
    assert rel_l2(_run_plan(gpu_device, 10, 256, x), oracle.fft_1d(x, 10)) <= TOL


@pytest.mark.parametrize("log_n", [8, 12])
def test_config2_forward_inverse(gpu_device, log_n):
    rng = np.random.default_rng(2)
    x = uniform_c64(rng, 256 << log_n)
    fwd = _run_plan(gpu_device, log_n, 256, x)
    assert rel_l2(fwd, oracle.fft_1d(x, log_n)) <= TOL
    inv = _run_plan(gpu_device, log_n, 256, fwd, "inverse", True)
    assert rel_l2(inv, oracle.fft_1d(fwd, log_n, "inverse", True)) <= TOL
    assert rel_l2(inv, x) <= TOL


def test_config3_n1024_b65536(gpu_device):
    rng = np.random.default_rng(3)
    x = normal_c64(rng, 65536 * 1024)
    print("[case] config3 N=1024 batch=65536", flush=True)
    got = _run_plan(gpu_device, 10, 65536, x)
    ref = oracle.fft_1d(x, 10, threads=8)
    assert rel_l2(got, ref) <= TOL
    # per-lane bound too: no lane may hide behind the global norm
    lanes = np.linalg.norm((got - ref).reshape(65536, 1024), axis=1) / np.linalg.norm(ref.reshape(65536, 1024), axis=1)
    assert lanes.max() <= 10 * TOL


def test_in_place_and_deterministic(gpu_device):
    rng = np.random.default_rng(9)
    x = uniform_c64(rng, 300 * 1024)
    a = _run_plan(gpu_device, 10, 300, x)
    b = _run_plan(gpu_device, 10, 300, x, in_place=True)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("log_n", [10, 16])
def test_exec_refuses_partial_overlap_and_misalignment(gpu_device, log_n):
    # checked on the host before any launch: in and out equal or disjoint,
    # both 8-byte aligned (a single-pass and a multi-pass plan)
    import ferrum_gpu
    from ferrum_gpu import _native as N
    from ferrum_gpu.hip import DeviceBuffer

    plan = ferrum_gpu.fft.Plan1D(log_n, 4, gpu_device)
    buf = DeviceBuffer(gpu_device, 2 * plan.nbytes)
    for d_in, d_out, what in ((buf.ptr, buf.ptr + 8 * (1 << log_n), "overlap"),
                              (buf.ptr + plan.nbytes - 8, buf.ptr, "overlap"),
                              (buf.ptr + 4, buf.ptr + plan.nbytes + 8, "aligned"),
                              (buf.ptr, buf.ptr + plan.nbytes + 4, "aligned")):
        with pytest.raises(N.FerrumGpuError, match=what):
            plan.execute(d_in, d_out)
    # disjoint neighbours and in place are fine
    plan.execute(buf.ptr, buf.ptr + plan.nbytes)
    plan.execute(buf.ptr, buf.ptr)
    gpu_device.sync()
    plan.destroy()


def test_persistent_device_and_one_shot_agree(gpu_device):
    rng = np.random.default_rng(10)
    x = uniform_c64(rng, 3 * 4096)
    assert np.array_equal(_fft(x, 12, device=gpu_device), _fft(x, 12))

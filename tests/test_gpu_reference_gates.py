"""The reference's own GPU correctness gates, re-created on this backend.

* examples/fft-1d-c2c/src/main.rs:55-120 -- 8 cases on (sin(i mod N),
  cos(i mod N)) with the per-element metric of :233-249,
  (|dre| + |dim|) / (|re| + |im| + 1) <= rel_tol (1e-4; 5e-4 at N = 4096).
* crates/ferrum-gpu-bench/src/bin/kernel-cross-check.rs:60-185 -- N = 256,
  1024, 4096, batch 4, input (sin(0.013 t), cos(0.021 t)), t = i mod N, metric
  max |gpu - cpu| / max(|cpu|, 1) <= 1e-3 (:21-57).
* crates/ferrum-gpu-bench/src/bin/batch-sweep-4096.rs:36-135 -- N = 4096,
  batch 512 (many co-resident workgroups, the race gate), input
  (sin(0.0007 i), cos(0.0011 i)) over the whole batch, same metric.

Each case is also held to this build's bar, relative L2 <= 1e-4 against the
CPU oracle.  Inputs are computed in float32 as the reference's `as f32`
arithmetic does; the oracle and the GPU see the same array.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _c64(re, im):
    x = np.empty(re.size, np.complex64)
    x.real, x.imag = re, im
    return x


def _example_metric(gpu, cpu):
    # examples/fft-1d-c2c/src/main.rs:233-249
    d = np.abs(gpu.real - cpu.real) + np.abs(gpu.imag - cpu.imag)
    return float(np.max(d / (np.abs(cpu.real) + np.abs(cpu.imag) + 1.0)))


def _cross_check_metric(gpu, cpu):
    # kernel-cross-check.rs:42-57, batch-sweep-4096.rs:65-73
    err = np.abs(gpu.astype(np.complex128) - cpu.astype(np.complex128))
    return float(np.max(err / np.maximum(np.abs(cpu.astype(np.complex128)), 1.0)))


EXAMPLE_CASES = [  # (log_n, batch, direction, normalize, rel_tol, label)
    (2, 1, "forward", False, 1e-4, "N=4 fwd"),
    (3, 1, "forward", False, 1e-4, "N=8 fwd"),
    (6, 1, "forward", False, 1e-4, "N=64 fwd"),
    (8, 1, "forward", False, 1e-4, "N=256 fwd"),
    (10, 1, "forward", False, 1e-4, "N=1024 fwd"),
    (12, 1, "forward", False, 5e-4, "N=4096 fwd"),
    (8, 8, "forward", False, 1e-4, "N=256 fwd batch=8"),
    (8, 1, "inverse", True, 1e-4, "N=256 inv normalize"),
]


@pytest.mark.parametrize("log_n,batch,direction,normalize,rel_tol,label", EXAMPLE_CASES,
                         ids=[c[-1] for c in EXAMPLE_CASES])
def test_example_fft_1d_c2c_cases(gpu_device, log_n, batch, direction, normalize, rel_tol, label):
    import ferrum_gpu

    n = 1 << log_n
    t = (np.arange(n * batch) % n).astype(np.float32)
    x = _c64(np.sin(t), np.cos(t))
    got = ferrum_gpu.fft.fft_1d_c2c_pow2(x, log_n, direction, normalize, device=gpu_device)
    cpu = oracle.fft_1d(x, log_n, direction, normalize)
    assert _example_metric(got, cpu) <= rel_tol, label
    assert rel_l2(got, cpu) <= TOL, label


@pytest.mark.parametrize("log_n", [8, 10, 12])
def test_kernel_cross_check(gpu_device, log_n):
    import ferrum_gpu

    n, batch = 1 << log_n, 4
    t = (np.arange(n * batch) % n).astype(np.float32)
    x = _c64(np.sin(t * np.float32(0.013)), np.cos(t * np.float32(0.021)))
    got = ferrum_gpu.fft.fft_1d_c2c_pow2(x, log_n, device=gpu_device)
    cpu = oracle.fft_1d(x, log_n)
    assert _cross_check_metric(got, cpu) <= 1e-3
    assert rel_l2(got, cpu) <= TOL


def test_batch_sweep_4096_race_gate(gpu_device):
    import ferrum_gpu

    n, batch = 4096, 512
    i = np.arange(n * batch).astype(np.float32)
    x = _c64(np.sin(i * np.float32(0.0007)), np.cos(i * np.float32(0.0011)))
    plan = ferrum_gpu.fft.Plan1D(12, batch, gpu_device)
    from ferrum_gpu.hip import DeviceBuffer

    a, b = DeviceBuffer(gpu_device, x.nbytes), DeviceBuffer(gpu_device, x.nbytes)
    a.copy_from_host(x)
    cpu = oracle.fft_1d(x, 12, threads=8)
    for _ in range(3):  # repeated launches: a missing barrier shows as run-to-run drift
        plan.execute(a, b)
        gpu_device.sync()
        got = np.empty_like(x)
        b.copy_to_host(got)
        assert _cross_check_metric(got, cpu) <= 1e-3
        assert rel_l2(got, cpu) <= TOL

"""GPU parity of the seeded synthetic-data generator (fg_fill_uniform_c64 /
fg_fill_normal_c64) against its CPU restatement in oracle/.

Uniform values are integer arithmetic plus an exact scaling: bit-exact.
Normal values go through f64 log / sqrt / cos / sin, whose device and host
implementations may differ in the last f64 bit; after rounding to f32 that
leaves at most one f32 ulp on a rare element (tolerance stated below).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _gen(gpu_device, kind, n, seed, offset=0):
    import ctypes

    from ferrum_gpu import _native as N
    from ferrum_gpu import synthetic
    from ferrum_gpu.hip import DeviceBuffer

    buf = DeviceBuffer(gpu_device, 8 * n + 16)
    getattr(synthetic, kind)(gpu_device, buf.ptr + offset, n, seed)
    out = np.empty(n, np.complex64)
    gpu_device.sync()
    N.check(N.lib.fg_copy_d2h(gpu_device.handle, out.ctypes.data, ctypes.c_void_p(buf.ptr + offset), out.nbytes))
    return out


@pytest.mark.parametrize("n,seed", [(1, 0), (7, 1), (4099, 2), ((1 << 24) + 3, 3), (1 << 20, 2**64 - 1)])
def test_uniform_bit_exact(gpu_device, n, seed):
    print(f"[case] fill uniform n={n} seed={seed}", flush=True)
    got = _gen(gpu_device, "uniform", n, seed)
    assert np.array_equal(got, oracle.fill_uniform_c64(n, seed))


@pytest.mark.parametrize("n,seed", [(5, 0), (4099, 3), ((1 << 24) + 3, 4)])
def test_normal_matches_oracle(gpu_device, n, seed):
    print(f"[case] fill normal n={n} seed={seed}", flush=True)
    got = _gen(gpu_device, "normal", n, seed, offset=8)      # 8-byte aligned, not 16
    exp = oracle.fill_normal_c64(n, seed)
    g, e = got.view(np.float32), exp.view(np.float32)
    ulp = np.spacing(np.abs(e))
    assert np.all(np.abs(g - e) <= ulp)                      # at most one f32 ulp apart
    assert np.mean(g == e) > 0.9999                          # and almost always identical


def test_fill_rejects_misaligned(gpu_device):
    from ferrum_gpu import _native as N
    from ferrum_gpu import synthetic
    from ferrum_gpu.hip import DeviceBuffer

    buf = DeviceBuffer(gpu_device, 64)
    with pytest.raises(N.FerrumGpuError, match="8-byte aligned"):
        synthetic.uniform(gpu_device, buf.ptr + 4, 4, 1)

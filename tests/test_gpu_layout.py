"""GPU parity of the split layout (SoA) FFT and the pointwise kernels.

Split plans must return exactly what the interleaved plan returns on the same
data (same kernels' arithmetic, different global layout: the reference's
*_split twins, kernels_body.rs:509-626, 986-1130, 1463-1610), and lie within
1e-4 of the CPU oracle.  The pointwise kernels (cmul_interleaved, cmul_split,
deinterleave, interleave, kernels_body.rs:1612-1672) are f32 elementwise work
with contraction off, so they must match the oracle bit for bit, aligned or
not, including ragged tails and sizes that take several grid-stride sweeps.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from conftest import rel_l2, uniform_c64
from test_multipass_model import rowpair_2d

pytestmark = pytest.mark.gpu

TOL = 1e-4


class Dev:
    """Device arrays at an optional byte offset inside a larger allocation."""

    def __init__(self, device):
        from ferrum_gpu import _native as N

        self.N, self.device, self.bufs = N, device, []

    def put(self, host: np.ndarray, offset: int = 0) -> int:
        from ferrum_gpu.hip import DeviceBuffer

        a = np.ascontiguousarray(host)
        buf = DeviceBuffer(self.device, a.nbytes + offset + 16)
        self.bufs.append(buf)
        ptr = buf.ptr + offset
        self.N.check(self.N.lib.fg_copy_h2d(self.device.handle, ctypes.c_void_p(ptr), a.ctypes.data, a.nbytes))
        return ptr

    def empty(self, nbytes: int, offset: int = 0) -> int:
        from ferrum_gpu.hip import DeviceBuffer

        buf = DeviceBuffer(self.device, nbytes + offset + 16)
        self.bufs.append(buf)
        return buf.ptr + offset

    def get(self, ptr: int, n: int, dtype) -> np.ndarray:
        out = np.empty(n, dtype)
        self.device.sync()
        self.N.check(self.N.lib.fg_copy_d2h(self.device.handle, out.ctypes.data, ctypes.c_void_p(ptr), out.nbytes))
        return out


# ------------------------------------------------------------ split FFT


def _run_both(gpu_device, plan, x, direction="forward", normalize=False):
    d = Dev(gpu_device)
    n = x.size
    src = d.put(x)
    dst = d.empty(x.nbytes)
    plan.execute(src, dst, direction, normalize)
    inter = d.get(dst, n, np.complex64)
    re, im = d.put(np.ascontiguousarray(x.real)), d.put(np.ascontiguousarray(x.imag))
    o_re, o_im = d.empty(4 * n), d.empty(4 * n)
    plan.execute_split(re, im, o_re, o_im, direction, normalize)
    split = d.get(o_re, n, np.float32) + 1j * d.get(o_im, n, np.float32)
    return inter, split.astype(np.complex64)


@pytest.mark.parametrize("log_n", list(range(2, 13)) + [13, 16, 20])
def test_split_1d_equals_interleaved(gpu_device, log_n):
    import ferrum_gpu

    # batch not a multiple of the transforms per workgroup: ragged last workgroup
    batch = max(1, (1 << 18) >> log_n) + 3
    print(f"[case] split 1d log_n={log_n} batch={batch}", flush=True)
    x = uniform_c64(np.random.default_rng(log_n), batch << log_n)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    inter, split = _run_both(gpu_device, plan, x)
    assert np.array_equal(inter, split)
    if log_n <= 16:
        assert rel_l2(split, oracle.fft_1d(x, log_n, threads=8)) <= TOL
    inter_i, split_i = _run_both(gpu_device, plan, inter, "inverse", True)
    assert np.array_equal(inter_i, split_i)
    assert rel_l2(split_i, x) <= TOL


@pytest.mark.parametrize("lr,lc", [(8, 8), (12, 12), (5, 9), (11, 4), (4, 4), (6, 6), (7, 7), (10, 4), (4, 8)])
def test_split_2d_equals_interleaved(gpu_device, lr, lc):
    import ferrum_gpu

    batch = 2
    x = uniform_c64(np.random.default_rng(lr + lc), batch << (lr + lc))
    plan = ferrum_gpu.fft.Plan2D(lr, batch, gpu_device, log_cols=lc)
    inter, split = _run_both(gpu_device, plan, x)
    if rowpair_2d(lr, lc):
        # the split layout stages and runs in place: the row and column passes,
        # where out of place the plan pairs rows (another rounding)
        assert rel_l2(split, inter) <= TOL
    else:
        assert np.array_equal(inter, split)
    exp = np.fft.fft2(x.reshape(batch, 1 << lr, 1 << lc).astype(np.complex128)).reshape(-1)
    assert rel_l2(split, exp) <= TOL


@pytest.mark.parametrize("log_n", [10, 14])
def test_split_in_place(gpu_device, log_n):
    import ferrum_gpu

    batch = 37
    x = uniform_c64(np.random.default_rng(100 + log_n), batch << log_n)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    d = Dev(gpu_device)
    re, im = d.put(np.ascontiguousarray(x.real)), d.put(np.ascontiguousarray(x.imag))
    plan.execute_split(re, im, re, im)
    got = (d.get(re, x.size, np.float32) + 1j * d.get(im, x.size, np.float32)).astype(np.complex64)
    assert rel_l2(got, oracle.fft_1d(x, log_n, threads=8)) <= TOL


def test_split_2d_one_pass_in_place(gpu_device):
    import ferrum_gpu

    batch = 5
    x = uniform_c64(np.random.default_rng(77), batch << 12)
    plan = ferrum_gpu.fft.Plan2D(6, batch, gpu_device)
    assert plan.kernel_names() == ["fg_fft2d_l6_6"]
    d = Dev(gpu_device)
    re, im = d.put(np.ascontiguousarray(x.real)), d.put(np.ascontiguousarray(x.imag))
    plan.execute_split(re, im, re, im, "inverse", True)
    got = (d.get(re, x.size, np.float32) + 1j * d.get(im, x.size, np.float32)).astype(np.complex64)
    assert rel_l2(got, oracle.fft_2d(x, 6, "inverse", True)) <= TOL


def test_split_rejects_crossed_parts(gpu_device):
    import ferrum_gpu
    from ferrum_gpu import _native as N

    plan = ferrum_gpu.fft.Plan1D(8, 4, gpu_device)
    d = Dev(gpu_device)
    re, im = d.empty(4 * 1024), d.empty(4 * 1024)
    with pytest.raises(N.FerrumGpuError, match="overlapping"):
        plan.execute_split(re, im, im, re)
    with pytest.raises(N.FerrumGpuError, match="overlapping"):
        plan.execute_split(re, im, re + 4, im)


# ------------------------------------------------------------- pointwise

SIZES = [1, 3, 4, 5, 1023, 4099, (1 << 16) + 1]


@pytest.mark.parametrize("n", SIZES + [(1 << 26) + 3])
@pytest.mark.parametrize("offset", [0, 8])
def test_cmul_c64_exact(gpu_device, n, offset):
    from ferrum_gpu import pointwise

    if n > (1 << 20) and offset:
        n = (1 << 24) + 5  # the element-wise kernel strides after 2^24 elements
    print(f"[case] cmul_c64 n={n} offset={offset}", flush=True)
    rng = np.random.default_rng(n + offset)
    a, b = uniform_c64(rng, n), uniform_c64(rng, n)
    d = Dev(gpu_device)
    pa, pb, po = d.put(a, offset), d.put(b, offset), d.empty(8 * n, offset)
    pointwise.cmul(gpu_device, pa, pb, po, n)
    exp = oracle.cmul_interleaved(a, b)
    assert np.array_equal(d.get(po, n, np.complex64), exp)
    pointwise.cmul(gpu_device, pa, pb, pa, n)          # in place: out is a
    assert np.array_equal(d.get(pa, n, np.complex64), exp)


@pytest.mark.parametrize("n", SIZES + [(1 << 26) + 3])
@pytest.mark.parametrize("offset", [0, 4])
def test_cmul_split_exact(gpu_device, n, offset):
    from ferrum_gpu import pointwise

    if n > (1 << 20) and offset:
        n = (1 << 24) + 5
    print(f"[case] cmul_split n={n} offset={offset}", flush=True)
    rng = np.random.default_rng(2 * n + offset)
    a, b = uniform_c64(rng, n), uniform_c64(rng, n)
    d = Dev(gpu_device)
    ar, ai = d.put(a.real.copy(), offset), d.put(a.imag.copy(), offset)
    br, bi = d.put(b.real.copy(), offset), d.put(b.imag.copy(), offset)
    o_re, o_im = d.empty(4 * n, offset), d.empty(4 * n, offset)
    pointwise.cmul_split(gpu_device, ar, ai, br, bi, o_re, o_im, n)
    e_re, e_im = oracle.cmul_split(a.real, a.imag, b.real, b.imag)
    assert np.array_equal(d.get(o_re, n, np.float32), e_re)
    assert np.array_equal(d.get(o_im, n, np.float32), e_im)
    pointwise.cmul_split(gpu_device, ar, ai, br, bi, br, bi, n)   # in place: outputs are b
    assert np.array_equal(d.get(br, n, np.float32), e_re)
    assert np.array_equal(d.get(bi, n, np.float32), e_im)


@pytest.mark.parametrize("n", SIZES + [(1 << 26) + 3])
@pytest.mark.parametrize("offset", [0, 4])
def test_deinterleave_interleave_exact(gpu_device, n, offset):
    from ferrum_gpu import pointwise

    if n > (1 << 20) and offset:
        n = (1 << 24) + 5
    print(f"[case] (de)interleave n={n} offset={offset}", flush=True)
    x = uniform_c64(np.random.default_rng(3 * n + offset), n)
    d = Dev(gpu_device)
    # complex64 data at a 4-byte offset is not 8-byte aligned; use 8 for it
    px = d.put(x, 2 * offset)
    re, im = d.empty(4 * n, offset), d.empty(4 * n, offset)
    pointwise.deinterleave(gpu_device, px, re, im, n)
    e_re, e_im = oracle.deinterleave(x)
    assert np.array_equal(d.get(re, n, np.float32), e_re)
    assert np.array_equal(d.get(im, n, np.float32), e_im)
    back = d.empty(8 * n, 2 * offset)
    pointwise.interleave(gpu_device, re, im, back, n)
    assert np.array_equal(d.get(back, n, np.complex64), oracle.interleave(e_re, e_im))


def test_pointwise_rejects_partial_overlap(gpu_device):
    from ferrum_gpu import _native as N
    from ferrum_gpu import pointwise

    d = Dev(gpu_device)
    a = d.empty(8 * 1024)
    with pytest.raises(N.FerrumGpuError, match="overlap"):
        pointwise.cmul(gpu_device, a, a, a + 8, 512)
    with pytest.raises(N.FerrumGpuError, match="overlap"):
        pointwise.deinterleave(gpu_device, a, a, a + 4096, 256)
    pointwise.cmul(gpu_device, a, a, a, 0)   # n = 0 is a no-op

"""Arrays the layouts accept that are not 16-byte aligned -- complex64 at an
8-byte offset, f32 at a 4-byte offset -- give the same bits as aligned ones,
and split arrays that are not 4-byte aligned are refused before any launch.
Each case runs the same plan on aligned and on offset device addresses
(inside buffers 16 bytes larger than the data) and compares the outputs bit
for bit, and the aligned output against the oracle."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rel_l2, uniform_c64

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _placed(dev, nbytes, data, off):
    """A device buffer of nbytes + 16 holding `data` at byte offset `off`."""
    from ferrum_gpu.hip import DeviceBuffer

    buf = DeviceBuffer(dev, nbytes + 16)
    raw = np.zeros(nbytes + 16, np.uint8)
    raw[off:off + data.nbytes] = data.view(np.uint8).reshape(-1)
    buf.copy_from_host(raw)
    return buf


def _read(dev, buf, nbytes, off, dtype):
    raw = np.empty(nbytes + 16, np.uint8)
    dev.sync()
    buf.copy_to_host(raw)
    return raw[off:off + nbytes].view(dtype).copy()


# (dims, log_n (2D: rows), log_cols, batch, expected first kernel): the
# 1024-point kernel in 1D (an even and an odd batch) and as the 2D row pass
# (512 x 1024 and 1024 x 1024 images), the row pairs of 1024 x 2048 images,
# and the 4096-point kernel
CASES = [
    (1, 10, None, 1536, "fg_fft_n10"),
    (1, 10, None, 2049, "fg_fft_n10"),
    (2, 9, 10, 2, "fg_fft_n10"),
    (2, 10, 10, 1, "fg_fft_n10"),
    (2, 10, 11, 1, "fg_fft2d_rowpair_n11"),
    (1, 12, None, 600, "fg_fft_n12"),
]


@pytest.mark.parametrize("dims,log_n,log_cols,batch,first", CASES)
@pytest.mark.parametrize("direction", ["forward", "inverse"])
def test_interleaved_offset_by_8_bytes(gpu_device, dims, log_n, log_cols, batch, first, direction):
    import ferrum_gpu

    plan = (ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device) if dims == 1
            else ferrum_gpu.fft.Plan2D(log_n, batch, gpu_device, log_cols=log_cols))
    names = plan.kernel_names()
    assert names[0].startswith(first), names
    nb = plan.nbytes
    rng = np.random.default_rng(log_n * 1000 + batch)
    x = uniform_c64(rng, nb // 8)
    outs = []
    for off_in, off_out in ((0, 0), (8, 8), (8, 0), (0, 8)):
        print(f"[case] dims={dims} log_n={log_n} batch={batch} {direction} offsets={off_in},{off_out}", flush=True)
        a = _placed(gpu_device, nb, x, off_in)
        b = _placed(gpu_device, nb, np.zeros(0, np.uint8), 0)
        plan.execute(a.ptr + off_in, b.ptr + off_out, direction, direction == "inverse")
        outs.append(_read(gpu_device, b, nb, off_out, np.complex64))
        a.free()
        b.free()
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    if dims == 1:
        want = oracle.fft_1d(x, log_n, direction, direction == "inverse", threads=8)
    else:
        from test_gpu_extras import oracle_2d_rect
        want = oracle_2d_rect(x, log_n, log_cols, direction, direction == "inverse")
    assert rel_l2(outs[0], want) <= TOL
    plan.destroy()


@pytest.mark.parametrize("log_n,batch", [(10, 1536), (10, 77)])
def test_split_offset_by_4_bytes(gpu_device, log_n, batch):
    import ferrum_gpu

    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    n = batch << log_n
    rng = np.random.default_rng(5000 + batch)
    x = uniform_c64(rng, n)
    re, im = np.ascontiguousarray(x.real), np.ascontiguousarray(x.imag)
    got = []
    for off in (0, 4, 12):
        print(f"[case] split log_n={log_n} batch={batch} offset={off}", flush=True)
        bufs = [_placed(gpu_device, 4 * n, re, off), _placed(gpu_device, 4 * n, im, off),
                _placed(gpu_device, 4 * n, np.zeros(0, np.uint8), 0),
                _placed(gpu_device, 4 * n, np.zeros(0, np.uint8), 0)]
        plan.execute_split(*[b.ptr + off for b in bufs], "forward", False)
        got.append((_read(gpu_device, bufs[2], 4 * n, off, np.float32), _read(gpu_device, bufs[3], 4 * n, off, np.float32)))
        for b in bufs:
            b.free()
    for r, i in got[1:]:
        assert np.array_equal(r.view(np.uint32), got[0][0].view(np.uint32))
        assert np.array_equal(i.view(np.uint32), got[0][1].view(np.uint32))
    assert rel_l2(got[0][0] + 1j * got[0][1], oracle.fft_1d(x, log_n, threads=8)) <= TOL
    plan.destroy()


def test_split_arrays_must_be_4_byte_aligned(gpu_device):
    # refused on the host, before any launch
    import ferrum_gpu
    from ferrum_gpu._native import FerrumGpuError
    from ferrum_gpu.hip import DeviceBuffer

    plan = ferrum_gpu.fft.Plan1D(10, 4, gpu_device)
    bufs = [DeviceBuffer(gpu_device, 4 * 4096 + 16) for _ in range(4)]
    ptrs = [b.ptr for b in bufs]
    ptrs[2] += 2
    with pytest.raises(FerrumGpuError, match="4-byte aligned"):
        plan.execute_split(*ptrs, "forward", False)
    for b in bufs:
        b.free()
    plan.destroy()

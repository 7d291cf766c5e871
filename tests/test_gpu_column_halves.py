"""2D column passes of 512 to 4096 rows with the exchanges in halves: 8-column
tiles at 2048 / 4096 rows (fg_tile_l{11,12}_g8_h_cc) and their two tile
orders, 16-column tiles at 512 / 1024 rows (fg_tile_l{9,10}_g16_h_cs).

A chunk whose grid is a multiple of 16 tiles runs in the line-group order
(FG_TILE_ORDER_LINE_GROUPS), any other chunk in the natural order; the order
only decides which workgroup takes which tile, so every chunking of a plan
must give the same bits, and the oracle's result (the reference's 1D
Stockham along rows, then along columns, as cpu_2d.rs:9-64 builds the 2D
transform) within 1e-4.  The chunk limits below make the last chunk ragged,
so both orders run in one plan.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2, uniform_c64
from test_gpu_extras import oracle_2d_rect
from test_multipass_model import choose_chunk, two_in_flight_shape

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture
def chunk_limit():
    import ferrum_gpu

    saved = ferrum_gpu.fft.get_chunk_bytes()
    yield ferrum_gpu.fft.set_chunk_bytes
    ferrum_gpu.fft.set_chunk_bytes(saved)


def _exec(dev, x, lr, lc, direction, normalize):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    batch = x.shape[0]
    plan = ferrum_gpu.fft.Plan2D(lr, batch, dev, log_cols=lc)
    d = plan.describe()
    a, b = DeviceBuffer(dev, plan.nbytes), DeviceBuffer(dev, plan.nbytes)
    a.copy_from_host(x)
    plan.execute(a, b, direction, normalize)
    dev.sync()
    out = np.empty_like(x)
    b.copy_to_host(out)
    names = plan.kernel_names()
    plan.destroy()
    a.free()
    b.free()
    return out, d, names


# (log rows, log cols, batch, images per chunk), images above 16384 points
# (smaller ones take the one-pass kernels); tiles per image = C / 8
CASES = [
    (9, 10, 3, 2),      # 16-column tiles: 64 per image
    (9, 6, 7, 3),       # 64 columns: 4 tiles per image
    (10, 5, 11, 4),     # 16-column tiles: 2 per image
    (10, 9, 5, 2),      # 512 columns in three chunks
    (11, 4, 9, 3),      # 6 tiles per chunk: natural order throughout
    (11, 7, 5, 2),
    (11, 9, 3, 1),      # 2048 x 512 (1024 columns and more: row pairs, test_gpu_rowpair.py)
    (12, 4, 11, 8),     # 16 tiles per chunk, the last chunk 6
    (12, 6, 3, 2),      # 16 tiles per chunk, the last 8 (natural)
    (12, 9, 2, 1),
]


@pytest.mark.parametrize("lr,lc,batch,per_chunk", CASES)
def test_halves_column_pass_chunked(gpu_device, chunk_limit, lr, lc, batch, per_chunk):
    image = 8 << (lr + lc)
    rng = np.random.default_rng(4000 + 16 * lr + lc)
    x = uniform_c64(rng, batch * (image // 8)).reshape(batch, 1 << lr, 1 << lc)
    # 2D plans run one chunk at a time, of up to the chunk limit
    limit = per_chunk * image
    chunk_limit(limit)
    print(f"[case] 2d {1 << lr}x{1 << lc} batch={batch} chunk={per_chunk} images", flush=True)
    fwd, d, names = _exec(gpu_device, x, lr, lc, "forward", False)
    per, _, two = choose_chunk(image, batch, limit, two_in_flight_shape(True, lr, lc))
    assert per == per_chunk and not two
    # 512 / 1024 rows: 16 columns, streamed out; 2048 / 4096 rows: 8 columns
    assert names[-1] == (f"fg_tile_l{lr}_g16_h_cs" if lr <= 10 else f"fg_tile_l{lr}_g8_h_cc"), names
    assert d["streams"] == 1
    assert d["units_per_chunk"] == per_chunk and d["chunks"] == -(-batch // per_chunk)
    assert rel_l2(fwd, oracle_2d_rect(x, lr, lc)) <= TOL
    inv, _, _ = _exec(gpu_device, fwd, lr, lc, "inverse", True)
    assert rel_l2(inv, oracle_2d_rect(fwd, lr, lc, "inverse", True)) <= TOL
    assert rel_l2(inv, x) <= TOL
    # one chunk for the whole batch: other grids, other tile orders, same bits
    chunk_limit(batch * image)
    one, d1, _ = _exec(gpu_device, x, lr, lc, "forward", False)
    assert d1["chunks"] == 1
    assert np.array_equal(one.view(np.uint32), fwd.view(np.uint32))


@pytest.mark.parametrize("lr", [10, 11, 12])
def test_halves_column_pass_f64_bins(gpu_device, lr):
    # a separable fp64 DFT on sampled (k_r, k_c) of a square image
    import ferrum_gpu

    n = 1 << lr
    rng = np.random.default_rng(77 + lr)
    x = uniform_c64(rng, n * n).reshape(1, n, n)
    print(f"[case] 2d {n}x{n} fp64 bins", flush=True)
    got = ferrum_gpu.fft.fft2_c2c_pow2(x, device=gpu_device)[0]
    xr = x[0].astype(np.complex128)
    ks = rng.integers(0, n, size=(16, 2))
    idx = np.arange(n)
    err = 0.0
    for kr, kc in ks:
        wr = np.exp(-2j * np.pi * ((kr * idx) % n) / n)
        wc = np.exp(-2j * np.pi * ((kc * idx) % n) / n)
        want = wr @ xr @ wc
        err = max(err, abs(got[kr, kc] - want) / np.sqrt(n * n))
    assert err <= 1e-4

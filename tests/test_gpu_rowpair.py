"""2D images of 2048 / 4096 rows of 1024 .. 4096 points and of 1024 rows of 2048
/ 4096 points out of place: the row
pass over row pairs (fg_fft2d_rowpair_n{10,11,12}: rows r and r + R/2, stored as
A + B to row 2r and (A - B) W_R^r to row 2r + 1), then R/2-point column DFTs
over the rows of each parity in place (element stride 2C; fg_tile_l11_g8_h_cc
at 4096 rows, fg_tile_l10_g16_h_cs at 2048, fg_tile_l9_g16_h_cs at 1024).

In place the same plan runs the row pass and the R-row column tiles.  Both
are checked against the oracle (the reference's 1D Stockham along rows, then
along columns, as cpu_2d.rs:9-64 builds the 2D transform) within 1e-4, in both
directions, chunked and unchunked (same bits: chunking only moves the
launches), and through a graph replay (same bits as the eager call).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2, uniform_c64
from test_gpu_extras import oracle_2d_rect
from test_multipass_model import plan_kernel_names, rowpair_2d

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture
def chunk_limit():
    import ferrum_gpu

    saved = ferrum_gpu.fft.get_chunk_bytes()
    yield ferrum_gpu.fft.set_chunk_bytes
    ferrum_gpu.fft.set_chunk_bytes(saved)


def _run(dev, x, lr, lc, direction="forward", normalize=False, in_place=False):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    plan = ferrum_gpu.fft.Plan2D(lr, x.shape[0], dev, log_cols=lc)
    a = DeviceBuffer(dev, plan.nbytes)
    b = a if in_place else DeviceBuffer(dev, plan.nbytes)
    a.copy_from_host(x)
    plan.execute(a, b, direction, normalize)
    dev.sync()
    out = np.empty_like(x)
    b.copy_to_host(out)
    d = plan.describe()
    names = plan.kernel_names()
    plan.destroy()
    a.free()
    if not in_place:
        b.free()
    return out, d, names


# (log rows, log cols, batch, images per chunk)
CASES = [(12, 11, 3, 2), (12, 12, 2, 1), (12, 12, 1, 1), (11, 11, 5, 2), (11, 12, 3, 2), (11, 10, 5, 2), (12, 10, 3, 2),
         (10, 11, 7, 3), (10, 12, 3, 2)]


@pytest.mark.parametrize("lr,lc,batch,per_chunk", CASES)
def test_rowpair_out_of_place(gpu_device, chunk_limit, lr, lc, batch, per_chunk):
    image = 8 << (lr + lc)
    x = uniform_c64(np.random.default_rng(900 + lc + batch), batch * (image // 8)).reshape(batch, 1 << lr, 1 << lc)
    chunk_limit(per_chunk * image)
    print(f"[case] rowpair {1 << lr}x{1 << lc} batch={batch} chunk={per_chunk} images", flush=True)
    fwd, d, names = _run(gpu_device, x, lr, lc)
    assert rowpair_2d(lr, lc)
    assert names[:d["passes"]] == plan_kernel_names(True, lr, True, lc) == \
        [f"fg_fft2d_rowpair_n{lc}", "fg_tile_l11_g8_h_cc" if lr == 12 else f"fg_tile_l{lr - 1}_g16_h_cs"]
    assert d["workspace_bytes"] == 0 and d["streams"] == 1
    assert d["units_per_chunk"] == per_chunk and d["chunks"] == -(-batch // per_chunk)
    assert rel_l2(fwd, oracle_2d_rect(x, lr, lc)) <= TOL
    inv, _, _ = _run(gpu_device, fwd, lr, lc, "inverse", True)
    assert rel_l2(inv, oracle_2d_rect(fwd, lr, lc, "inverse", True)) <= TOL
    assert rel_l2(inv, x) <= TOL
    raw, _, _ = _run(gpu_device, fwd, lr, lc, "inverse", False)
    assert rel_l2(raw, oracle_2d_rect(fwd, lr, lc, "inverse", False)) <= TOL
    # the whole batch in one chunk: same bits
    chunk_limit(batch * image)
    one, d1, _ = _run(gpu_device, x, lr, lc)
    assert d1["chunks"] == 1
    assert np.array_equal(one.view(np.uint32), fwd.view(np.uint32))


@pytest.mark.parametrize("lr,lc", [(12, 10), (12, 11), (12, 12), (11, 10), (11, 11), (11, 12), (10, 11), (10, 12)])
def test_rowpair_in_place_takes_the_row_column_passes(gpu_device, lr, lc):
    batch = 2
    x = uniform_c64(np.random.default_rng(950 + lc), batch << (lr + lc)).reshape(batch, 1 << lr, 1 << lc)
    print(f"[case] rowpair plan in place {1 << lr}x{1 << lc} batch={batch}", flush=True)
    got, _, _ = _run(gpu_device, x, lr, lc, in_place=True)
    want = oracle_2d_rect(x, lr, lc)
    assert rel_l2(got, want) <= TOL
    inv, _, _ = _run(gpu_device, got, lr, lc, "inverse", True, in_place=True)
    assert rel_l2(inv, x) <= TOL
    out, _, _ = _run(gpu_device, x, lr, lc)
    assert rel_l2(out, got) <= TOL  # another rounding, the same transform


def test_rowpair_sampled_bins_f64(gpu_device):
    # separable fp64 DFT at sampled (k_r, k_c), both parities of k_r
    lr, lc = 12, 12
    n = 1 << lr
    rng = np.random.default_rng(961)
    x = uniform_c64(rng, n * n).reshape(1, n, n)
    print("[case] rowpair 4096x4096 fp64 bins", flush=True)
    got, _, _ = _run(gpu_device, x, lr, lc)
    img = x[0].astype(np.complex128)
    idx = np.arange(n)
    for kr, kc in [(0, 0), (1, 0), (2048, 5), (2049, 4095), (777, 3001), (3000, 17)]:
        v = np.exp(-2j * np.pi * ((kr * idx) % n) / n) @ img @ np.exp(-2j * np.pi * ((kc * idx) % n) / n)
        assert abs(got[0, kr, kc] - v) <= 1e-4 * np.linalg.norm(img), (kr, kc)


def test_rowpair_graph_replay(gpu_device):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    lr, lc, batch = 12, 11, 2
    x = uniform_c64(np.random.default_rng(970), batch << (lr + lc)).reshape(batch, 1 << lr, 1 << lc)
    print("[case] rowpair graph 4096x2048 batch=2", flush=True)
    plan = ferrum_gpu.fft.Plan2D(lr, batch, gpu_device, log_cols=lc)
    a, b = DeviceBuffer(gpu_device, plan.nbytes), DeviceBuffer(gpu_device, plan.nbytes)
    a.copy_from_host(x)
    plan.execute(a, b)
    gpu_device.sync()
    eager = np.empty_like(x)
    b.copy_to_host(eager)
    g = plan.capture_graph(a, b, reps=2)
    for _ in range(3):
        b.copy_from_host(np.zeros_like(x))
        g.launch()
        gpu_device.sync()
        got = np.empty_like(x)
        b.copy_to_host(got)
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32))
    g.destroy()
    plan.destroy()
    a.free()
    b.free()
    assert rel_l2(eager, oracle_2d_rect(x, lr, lc)) <= TOL

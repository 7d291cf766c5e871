"""Chunked execution of multi-launch plans (1D N > 16384 and 2D images above 16384 points).

A multi-launch plan runs all of its passes over one chunk of whole
transforms (images) before the next, keeping the chunk's intermediate array
cached; the chunk limit is process-wide (ferrum_gpu.fft.set_chunk_bytes) and
read when a plan is created.  Chunking changes only which transforms a launch
covers, the cache hints of its accesses and the tile widths of the passes
that read the cached intermediate (how many columns a workgroup owns), never
the arithmetic done on a column, so every chunking of a plan must give
bit-identical output -- and the oracle's result within 1e-4.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import normal_c64, rel_l2, uniform_c64
from test_multipass_model import choose_chunk, plan_kernel_names, rowpair_2d, two_in_flight_shape

pytestmark = pytest.mark.gpu

TOL = 1e-4
MIB = 1 << 20


@pytest.fixture
def chunk_limit():
    """Sets the process-wide chunk limit for the test and restores it after."""
    import ferrum_gpu

    saved = ferrum_gpu.fft.get_chunk_bytes()
    yield ferrum_gpu.fft.set_chunk_bytes
    ferrum_gpu.fft.set_chunk_bytes(saved)


def _run(dev, x, log_n, batch, two_d, direction="forward", normalize=False, in_place=False):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    plan = (ferrum_gpu.fft.Plan2D if two_d else ferrum_gpu.fft.Plan1D)(log_n, batch, dev)
    d = plan.describe()
    a = DeviceBuffer(dev, plan.nbytes)
    b = a if in_place else DeviceBuffer(dev, plan.nbytes)
    a.copy_from_host(x)
    plan.execute(a, b, direction, normalize)
    dev.sync()
    out = np.empty_like(x)
    b.copy_to_host(out)
    names = plan.kernel_names()
    plan.destroy()
    return out, d, names


# (two_d, log_n, batch): transform sizes 64 KiB .. 128 MiB, batches that
# do and do not divide into chunks.
CASES = [
    (False, 17, 37),
    (False, 16, 64),
    (False, 20, 3),
    (True, 8, 40),
    (True, 10, 9),
    (True, 11, 3),
]


@pytest.mark.parametrize("two_d,log_n,batch", CASES)
def test_every_chunking_gives_the_same_bits(gpu_device, chunk_limit, two_d, log_n, batch):
    elems = 1 << (2 * log_n if two_d else log_n)
    unit = 8 * elems
    rng = np.random.default_rng(900 + log_n)
    x = uniform_c64(rng, batch * elems)
    ref = oracle.fft_2d(x, log_n) if two_d else oracle.fft_1d(x, log_n, threads=8)
    outs = {}
    # 0: one chunk, every pass streaming; one unit at a time; one and three
    # units per chunk with two in flight; the default 256 MiB.
    shape = two_in_flight_shape(two_d, log_n)
    for limit in (0, unit, 2 * unit, 6 * unit, 256 * MIB):
        chunk_limit(limit)
        print(f"[case] two_d={two_d} log_n={log_n} batch={batch} chunk_limit={limit}", flush=True)
        got, d, names = _run(gpu_device, x, log_n, batch, two_d)
        assert rel_l2(got, ref) <= TOL
        if limit == 0:
            assert d["chunks"] == 1 and not d["cache_resident"] and d["units_per_chunk"] == batch
            assert not any(n.endswith(("_sc", "_cs")) for n in names)
        else:
            per, _, two = choose_chunk(unit, batch, limit, shape)
            assert d["cache_resident"] and d["units_per_chunk"] == per
            assert d["chunks"] == -(-batch // per) and d["streams"] == (2 if two else 1)
            # first pass streams in, last streams out, middle passes stay
            # cached; narrow tiles always cached (the model's names per pass)
            # (the row-pair pass always streams in and stores cached: no suffix)
            assert names[0].endswith("_sc") or names[0].startswith("fg_fft2d_rowpair_")
            assert names[:d["passes"]] == plan_kernel_names(two_d, log_n, cached=True, streams=d["streams"])
        assert d["launches"] == d["passes"] * d["chunks"] == len(names)
        outs[limit] = got
    for limit, got in outs.items():
        assert np.array_equal(got, outs[0]), f"chunk limit {limit} changed the output bits"


@pytest.mark.parametrize("two_d,log_n,batch", [(False, 16, 10), (True, 11, 3)])
@pytest.mark.parametrize("normalize", [False, True])
def test_chunked_inverse_and_in_place(gpu_device, chunk_limit, two_d, log_n, batch, normalize):
    elems = 1 << (2 * log_n if two_d else log_n)
    # two units per chunk (the last chunk partial for odd batches): two such
    # chunks in flight for 1D
    chunk_limit((4 if two_in_flight_shape(two_d, log_n) else 2) * 8 * elems)
    rng = np.random.default_rng(950 + log_n)
    x = normal_c64(rng, batch * elems)
    ref = (oracle.fft_2d(x, log_n, "inverse", normalize) if two_d
           else oracle.fft_1d(x, log_n, "inverse", normalize, threads=8))
    got, d, _ = _run(gpu_device, x, log_n, batch, two_d, "inverse", normalize)
    assert d["chunks"] == -(-batch // 2)
    assert rel_l2(got, ref) <= TOL
    got_ip, _, _ = _run(gpu_device, x, log_n, batch, two_d, "inverse", normalize, in_place=True)
    if two_d and rowpair_2d(log_n, log_n):
        # out of place the plan pairs rows (another rounding of the same transform)
        assert rel_l2(got_ip, got) <= TOL
    else:
        assert np.array_equal(got_ip, got)


def test_chunked_split_layout(gpu_device, chunk_limit):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    log_n, batch = 16, 12
    n = batch << log_n
    chunk_limit(8 * 8 << log_n)  # two chunks of 4 in flight
    rng = np.random.default_rng(977)
    x = uniform_c64(rng, n)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    assert plan.describe()["chunks"] == 3
    parts = [DeviceBuffer(gpu_device, 4 * n) for _ in range(4)]
    parts[0].copy_from_host(np.ascontiguousarray(x.real))
    parts[1].copy_from_host(np.ascontiguousarray(x.imag))
    plan.execute_split(parts[0], parts[1], parts[2], parts[3])
    gpu_device.sync()
    re, im = np.empty(n, np.float32), np.empty(n, np.float32)
    parts[2].copy_to_host(re)
    parts[3].copy_to_host(im)
    assert rel_l2(re + 1j * im, oracle.fft_1d(x, log_n, threads=8)) <= TOL
    plan.destroy()


def test_chunk_limit_applies_to_new_plans_only(gpu_device, chunk_limit):
    import ferrum_gpu

    chunk_limit(256 * MIB)
    a = ferrum_gpu.fft.Plan1D(16, 512, gpu_device)  # 256 MiB: two chunks of 256 transforms in flight
    chunk_limit(0)
    b = ferrum_gpu.fft.Plan1D(16, 512, gpu_device)
    assert a.describe()["chunks"] == 2 and a.describe()["units_per_chunk"] == 256
    assert b.describe()["chunks"] == 1 and not b.describe()["cache_resident"]
    # single-launch plans never chunk
    c = ferrum_gpu.fft.Plan1D(10, 65536, gpu_device)
    assert c.describe()["chunks"] == 1 and c.describe()["passes"] == 1
    for p in (a, b, c):
        p.destroy()


@pytest.mark.parametrize("chunked", [True, False], ids=["chunked", "unchunked"])
def test_plan_kernels_follow_the_tile_width_tables(gpu_device, chunk_limit, chunked):
    # Passes that read HBM use the wide tiles, passes over a chunk's cached
    # intermediate the cache-resident widths: the host's choice for every
    # multi-launch plan equals the CPU model's (test_multipass_model), which
    # is the geometry the CPU tests prove against the oracle.
    import ferrum_gpu

    chunk_limit(128 * MIB if chunked else 0)
    for log_n in range(13, 25):
        plan = ferrum_gpu.fft.Plan1D(log_n, 1, gpu_device)
        assert plan.kernel_names() == plan_kernel_names(False, log_n, chunked), log_n
        plan.destroy()
    for lr in range(4, 13):
        for lc in (4, 7, lr, 12):
            plan = ferrum_gpu.fft.Plan2D(lr, 1, gpu_device, log_cols=lc)
            assert plan.kernel_names() == plan_kernel_names(True, lr, chunked, lc), (lr, lc)
            plan.destroy()


def test_default_chunking_of_the_baseline_configs(gpu_device, chunk_limit):
    # The default limit (256 MiB of chunks in flight): configs 1-3 are single
    # launches; config 4 (four 128 MiB transforms) runs two chunks of one at a
    # time on two streams; config 5 (two 128 MiB images) one chunk of both on
    # one stream.
    import ferrum_gpu

    chunk_limit(256 * MIB)
    for log_n, batch in ((10, 256), (8, 256), (12, 256), (10, 65536)):
        p = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
        d = p.describe()
        assert d["launches"] == 1 and d["chunks"] == 1 and d["streams"] == 1, (log_n, batch, d)
        p.destroy()
    p4 = ferrum_gpu.fft.Plan1D(24, 4, gpu_device)
    d4 = p4.describe()
    assert (d4["passes"], d4["chunks"], d4["units_per_chunk"], d4["streams"]) == (3, 4, 1, 2)
    assert d4["cache_resident"]
    p4.destroy()
    p5 = ferrum_gpu.fft.Plan2D(12, 2, gpu_device)
    d5 = p5.describe()
    assert (d5["passes"], d5["chunks"], d5["units_per_chunk"], d5["streams"]) == (2, 1, 2, 1)
    assert d5["cache_resident"] and d5["workspace_bytes"] == 0
    assert p5.kernel_names() == ["fg_fft2d_rowpair_n12", "fg_tile_l11_g8_h_cc"]
    p5.destroy()

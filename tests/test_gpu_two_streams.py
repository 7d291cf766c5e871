"""Two-stream execution of multi-pass 1D plans (fg_fft_plan_streams == 2).

A multi-pass 1D plan of two or more chunks runs its odd chunks on a second
stream of its own, with a second workspace, forked from the caller's stream
when an execution starts and joined back when it ends.  Which stream runs a
chunk changes nothing in the arithmetic, so the output must be bit-identical
to the same plan run as one chunk on one stream, and the oracle's (the
reference's Stockham, cpu.rs:90-124) within 1e-4; work enqueued afterwards
on the caller's stream must see the whole output; events must be stamped on
each launch's own stream; and under graph capture the plan runs on the
captured stream alone.  2D plans run one stream in every chunking.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import normal_c64, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture
def chunk_limit():
    import ferrum_gpu

    saved = ferrum_gpu.fft.get_chunk_bytes()
    yield ferrum_gpu.fft.set_chunk_bytes
    ferrum_gpu.fft.set_chunk_bytes(saved)


def _run(dev, x, log_n, batch, direction="forward", normalize=False):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    plan = ferrum_gpu.fft.Plan1D(log_n, batch, dev)
    d = plan.describe()
    a, b = DeviceBuffer(dev, plan.nbytes), DeviceBuffer(dev, plan.nbytes)
    a.copy_from_host(x)
    plan.execute(a, b, direction, normalize)
    dev.sync()
    out = np.empty_like(x)
    b.copy_to_host(out)
    plan.destroy()
    a.free()
    b.free()
    return out, d


def _lanes(out, x, log_n, batch, direction="forward", normalize=False):
    n = 1 << log_n
    err = 0.0
    for lane in sorted({0, batch // 2, batch - 1}):
        got = out[lane * n:(lane + 1) * n]
        want = oracle.fft_1d(x[lane * n:(lane + 1) * n], log_n, direction, normalize, threads=8)
        err = max(err, rel_l2(got, want))
    return err


# (log_n, batch, transforms per chunk): an even and an odd number of chunks,
# a ragged last chunk, and config 4's shape
CASES = [(16, 7, 2), (17, 4, 1), (18, 3, 1), (20, 3, 1), (22, 5, 2), (24, 2, 1)]


@pytest.mark.parametrize("log_n,batch,per_chunk", CASES)
def test_two_streams_match_one_stream_bits(gpu_device, chunk_limit, log_n, batch, per_chunk):
    n = 1 << log_n
    rng = np.random.default_rng(log_n * 31 + batch)
    x = normal_c64(rng, batch * n)
    print(f"[case] two streams log_n={log_n} batch={batch} chunk={per_chunk}", flush=True)
    chunk_limit(2 * per_chunk * n * 8)  # the limit bounds both chunks in flight
    two, d2 = _run(gpu_device, x, log_n, batch)
    assert d2["streams"] == 2 and d2["chunks"] == -(-batch // per_chunk)
    chunk_limit(2 * batch * n * 8)
    one, d1 = _run(gpu_device, x, log_n, batch)
    assert d1["streams"] == 1 and d1["chunks"] == 1
    assert np.array_equal(two.view(np.uint32), one.view(np.uint32))
    assert _lanes(two, x, log_n, batch) <= TOL


def test_two_stream_output_is_ordered_on_the_callers_stream(gpu_device, chunk_limit):
    # forward then normalised inverse back to back on a user stream, no
    # synchronisation between them: the inverse must read the whole forward
    # output, and the copy after it the whole inverse output
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer, Stream

    log_n, batch = 20, 5
    n = 1 << log_n
    chunk_limit(2 * n * 8)
    x = normal_c64(np.random.default_rng(12), batch * n)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    assert plan.describe()["streams"] == 2
    s = Stream(gpu_device)
    a, b, c = (DeviceBuffer(gpu_device, plan.nbytes) for _ in range(3))
    a.copy_from_host(x)
    for _ in range(3):
        plan.execute(a, b, "forward", False, stream=s.handle)
        plan.execute(b, c, "inverse", True, stream=s.handle)
        plan.execute(c, a, "forward", False, stream=s.handle)
        plan.execute(a, c, "inverse", True, stream=s.handle)
        plan.execute(c, a, "forward", False, stream=s.handle)
        plan.execute(a, a, "inverse", True, stream=s.handle)   # in place
    s.sync()
    back = np.empty_like(x)
    a.copy_to_host(back)
    assert rel_l2(back, x) <= 1e-5
    s.destroy()
    plan.destroy()


def test_two_stream_events_on_each_launchs_stream(gpu_device, chunk_limit):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer, Event

    log_n, batch = 16, 8
    n = 1 << log_n
    chunk_limit(4 * n * 8)
    x = normal_c64(np.random.default_rng(5), batch * n)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    d = plan.describe()
    assert d["streams"] == 2 and d["chunks"] == 4 and d["launches"] == 8
    a, b = DeviceBuffer(gpu_device, plan.nbytes), DeviceBuffer(gpu_device, plan.nbytes)
    a.copy_from_host(x)
    start = Event(gpu_device)
    evs = [Event(gpu_device) for _ in range(d["launches"])]
    start.record()
    plan.execute_recording(a, b, evs)
    gpu_device.sync()
    t = [start.elapsed_ms(e) for e in evs]
    passes = d["passes"]
    # within a stream, a chunk's passes and the chunks follow one another
    for s in (0, 1):
        mine = [t[i] for i in range(len(t)) if (i // passes) % 2 == s]
        assert all(v > 0 for v in mine) and mine == sorted(mine), (s, t)
    out = np.empty_like(x)
    b.copy_to_host(out)
    ref, _ = _run(gpu_device, x, log_n, batch)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    plan.destroy()


def test_two_stream_plan_in_a_graph_runs_on_the_captured_stream(gpu_device, chunk_limit):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    log_n, batch = 20, 6
    n = 1 << log_n
    chunk_limit(2 * n * 8)
    x = normal_c64(np.random.default_rng(8), batch * n)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    assert plan.describe()["streams"] == 2
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


def test_two_stream_split_layout(gpu_device, chunk_limit):
    # the split path interleaves on the caller's stream, runs the two-stream
    # execution in place and deinterleaves after the join
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    log_n, batch = 17, 5
    n = 1 << log_n
    chunk_limit(2 * n * 8)
    x = normal_c64(np.random.default_rng(21), batch * n)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    assert plan.describe()["streams"] == 2
    bufs = [DeviceBuffer(gpu_device, 4 * batch * n) for _ in range(4)]
    bufs[0].copy_from_host(np.ascontiguousarray(x.real))
    bufs[1].copy_from_host(np.ascontiguousarray(x.imag))
    plan.execute_split(*bufs, "forward", False)
    gpu_device.sync()
    re, im = np.empty(batch * n, np.float32), np.empty(batch * n, np.float32)
    bufs[2].copy_to_host(re)
    bufs[3].copy_to_host(im)
    ref, _ = _run(gpu_device, x, log_n, batch)
    assert np.array_equal(re.view(np.uint32), np.ascontiguousarray(ref.real).view(np.uint32))
    assert np.array_equal(im.view(np.uint32), np.ascontiguousarray(ref.imag).view(np.uint32))
    plan.destroy()


def test_which_plans_take_two_streams(gpu_device, chunk_limit):
    import ferrum_gpu

    chunk_limit(256 << 20)
    assert ferrum_gpu.fft.Plan1D(24, 4, gpu_device).describe()["streams"] == 2   # config 4: four chunks
    assert ferrum_gpu.fft.Plan1D(24, 1, gpu_device).describe()["streams"] == 1   # one chunk
    assert ferrum_gpu.fft.Plan1D(10, 65536, gpu_device).describe()["streams"] == 1   # single pass
    assert ferrum_gpu.fft.Plan2D(12, 4, gpu_device).describe()["streams"] == 1   # narrow column tiles
    # every 2D plan runs one stream: 256 x 256 x 1024 (512 MiB) in two chunks
    # of 256 MiB with the wide 32-column tiles exchanging in halves
    p2 = ferrum_gpu.fft.Plan2D(8, 1024, gpu_device)
    d2 = p2.describe()
    assert d2["streams"] == 1 and d2["chunks"] == 2 and p2.kernel_names()[1] == "fg_tile_l8_g32_h_cs"
    assert ferrum_gpu.fft.Plan2D(9, 2048, gpu_device, log_cols=6).describe()["streams"] == 1
    assert ferrum_gpu.fft.Plan2D(4, 2048, gpu_device, log_cols=11).describe()["streams"] == 1
    # 2^17 = 256 x 512: one chunk keeps the 8-row last pass on one stream,
    # two or more take 16-row tiles (exchanging in halves) and two streams
    one = ferrum_gpu.fft.Plan1D(17, 1, gpu_device)
    assert one.describe()["streams"] == 1 and one.kernel_names()[-1] == "fg_tile_l9_g8_r_cc"
    many = ferrum_gpu.fft.Plan1D(17, 512, gpu_device)
    assert many.describe()["streams"] == 2 and many.kernel_names()[-1] == "fg_tile_l9_g16_rh_cs"
    # 2^18 = 256 x 1024: the 1024-point last pass (16 rows, exchanges in halves)
    assert ferrum_gpu.fft.Plan1D(18, 256, gpu_device).kernel_names()[:2] == ["fg_tile_l8_g32_h_sc", "fg_tile_l10_g16_rh_cs"]


def test_two_stream_plan_behind_the_host_array_path(gpu_device, chunk_limit):
    # fft_1d_c2c_pow2 on host arrays: staging copies on the device stream
    # around a plan whose chunks alternate over two streams
    import ferrum_gpu

    log_n, batch = 16, 9
    n = 1 << log_n
    chunk_limit(2 * n * 8)
    x = normal_c64(np.random.default_rng(99), batch * n)
    for direction, normalize in (("forward", False), ("inverse", True)):
        got = ferrum_gpu.fft.fft_1d_c2c_pow2(x, log_n, direction, normalize, device=gpu_device)
        want = oracle.fft_1d(x, log_n, direction, normalize, threads=8)
        assert rel_l2(got, want) <= TOL


# 2D (log rows, log cols, batch, images per chunk): every 2D plan runs one
# stream, in chunks of the whole limit; chunked and unchunked, the same bits
CASES_2D = [(8, 8, 7, 2), (5, 10, 5, 2), (9, 7, 3, 1), (7, 12, 2, 1), (10, 8, 5, 2), (10, 12, 3, 1)]


@pytest.mark.parametrize("lr,lc,batch,per_chunk", CASES_2D)
def test_2d_plans_run_one_stream_in_every_chunking(gpu_device, chunk_limit, lr, lc, batch, per_chunk):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer
    from test_gpu_extras import oracle_2d_rect

    image = 8 << (lr + lc)
    x = normal_c64(np.random.default_rng(lr * 16 + lc), batch * (image // 8)).reshape(batch, 1 << lr, 1 << lc)
    outs = []
    for limit, chunks in ((per_chunk * image, -(-batch // per_chunk)), (batch * image, 1)):
        chunk_limit(limit)
        print(f"[case] 2d {1 << lr}x{1 << lc} batch={batch} chunk limit={limit}", flush=True)
        plan = ferrum_gpu.fft.Plan2D(lr, batch, gpu_device, log_cols=lc)
        d = plan.describe()
        assert d["streams"] == 1 and d["chunks"] == chunks
        a, b = DeviceBuffer(gpu_device, plan.nbytes), DeviceBuffer(gpu_device, plan.nbytes)
        a.copy_from_host(x)
        plan.execute(a, b, "forward")
        plan.execute(b, a, "inverse", True)
        gpu_device.sync()
        fwd, back = np.empty_like(x), np.empty_like(x)
        b.copy_to_host(fwd)
        a.copy_to_host(back)
        outs.append((fwd, back))
        plan.destroy()
    assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
    assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))
    assert rel_l2(outs[0][0], oracle_2d_rect(x, lr, lc)) <= TOL
    assert rel_l2(outs[0][1], x) <= TOL


def test_set_streams_one_and_back_same_bits(gpu_device, chunk_limit):
    # set_streams(1) runs the two-stream plan's chunks on the caller's stream
    # alone (the bench's per-pass figures), set_streams(2) restores the
    # overlap; the output is the same bits every way, and the chunk stream is
    # one per device, shared by every two-stream plan
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer

    log_n, batch = 20, 4
    n = 1 << log_n
    chunk_limit(2 * n * 8)
    x = normal_c64(np.random.default_rng(91), batch * n)
    print("[case] set_streams 2 -> 1 -> 2, log_n=20 batch=4", flush=True)
    plan = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    other = ferrum_gpu.fft.Plan1D(log_n, batch, gpu_device)
    assert plan.describe()["streams"] == 2 and other.describe()["streams"] == 2
    a, b = DeviceBuffer(gpu_device, plan.nbytes), DeviceBuffer(gpu_device, plan.nbytes)
    a.copy_from_host(x)
    outs = []
    for streams, p in ((2, plan), (1, plan), (2, plan), (2, other)):
        p.set_streams(streams)
        assert p.describe()["streams"] == streams
        for direction, normalize in (("forward", False), ("inverse", True)):
            p.execute(a, b, direction, normalize)
            gpu_device.sync()
            o = np.empty_like(x)
            b.copy_to_host(o)
            outs.append(o)
    for i, o in enumerate(outs):   # forward, inverse, forward, inverse, ...
        assert np.array_equal(o.view(np.uint32), outs[i % 2].view(np.uint32)), i
    assert _lanes(outs[0], x, log_n, batch) <= TOL
    # one-stream plans refuse a second stream; bad values are refused
    single = ferrum_gpu.fft.Plan1D(10, 64, gpu_device)
    with pytest.raises(Exception):
        single.set_streams(2)
    with pytest.raises(Exception):
        plan.set_streams(3)
    single.set_streams(1)
    for p in (plan, other, single):
        p.destroy()
    a.free()
    b.free()

"""Per-launch timing events (fg_fft_exec_events / Plan*.execute_recording).

Each event is stamped by its launch's dispatch, so a recorded execution must
compute exactly what fg_fft_exec computes (bit-identical output), stamp its
events in launch order, and refuse an event count that is not the plan's
launch count.  Events may be passed as a list or as a prebuilt EventList.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rel_l2, uniform_c64

pytestmark = pytest.mark.gpu

MIB = 1 << 20


@pytest.fixture
def chunk_limit():
    import ferrum_gpu

    saved = ferrum_gpu.fft.get_chunk_bytes()
    yield ferrum_gpu.fft.set_chunk_bytes
    ferrum_gpu.fft.set_chunk_bytes(saved)


# (two_d, log_n, batch, chunk MiB): one launch; two and three passes; chunked
CASES = [
    (False, 10, 64, 128),
    (False, 14, 16, 128),
    (False, 21, 2, 128),
    (False, 16, 48, 1),
    (True, 8, 12, 1),
]


@pytest.mark.parametrize("two_d,log_n,batch,chunk_mib", CASES)
@pytest.mark.parametrize("as_list", [True, False], ids=["list", "EventList"])
def test_recorded_execution_equals_plain(gpu_device, chunk_limit, two_d, log_n, batch, chunk_mib, as_list):
    import ferrum_gpu
    from ferrum_gpu.hip import DeviceBuffer, Event, EventList

    chunk_limit(chunk_mib * MIB)
    plan = (ferrum_gpu.fft.Plan2D if two_d else ferrum_gpu.fft.Plan1D)(log_n, batch, gpu_device)
    launches = plan.describe()["launches"]
    assert launches >= 1
    elems = plan.elems
    rng = np.random.default_rng(log_n * 31 + batch)
    x = uniform_c64(rng, batch * elems)
    a, b, c = (DeviceBuffer(gpu_device, plan.nbytes) for _ in range(3))
    a.copy_from_host(x)

    plan.execute(a, b, "forward")
    start = Event(gpu_device)
    evs = [Event(gpu_device) for _ in range(launches)]
    arg = evs if as_list else EventList(evs)
    start.record(gpu_device.default_stream)
    plan.execute_recording(a, c, arg, "forward", stream=gpu_device.default_stream)
    gpu_device.sync()

    plain, rec = np.empty_like(x), np.empty_like(x)
    b.copy_to_host(plain)
    c.copy_to_host(rec)
    assert np.array_equal(plain.view(np.uint64), rec.view(np.uint64))
    if two_d:
        n = 1 << log_n
        want = oracle.fft_2d(x.reshape(batch, n, n), log_n).reshape(-1)
    else:
        want = oracle.fft_1d(x, log_n)
    assert rel_l2(rec, want) < 1e-4

    # launch order: every launch took a non-negative time after the previous
    # stamp on its stream (two-stream plans: odd chunks on the plan's own)
    d = plan.describe()
    streams, passes = d["streams"], d["passes"]
    for s in range(streams):
        mine = [e for i, e in enumerate(evs) if streams == 1 or (i // passes) % 2 == s]
        prev, total = start, 0.0
        for e in mine:
            dt = prev.elapsed_ms(e)
            assert dt >= 0.0
            total += dt
            prev = e
        assert start.elapsed_ms(mine[-1]) == pytest.approx(total, rel=1e-3, abs=1e-3)
    plan.destroy()


def test_event_count_must_match_launches(gpu_device):
    import ferrum_gpu
    from ferrum_gpu._native import FerrumGpuError
    from ferrum_gpu.hip import DeviceBuffer, Event, EventList

    plan = ferrum_gpu.fft.Plan1D(14, 4, gpu_device)
    launches = plan.describe()["launches"]
    a = DeviceBuffer(gpu_device, plan.nbytes)
    for n in (launches - 1, launches + 1):
        evs = [Event(gpu_device) for _ in range(n)]
        with pytest.raises(FerrumGpuError, match=f"need {launches} events, got {n}"):
            plan.execute_recording(a, a, EventList(evs))
    with pytest.raises(TypeError):
        EventList([object()])
    plan.destroy()

"""Finalizers of the Python package during a stream capture (no GPU needed).

A HIP free (buffer, stream, event, graph, plan, module, device) made while a
capture is open on the thread would end that capture invalid, and Python's
garbage collector runs finalizers at any point.  ``ferrum_gpu.hip.Capture``
therefore holds the release calls of objects finalized inside its block and
makes them when the thread's outermost block ends, also when the block raises.
The native library is replaced by a recorder here, so nothing touches a GPU.
"""

from __future__ import annotations

import ctypes

import pytest

import ferrum_gpu
from ferrum_gpu import hip


class _Recorder:
    """Stands in for the native library: records the calls the tests expect."""

    def __init__(self):
        self.calls = []

    def fg_graph_capture_begin(self, dev, stream_out):
        self.calls.append("begin")
        return 0

    def fg_graph_capture_end(self, dev, stream, graph_out):
        self.calls.append("end")
        return 0

    def fg_free(self, dev, p):
        self.calls.append(("free", p.value))
        return 0

    def fg_event_destroy(self, e):
        self.calls.append(("event", e.value))
        return 0

    def fg_fft_plan_destroy(self, p):
        self.calls.append(("plan", p.value))
        return 0

    def fg_graph_destroy(self, g):
        self.calls.append(("graph", g.value))
        return 0


class _Dev:
    handle = ctypes.c_void_p(0x10)


@pytest.fixture
def rec(monkeypatch):
    r = _Recorder()
    monkeypatch.setattr(hip._n, "lib", r)
    return r


def _buffer(addr):
    b = object.__new__(hip.DeviceBuffer)
    b.device = _Dev()
    b.nbytes = 8
    b._p = ctypes.c_void_p(addr)
    return b


def test_buffer_released_after_the_capture(rec):
    with hip.Capture(_Dev()):
        b = _buffer(0x1000)
        del b
        assert ("free", 0x1000) not in rec.calls
    assert rec.calls == ["begin", "end", ("free", 0x1000)]


def test_release_outside_a_capture_is_immediate(rec):
    b = _buffer(0x2000)
    del b
    assert rec.calls == [("free", 0x2000)]


def test_nested_captures_release_after_the_outermost(rec):
    with hip.Capture(_Dev()):
        with hip.Capture(_Dev()):
            e = object.__new__(hip.Event)
            e._e = ctypes.c_void_p(0x30)
            del e
        assert ("event", 0x30) not in rec.calls
    assert rec.calls[-1] == ("event", 0x30)


def test_release_runs_when_the_block_raises(rec):
    with pytest.raises(RuntimeError):
        with hip.Capture(_Dev()):
            b = _buffer(0x4000)
            del b
            raise RuntimeError("inside the capture")
    assert rec.calls[-1] == ("free", 0x4000)


def test_plan_and_graph_released_in_order(rec):
    # a graph keeps its plan alive: the graph is destroyed first, then the plan
    with hip.Capture(_Dev()):
        p = object.__new__(ferrum_gpu.fft.Plan1D)
        p._p = ctypes.c_void_p(0x50)
        g = hip.Graph(_Dev(), ctypes.c_void_p(0x60), keep=[p])
        del p
        assert not any(c[0] == "plan" for c in rec.calls if isinstance(c, tuple))
        del g
    assert rec.calls[-2:] == [("graph", 0x60), ("plan", 0x50)]


def test_released_objects_are_not_released_twice(rec):
    with hip.Capture(_Dev()):
        b = _buffer(0x7000)
        b.__del__()
        del b
    assert rec.calls.count(("free", 0x7000)) == 1

"""ferrum_gpu.hip -- the device handle and the substrate objects over HIP.

``Device`` is the HIP counterpart of the reference's ``ferrum_gpu.cuda.Device``
(crates/ferrum-gpu-py/src/lib.rs:389-417, python/ferrum_gpu/cuda.py): construct
once, pass as ``device=`` to the FFT functions, ``sync()`` the default stream.
``DeviceBuffer``, ``Event``, ``Module`` and ``Kernel`` expose the rest of the
Backend contract (crates/ferrum-gpu-core/src/backend.rs:12-77) for
device-resident work and for the bench.
"""

from __future__ import annotations

import ctypes
import gc
import threading

import numpy as np

from ferrum_gpu import _native as _n

__all__ = ["Device", "DeviceBuffer", "Event", "EventList", "Stream", "Graph", "Capture", "Module", "Kernel",
           "device_count"]


# A finalizer that frees a HIP object (memory, stream, event, graph, plan,
# module, device) while a Capture block is open on its thread would make a
# call a stream capture cannot record, and the capture would end invalid.  The
# garbage collector and dropped references run finalizers at any point, so
# while a block is open their release calls wait in a list and run when the
# thread's last block ends.
_capture_state = threading.local()


def _release(fn, *args) -> None:
    """A finalizer's release call: now, or after the Capture blocks open on
    this thread have ended."""
    if getattr(_capture_state, "depth", 0) > 0:
        _capture_state.deferred.append((fn, args))
    else:
        fn(*args)


def device_count() -> int:
    c = ctypes.c_int(0)
    _n.check(_n.lib.fg_device_count(ctypes.byref(c)))
    return c.value


class Device:
    """A GPU with its default stream and loaded FFT code object."""

    def __init__(self, ordinal: int = 0):
        h = ctypes.c_void_p()
        rc = _n.lib.fg_device_open(int(ordinal), ctypes.byref(h))
        if rc != _n.FG_OK:
            # crates/ferrum-gpu-py/src/lib.rs:403-406 reports ValueError.
            raise ValueError(f"Device::new({ordinal}): {_n.last_error()}")
        self._h = h
        self.ordinal = int(ordinal)

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise ValueError("device is closed")
        return self._h

    def sync(self) -> None:
        """Synchronise the default stream (lib.rs:410-416)."""
        rc = _n.lib.fg_device_sync(self.handle)
        if rc != _n.FG_OK:
            raise ValueError(f"sync: {_n.last_error()}")

    @property
    def default_stream(self) -> int:
        s = ctypes.c_void_p()
        _n.check(_n.lib.fg_device_default_stream(self.handle, ctypes.byref(s)))
        return s.value or 0

    def info(self) -> dict:
        arch = ctypes.create_string_buffer(64)
        cu, mem, clk = ctypes.c_int(), ctypes.c_size_t(), ctypes.c_int()
        _n.check(_n.lib.fg_device_info(self.handle, arch, 64, ctypes.byref(cu), ctypes.byref(mem),
                                       ctypes.byref(clk)))
        return {"arch": arch.value.decode(), "cu_count": cu.value, "total_mem": mem.value,
                "clock_khz": clk.value}

    def close(self) -> None:
        """Release the device; refused (FerrumGpuError) while plans or graphs
        made on it are alive."""
        if getattr(self, "_h", None) is not None:
            _n.check(_n.lib.fg_device_close(self._h))
            self._h = None

    def __del__(self):  # pragma: no cover - interpreter teardown order
        try:
            if getattr(self, "_h", None) is not None:
                _release(_n.lib.fg_device_close, self._h)
                self._h = None
        except Exception:
            pass

    def __repr__(self) -> str:
        return f"ferrum_gpu.hip.Device({self.ordinal})"


class DeviceBuffer:
    """A zero-initialised device allocation (Buffer<T, B>, crates/ferrum-gpu/src/buffer.rs:8-47)."""

    def __init__(self, device: Device, nbytes: int):
        self.device = device
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _n.check(_n.lib.fg_alloc_zeros(device.handle, self.nbytes, ctypes.byref(p)))
        self._p = p

    @property
    def ptr(self) -> int:
        return self._p.value or 0

    def copy_from_host(self, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        if a.nbytes > self.nbytes:
            raise ValueError("copy_from_host: source longer than the buffer")
        _n.check(_n.lib.fg_copy_h2d(self.device.handle, self._p, a.ctypes.data, a.nbytes))

    def copy_to_host(self, out: np.ndarray) -> np.ndarray:
        if not out.flags.c_contiguous or out.nbytes > self.nbytes:
            raise ValueError("copy_to_host: destination must be contiguous and fit the buffer")
        _n.check(_n.lib.fg_copy_d2h(self.device.handle, out.ctypes.data, self._p, out.nbytes))
        return out

    def free(self) -> None:
        if getattr(self, "_p", None) is not None and self._p.value:
            _n.lib.fg_free(self.device.handle, self._p)
        self._p = ctypes.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            if getattr(self, "_p", None) is not None and self._p.value:
                # the device object rides along, so it outlives a deferred free
                _release(lambda dev, p: _n.lib.fg_free(dev.handle, p), self.device, self._p)
                self._p = ctypes.c_void_p()
        except Exception:
            pass


class Stream:
    """A stream of the device at the default priority (Backend stream handle,
    crates/ferrum-gpu-core/src/backend.rs:73-76); ``handle`` is what the
    ``stream=`` arguments take."""

    def __init__(self, device: Device):
        s = ctypes.c_void_p()
        _n.check(_n.lib.fg_stream_create(device.handle, ctypes.byref(s)))
        self.device = device
        self._s = s

    @property
    def handle(self) -> int:
        return self._s.value or 0

    def sync(self) -> None:
        _n.check(_n.lib.fg_stream_sync(self.device.handle, self._s))

    def destroy(self) -> None:
        """Waits for the stream's work, then destroys it."""
        if getattr(self, "_s", None) is not None and self._s.value:
            _n.check(_n.lib.fg_stream_destroy(self.device.handle, self._s))
        self._s = ctypes.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            if getattr(self, "_s", None) is not None and self._s.value:
                _release(lambda dev, st: _n.lib.fg_stream_destroy(dev.handle, st), self.device, self._s)
                self._s = ctypes.c_void_p()
        except Exception:
            pass


class Graph:
    """An executable HIP graph: a captured sequence of stream-ordered calls
    replayed by ``launch`` with one submission.  ``keep`` holds the objects
    (plans) the recorded calls use, so they outlive the graph."""

    def __init__(self, device: Device, handle: ctypes.c_void_p, keep=()):
        self.device = device
        self._g = handle
        self._keep = tuple(keep)

    def launch(self, stream: int = 0) -> None:
        """Enqueue one replay on ``stream`` (0: the device default stream)."""
        if not self._g.value:
            raise ValueError("graph is destroyed")
        _n.check(_n.lib.fg_graph_launch(self._g, ctypes.c_void_p(stream or None)))

    @property
    def node_count(self) -> int:
        n = ctypes.c_size_t()
        _n.check(_n.lib.fg_graph_node_count(self._g, ctypes.byref(n)))
        return n.value

    def destroy(self) -> None:
        """Waits for the device's work, then frees the graph."""
        if getattr(self, "_g", None) is not None and self._g.value:
            _n.check(_n.lib.fg_graph_destroy(self._g))
        self._g = ctypes.c_void_p()
        self._keep = ()

    def __del__(self):  # pragma: no cover
        try:
            if getattr(self, "_g", None) is not None and self._g.value:
                # the kept plans ride along, so they outlive a deferred destroy
                _release(lambda g, keep: _n.lib.fg_graph_destroy(g), self._g, self._keep)
                self._g = ctypes.c_void_p()
                self._keep = ()
        except Exception:
            pass


class Capture:
    """Records the stream-ordered calls made on ``stream`` inside the block
    into a Graph instead of running them::

        with Capture(dev, keep=[plan]) as cap:
            plan.execute(a, b, "forward", stream=cap.stream)
            plan.execute(b, c, "inverse", True, stream=cap.stream)
        cap.graph.launch()

    Calls must come from the capturing thread; the caller keeps the buffers
    the recorded calls use alive while the graph is launched.  Objects of
    this package that are garbage-collected inside the block release their
    HIP resources when the block ends (a release inside it would end the
    capture invalid); explicit ``free`` / ``destroy`` / ``close`` calls inside
    the block are the caller's to avoid."""

    def __init__(self, device: Device, keep=()):
        self.device = device
        self._keep = tuple(keep)
        self._s = ctypes.c_void_p()
        self.graph: Graph | None = None

    @property
    def stream(self) -> int:
        return self._s.value or 0

    def __enter__(self) -> "Capture":
        gc.collect()  # garbage already unreachable is released before the capture begins
        _n.check(_n.lib.fg_graph_capture_begin(self.device.handle, ctypes.byref(self._s)))
        if getattr(_capture_state, "depth", 0) == 0:
            _capture_state.deferred = []
        _capture_state.depth = getattr(_capture_state, "depth", 0) + 1
        return self

    def __exit__(self, exc_type, exc, tb) -> bool:
        g = ctypes.c_void_p()
        try:
            rc = _n.lib.fg_graph_capture_end(self.device.handle, self._s, ctypes.byref(g))
        finally:
            self._s = ctypes.c_void_p()
            _capture_state.depth -= 1
            if _capture_state.depth == 0:
                deferred, _capture_state.deferred = _capture_state.deferred, []
                for fn, args in deferred:
                    try:
                        fn(*args)
                    except Exception:
                        pass
        if exc_type is not None:
            if rc == _n.FG_OK and g.value:
                _n.lib.fg_graph_destroy(g)
            return False
        _n.check(rc)
        self.graph = Graph(self.device, g, self._keep)
        return False


class Event:
    """A HIP event for stream-ordered timing."""

    def __init__(self, device: Device):
        e = ctypes.c_void_p()
        _n.check(_n.lib.fg_event_create(device.handle, ctypes.byref(e)))
        self._e = e

    def record(self, stream: int = 0) -> None:
        _n.check(_n.lib.fg_event_record(self._e, ctypes.c_void_p(stream or None)))

    def synchronize(self) -> None:
        _n.check(_n.lib.fg_event_sync(self._e))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _n.check(_n.lib.fg_event_elapsed_ms(self._e, end._e, ctypes.byref(ms)))
        return ms.value

    def __del__(self):  # pragma: no cover
        try:
            _release(_n.lib.fg_event_destroy, self._e)
        except Exception:
            pass


class EventList:
    """Events with their handle array built once, so that a loop which passes
    them to ``Plan*.execute_recording`` call after call does no per-call
    marshalling (a few microseconds of host time per call)."""

    def __init__(self, events):
        self.events = list(events)
        for e in self.events:
            if not isinstance(e, Event):
                raise TypeError("EventList holds ferrum_gpu.hip.Event objects")
        self.handles = (ctypes.c_void_p * len(self.events))(*[e._e.value for e in self.events])

    def __len__(self) -> int:
        return len(self.events)

    def __getitem__(self, i):
        return self.events[i]


class Kernel:
    def __init__(self, module: "Module", name: str):
        k = ctypes.c_void_p()
        _n.check(_n.lib.fg_kernel_get(module._m, name.encode(), ctypes.byref(k)))
        self._k = k
        self.module = module
        self.name = name

    def launch(self, grid, block, args, shared_bytes: int = 0, stream: int = 0) -> None:
        """Backend::launch: ``args`` is a list of ctypes scalars (c_void_p for pointers)."""
        g = (ctypes.c_uint32 * 3)(*(list(grid) + [1, 1, 1])[:3])
        b = (ctypes.c_uint32 * 3)(*(list(block) + [1, 1, 1])[:3])
        ptrs = (ctypes.c_void_p * len(args))(*[ctypes.cast(ctypes.pointer(a), ctypes.c_void_p) for a in args])
        _n.check(_n.lib.fg_launch(self.module.device.handle, ctypes.c_void_p(stream or None), self._k, g, b,
                                  shared_bytes, ptrs))


class Module:
    """A loaded code object (Backend::load_module)."""

    def __init__(self, device: Device, image: bytes | None = None, backend_id: int = _n.FG_BACKEND_HIP):
        self.device = device
        m = ctypes.c_void_p()
        if image is None:
            _n.check(_n.lib.fg_device_fft_module(device.handle, ctypes.byref(m)))
        else:
            self._image = ctypes.create_string_buffer(bytes(image), len(image))
            _n.check(_n.lib.fg_module_load(device.handle, backend_id, self._image, len(image), ctypes.byref(m)))
        self._m = m

    def kernel(self, name: str) -> Kernel:
        return Kernel(self, name)

    def __del__(self):  # pragma: no cover
        try:
            # the device and the image ride along, so they outlive a deferred unload
            _release(lambda m, dev, image: _n.lib.fg_module_unload(m), self._m, self.device,
                     getattr(self, "_image", None))
        except Exception:
            pass

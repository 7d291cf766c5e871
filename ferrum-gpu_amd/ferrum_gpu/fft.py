"""ferrum_gpu.fft -- batched power-of-two C2C complex64 FFTs on MI355X.

``fft_1d_c2c_pow2`` and ``fft_2d_c2c_pow2`` keep the reference's signatures,
argument meaning and error messages (crates/ferrum-gpu-py/src/lib.rs:425-588).
Two deliberate widenings: 1D accepts ``log_n`` up to 24 (the reference stops at
12, lib.rs:455-459), and 2D also accepts a ``(B, N, N)`` stack of images.

``Plan1D`` / ``Plan2D`` are the device-resident form: plan once, then execute
on device buffers with no host copies (what the bench measures).
"""

from __future__ import annotations

import ctypes
import operator

import numpy as np

from ferrum_gpu import _native as _n
from ferrum_gpu.hip import Device, DeviceBuffer, EventList, Graph, _release

__all__ = ["fft_1d_c2c_pow2", "fft_2d_c2c_pow2", "fft2_c2c_pow2", "Plan1D", "Plan2D", "Graph", "transpose",
           "set_chunk_bytes", "get_chunk_bytes", "MIN_LOG_N", "MAX_LOG_N", "MIN_LOG_N_2D", "MAX_LOG_N_2D"]

MIN_LOG_N, MAX_LOG_N = 2, 24
MIN_LOG_N_2D, MAX_LOG_N_2D = 4, 12


def _as_u32(log_n) -> int:
    # PyO3 extracts log_n as u32: non-integers raise TypeError, negatives OverflowError.
    try:
        v = operator.index(log_n)
    except TypeError:
        raise TypeError(f"argument 'log_n': '{type(log_n).__name__}' object cannot be interpreted as an integer")
    if v < 0 or v > 0xFFFFFFFF:
        raise OverflowError("argument 'log_n': can't convert to u32")
    return v


_DIRECTIONS = {"forward": _n.FG_FORWARD, "inverse": _n.FG_INVERSE}


def _direction(direction) -> int:
    # `direction: &str` (lib.rs:451, 533): PyO3 0.23 refuses anything but a
    # str with a TypeError before the function body runs.
    if not isinstance(direction, str):
        raise TypeError(f"argument 'direction': '{type(direction).__name__}' object cannot be converted to "
                        "'PyString'")
    try:
        return _DIRECTIONS[direction]
    except KeyError:
        pass
    # Rust formats the offending string with {:?} (double-quoted), lib.rs:472-476.
    raise ValueError(f"direction must be 'forward' or 'inverse', got \"{direction}\"")


def _normalize(normalize) -> int:
    # `normalize: bool` (lib.rs:452, 534): PyO3 0.23 extracts Python bool and
    # numpy.bool_ only; anything else (0, 1, "yes", None) is a TypeError.
    if isinstance(normalize, (bool, np.bool_)):
        return 1 if normalize else 0
    raise TypeError(f"argument 'normalize': '{type(normalize).__name__}' object cannot be converted to 'PyBool'")


def _device_handle(device):
    if device is None:
        return None
    if not isinstance(device, Device):
        # `device: Option<PyRef<Device>>` (lib.rs:453, 535).
        raise TypeError(f"argument 'device': '{type(device).__name__}' object cannot be converted to 'Device'")
    return device.handle


def _complex64_array(arr, ndims: tuple[int, ...]) -> np.ndarray:
    # PyReadonlyArray{1,2}<Complex32> extraction: a complex64 ndarray of the
    # right rank (lib.rs:449, 531).  Contiguity is checked later, where the
    # body calls as_slice() (_contiguous).
    if not isinstance(arr, np.ndarray):
        raise TypeError(f"argument 'arr': '{type(arr).__name__}' object cannot be converted to 'PyArray'")
    if arr.dtype != np.complex64:
        raise TypeError(f"argument 'arr': type mismatch: from={arr.dtype}, to=complex64")
    if arr.ndim not in ndims:
        raise TypeError(f"argument 'arr': dimensionality mismatch: from={arr.ndim}, to={ndims[0]}")
    return arr


def _contiguous(a: np.ndarray) -> None:
    # arr.as_slice()? (lib.rs:461, 560): numpy's NotContiguousError, a TypeError.
    if not a.flags.c_contiguous:
        raise TypeError("The given array is not contiguous")


def fft_1d_c2c_pow2(arr, log_n, direction="forward", normalize=False, device=None):
    """FFT of a 1D ``complex64`` numpy array of length ``batch * 2**log_n``.

    Arguments mirror crates/ferrum-gpu-py/src/lib.rs:425-444: ``direction`` is
    "forward" (default) or "inverse"; ``normalize`` scales the inverse by 1/N;
    ``device`` is an optional persistent :class:`ferrum_gpu.hip.Device`.
    Returns a new ``complex64`` array of the same length.

    Checks run in the reference's order: argument extraction (TypeError) for
    every argument first, then the body's checks (lib.rs:455-477).
    """
    a = _complex64_array(arr, (1,))
    log_n = _as_u32(log_n)
    if not isinstance(direction, str):
        _direction(direction)
    norm = _normalize(normalize)
    h = _device_handle(device)
    if not (MIN_LOG_N <= log_n <= MAX_LOG_N):
        raise ValueError(f"log_n must be in [{MIN_LOG_N}, {MAX_LOG_N}], got {log_n}")
    n = 1 << log_n
    _contiguous(a)
    total = a.size
    if total == 0 or total % n != 0:
        raise ValueError(f"arr len {total} must be a positive multiple of N = {n}")
    d = _direction(direction)
    out = np.empty_like(a)
    rc = _n.lib.fg_fft_1d_c2c_pow2_host(h, a.ctypes.data, out.ctypes.data, total, log_n, d, norm)
    if rc != _n.FG_OK:
        raise ValueError(f"ferrum-gpu fft error: {_n.last_error()}")
    return out


def fft_2d_c2c_pow2(arr, log_n, direction="forward", normalize=False, device=None):
    """2D FFT of a square ``complex64`` array of shape ``(N, N)`` (or ``(B, N, N)``).

    Arguments mirror crates/ferrum-gpu-py/src/lib.rs:506-526; ``normalize``
    scales the inverse by 1/(N*N).  Returns a new array of the same shape.
    Checks run in the reference's order (argument extraction, then
    lib.rs:537-560).
    """
    a = _complex64_array(arr, (2, 3))
    log_n = _as_u32(log_n)
    if not isinstance(direction, str):
        _direction(direction)
    norm = _normalize(normalize)
    h = _device_handle(device)
    if not (MIN_LOG_N_2D <= log_n <= MAX_LOG_N_2D):
        raise ValueError(f"2D requires log_n in [{MIN_LOG_N_2D}, {MAX_LOG_N_2D}]; got {log_n}")
    n = 1 << log_n
    dims = list(a.shape)
    if dims[-2:] != [n, n] or (a.ndim == 3 and dims[0] == 0):
        raise ValueError(f"arr shape {dims} != ({n}, {n})")
    d = _direction(direction)
    _contiguous(a)
    batch = 1 if a.ndim == 2 else dims[0]
    out = np.empty_like(a)
    rc = _n.lib.fg_fft_2d_c2c_pow2_host(h, a.ctypes.data, out.ctypes.data, log_n, batch, d, norm)
    if rc != _n.FG_OK:
        raise ValueError(f"ferrum-gpu fft 2d error: {_n.last_error()}")
    return out


def _ptr(x):
    """A device address for a void* parameter from a DeviceBuffer (its own
    c_void_p, which ctypes passes without converting), a GPU torch tensor or
    an int."""
    if isinstance(x, DeviceBuffer):
        return x._p
    if hasattr(x, "data_ptr"):  # a torch tensor on the GPU
        return x.data_ptr()
    return int(x)


def _ptr_sized(x, need: int, what: str):
    """_ptr(x), refusing a DeviceBuffer or tensor smaller than ``need`` bytes:
    the kernels would read and write past its end.  A raw address cannot be
    checked; the caller vouches for it."""
    if isinstance(x, DeviceBuffer):
        if x.nbytes < need:
            raise ValueError(f"{what}: buffer of {x.nbytes} bytes, the plan reads or writes {need}")
        return x._p
    if hasattr(x, "data_ptr"):
        have = x.numel() * x.element_size()
        if have < need or not x.is_contiguous():
            raise ValueError(f"{what}: tensor of {have} bytes (contiguous: {x.is_contiguous()}), the plan "
                             f"reads or writes {need} contiguous bytes")
        return x.data_ptr()
    return int(x)


# Bound once: the per-call cost of the device-resident entry points is host
# time that launch-bound callers (small batches) pay on every call.
_fft_exec = _n.lib.fg_fft_exec
_fft_exec_events = _n.lib.fg_fft_exec_events


class _Plan:
    def __init__(self, device: Device, handle: ctypes.c_void_p, elems: int, batch: int):
        self.device = device
        self._p = handle
        self.elems = elems
        self.batch = batch
        self._nbytes = batch * elems * 8

    @property
    def nbytes(self) -> int:
        """Bytes of one input (or output) buffer: batch * elems * 8."""
        return self.batch * self.elems * 8

    def execute(self, d_in, d_out, direction="forward", normalize=False, stream: int = 0) -> None:
        """Stream-ordered, asynchronous execution on device buffers: equal (in
        place) or disjoint, 8-byte aligned."""
        nb = self._nbytes
        rc = _fft_exec(self._p, _ptr_sized(d_in, nb, "d_in"), _ptr_sized(d_out, nb, "d_out"), _direction(direction),
                       1 if normalize else 0, stream or None)
        if rc:
            _n.check(rc)

    def execute_recording(self, d_in, d_out, events, direction="forward", normalize=False,
                          stream: int = 0) -> None:
        """execute() that records events[i] right after launch i (len(events) ==
        launches), without synchronising; launch i ran between the previous event
        recorded on the stream and events[i].  ``events`` is a sequence of
        Event or a prebuilt ``hip.EventList``."""
        if isinstance(events, EventList):
            arr = events.handles
        else:
            arr = (ctypes.c_void_p * len(events))(*[e._e.value for e in events])
        nb = self._nbytes
        rc = _fft_exec_events(self._p, _ptr_sized(d_in, nb, "d_in"), _ptr_sized(d_out, nb, "d_out"),
                              _direction(direction), 1 if normalize else 0, stream or None, arr, len(arr))
        if rc:
            _n.check(rc)

    def execute_split(self, in_re, in_im, out_re, out_im, direction="forward", normalize=False,
                      stream: int = 0) -> None:
        """execute() on the split layout: real and imaginary parts in separate
        float32 device arrays of ``batch * elems`` each (the reference's *_split
        kernels).  out_re/out_im may be in_re/in_im; stream-ordered."""
        d = _direction(direction)
        half = self._nbytes // 2
        ptrs = [_ptr_sized(b, half, name) for b, name in
                ((in_re, "in_re"), (in_im, "in_im"), (out_re, "out_re"), (out_im, "out_im"))]
        _n.check(_n.lib.fg_fft_exec_split(self._p, *ptrs, d, int(bool(normalize)), ctypes.c_void_p(stream or None)))

    def execute_split_noalloc(self, in_re, in_im, out_re, out_im, direction="forward", normalize=False,
                              stream: int = 0) -> None:
        """execute_split() that allocates nothing (fg_fft_exec_split_noalloc):
        multi-launch plans stage through the library's fixed 64 MiB device
        scratch area instead of a buffer of their own, so the call may be
        captured into a graph on any use.  Calls that overlap in time on one
        GPU share that area and race."""
        d = _direction(direction)
        half = self._nbytes // 2
        ptrs = [_ptr_sized(b, half, name) for b, name in
                ((in_re, "in_re"), (in_im, "in_im"), (out_re, "out_re"), (out_im, "out_im"))]
        _n.check(_n.lib.fg_fft_exec_split_noalloc(self._p, *ptrs, d, int(bool(normalize)),
                                                  ctypes.c_void_p(stream or None)))

    def capture_graph(self, d_in, d_out, direction="forward", normalize=False, reps: int = 1) -> "Graph":
        """A HIP graph of ``reps`` back-to-back ``execute(d_in, d_out, ...)``
        calls, replayed with one submission by ``Graph.launch``.  The graph
        uses the buffers by address: keep them alive while it is launched
        (the Graph holds a reference to this plan, and the plan cannot be
        destroyed while the graph exists)."""
        d = _direction(direction)
        g = ctypes.c_void_p()
        nb = self._nbytes
        _n.check(_n.lib.fg_fft_graph_create(self._p, _ptr_sized(d_in, nb, "d_in"), _ptr_sized(d_out, nb, "d_out"), d,
                                            int(bool(normalize)), int(reps), ctypes.byref(g)))
        return Graph(self.device, g, keep=(self,))

    def kernel_names(self, in_place: bool = False) -> list[str]:
        """Kernel of each launch, in launch order, of an out-of-place execution
        (or of an in-place one: 2D plans of 2048 / 4096 rows of 1024 .. 4096
        columns run other kernels in place)."""
        fn = _n.lib.fg_fft_plan_kernel_in_place if in_place else _n.lib.fg_fft_plan_kernel
        names = []
        for i in range(self.describe()["launches"]):
            buf = ctypes.create_string_buffer(128)
            _n.check(fn(self._p, i, buf, 128))
            names.append(buf.value.decode())
        return names

    def set_streams(self, streams: int) -> None:
        """Run the chunks on one stream (1) or, for a plan created with
        describe()["streams"] == 2, on two again (2); same bits either way.
        No execution of the plan may be in flight."""
        _n.check(_n.lib.fg_fft_plan_set_streams(self._p, int(streams)))

    def describe(self) -> dict:
        launches = ctypes.c_int()
        name = ctypes.create_string_buffer(128)
        ws = ctypes.c_size_t()
        _n.check(_n.lib.fg_fft_plan_describe(self._p, ctypes.byref(launches), name, 128, ctypes.byref(ws)))
        passes, units, chunks, cached = ctypes.c_int(), ctypes.c_size_t(), ctypes.c_int(), ctypes.c_int()
        _n.check(_n.lib.fg_fft_plan_chunking(self._p, ctypes.byref(passes), ctypes.byref(units),
                                             ctypes.byref(chunks), ctypes.byref(cached)))
        streams = ctypes.c_int()
        _n.check(_n.lib.fg_fft_plan_streams(self._p, ctypes.byref(streams)))
        return {"launches": launches.value, "main_kernel": name.value.decode(), "workspace_bytes": ws.value,
                "passes": passes.value, "units_per_chunk": units.value, "chunks": chunks.value,
                "cache_resident": bool(cached.value), "streams": streams.value}

    def destroy(self) -> None:
        """Free the plan; refused (FerrumGpuError) while graphs of it exist."""
        if getattr(self, "_p", None) is not None and self._p.value:
            _n.check(_n.lib.fg_fft_plan_destroy(self._p))
        self._p = ctypes.c_void_p()

    def __del__(self):  # pragma: no cover
        try:
            if getattr(self, "_p", None) is not None and self._p.value:
                # released after any Capture block open on this thread (ferrum_gpu.hip._release)
                _release(_n.lib.fg_fft_plan_destroy, self._p)
                self._p = ctypes.c_void_p()
        except Exception:
            pass


class Plan1D(_Plan):
    """Plan for ``batch`` transforms of length ``2**log_n`` (Plan::new, plan.rs:57-68)."""

    def __init__(self, log_n: int, batch: int, device: Device):
        p = ctypes.c_void_p()
        _n.check(_n.lib.fg_fft_plan_1d(device.handle, int(log_n), int(batch), ctypes.byref(p)))
        super().__init__(device, p, 1 << int(log_n), int(batch))
        self.log_n = int(log_n)


class Plan2D(_Plan):
    """Plan for ``batch`` N x N images, N = ``2**log_n`` (Plan2D::new, plan.rs:111-119).

    With ``log_cols`` the images are ``2**log_n`` rows x ``2**log_cols`` columns.
    """

    def __init__(self, log_n: int, batch: int, device: Device, log_cols: int | None = None):
        p = ctypes.c_void_p()
        log_rows = int(log_n)
        log_c = log_rows if log_cols is None else int(log_cols)
        if log_cols is None:
            _n.check(_n.lib.fg_fft_plan_2d(device.handle, log_rows, int(batch), ctypes.byref(p)))
        else:
            _n.check(_n.lib.fg_fft_plan_2d_rect(device.handle, log_rows, log_c, int(batch), ctypes.byref(p)))
        super().__init__(device, p, 1 << (log_rows + log_c), int(batch))
        self.log_n = log_rows
        self.log_cols = log_c


def fft2_c2c_pow2(arr, direction="forward", normalize=False, device=None):
    """2D FFT over the last two axes of a ``complex64`` array of shape
    ``(..., 2**a, 2**b)`` (4 <= a, b <= 12), rows and columns of any
    power-of-two lengths; ``normalize`` scales the inverse by 1/(rows*cols)."""
    a = _complex64_array(arr, (2, 3, 4))
    norm = _normalize(normalize)
    h = _device_handle(device)
    rows, cols = a.shape[-2], a.shape[-1]
    lr, lc = rows.bit_length() - 1, cols.bit_length() - 1
    if rows != 1 << lr or cols != 1 << lc or not (MIN_LOG_N_2D <= lr <= MAX_LOG_N_2D) \
            or not (MIN_LOG_N_2D <= lc <= MAX_LOG_N_2D):
        raise ValueError(f"arr shape {list(a.shape)}: the last two axes must be powers of two in "
                         f"[2^{MIN_LOG_N_2D}, 2^{MAX_LOG_N_2D}]")
    batch = a.size // (rows * cols)
    if batch == 0:
        raise ValueError(f"arr shape {list(a.shape)} holds no image")
    d = _direction(direction)
    _contiguous(a)
    out = np.empty_like(a)
    rc = _n.lib.fg_fft_2d_rect_host(h, a.ctypes.data, out.ctypes.data, lr, lc, batch, d, norm)
    if rc != _n.FG_OK:
        raise ValueError(f"ferrum-gpu fft 2d error: {_n.last_error()}")
    return out


def transpose(device: Device, d_in, d_out, rows: int, cols: int, batch: int = 1, stream: int = 0) -> None:
    """out[b][c][r] = in[b][r][c] for ``batch`` rows x cols complex64 matrices on
    the device (stream-ordered; in and out must not alias)."""
    rows, cols, batch = int(rows), int(cols), int(batch)
    nb = 8 * rows * cols * batch
    _n.check(_n.lib.fg_transpose_c64(device.handle, _ptr_sized(d_in, nb, "d_in"), _ptr_sized(d_out, nb, "d_out"),
                                     rows, cols, batch, ctypes.c_void_p(stream or None)))


def set_chunk_bytes(nbytes: int) -> None:
    """Chunk limit, in bytes, for multi-launch plans (1D N > 32768, 2D) created
    from now on, process-wide.  Such a plan runs every pass over one chunk of
    whole transforms (images) before the next chunk, so the chunk's
    intermediate array stays in the GPU's Infinity Cache.  ``nbytes`` bounds
    the chunks in flight: plans that run two chunks at a time (describe()
    "streams" == 2) take chunks of at most nbytes / 2, the others of at most
    ``nbytes``.  0 turns chunking off (one chunk, every pass streaming).
    Default 256 MiB, or FERRUM_GPU_CHUNK_MIB at library load."""
    if int(nbytes) < 0:
        raise ValueError(f"chunk bytes must be >= 0, got {nbytes}")
    _n.check(_n.lib.fg_fft_set_chunk_bytes(int(nbytes)))


def get_chunk_bytes() -> int:
    """The current chunk limit for new multi-launch plans (set_chunk_bytes)."""
    v = ctypes.c_size_t()
    _n.check(_n.lib.fg_fft_get_chunk_bytes(ctypes.byref(v)))
    return v.value

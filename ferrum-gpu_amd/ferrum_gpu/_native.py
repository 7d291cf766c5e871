"""ctypes binding of libferrum_gpu.so (the C ABI in include/ferrum_gpu.h).

This module plays the part of the reference's PyO3 cdylib
``ferrum_gpu._native`` (crates/ferrum-gpu-py/src/lib.rs:591-604).  ctypes
releases the GIL for the duration of every foreign call, which is what the
reference's ``py.allow_threads`` does around GPU work (lib.rs:490, 570).

The library is loaded from this package directory; if it is missing the import
fails loudly -- there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("FERRUM_GPU_LIBRARY", os.path.join(_HERE, "libferrum_gpu.so"))

FG_OK = 0
FG_ERR_INVALID_ARGUMENT = -1
FG_ERR_DRIVER = -2
FG_ERR_BACKEND_MISMATCH = -3
FG_ERR_KERNEL_NOT_FOUND = -4
FG_ERR_TARGET_MISMATCH = -5
FG_ERR_OUT_OF_MEMORY = -6
FG_ERR_NO_DEVICE = -7
FG_ERR_INTERNAL = -8

FG_BACKEND_CUDA, FG_BACKEND_VULKAN, FG_BACKEND_HIP = 1, 2, 3
FG_FORWARD, FG_INVERSE = 1, -1

_ERROR_NAMES = {
    FG_ERR_INVALID_ARGUMENT: "InvalidArgument",
    FG_ERR_DRIVER: "Driver",
    FG_ERR_BACKEND_MISMATCH: "BackendMismatch",
    FG_ERR_KERNEL_NOT_FOUND: "KernelNotFound",
    FG_ERR_TARGET_MISMATCH: "TargetMismatch",
    FG_ERR_OUT_OF_MEMORY: "OutOfMemory",
    FG_ERR_NO_DEVICE: "NoDevice",
    FG_ERR_INTERNAL: "Internal",
}


class FerrumGpuError(RuntimeError):
    """A non-zero status from the C ABI; ``code`` is the FG_ERR_* value."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code
        self.kind = _ERROR_NAMES.get(code, "Unknown")


if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"ferrum_gpu: native library not found at {LIB_PATH}; build it with "
        "`python -c 'import __graft_entry__ as g; g.build()'` (make -C ferrum-gpu_amd/csrc)"
    )

lib = ctypes.CDLL(LIB_PATH)

_i, _u32, _sz, _vp, _f = ctypes.c_int, ctypes.c_uint32, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float
_P = ctypes.POINTER


def _sig(name, *argtypes, restype=ctypes.c_int):
    fn = getattr(lib, name)
    fn.argtypes = list(argtypes)
    fn.restype = restype
    return fn


_sig("fg_last_error", restype=ctypes.c_char_p)
_sig("fg_version", restype=ctypes.c_char_p)
_sig("fg_backend_id")
_sig("fg_device_count", _P(_i))
_sig("fg_device_open", _i, _P(_vp))
_sig("fg_device_close", _vp)
_sig("fg_device_sync", _vp)
_sig("fg_device_default_stream", _vp, _P(_vp))
_sig("fg_device_info", _vp, ctypes.c_char_p, _sz, _P(_i), _P(_sz), _P(_i))
_sig("fg_alloc_zeros", _vp, _sz, _P(_vp))
_sig("fg_free", _vp, _vp)
_sig("fg_copy_h2d", _vp, _vp, _vp, _sz)
_sig("fg_copy_d2h", _vp, _vp, _vp, _sz)
_sig("fg_copy_h2d_async", _vp, _vp, _vp, _sz, _vp)
_sig("fg_copy_d2h_async", _vp, _vp, _vp, _sz, _vp)
_sig("fg_copy_d2d_async", _vp, _vp, _vp, _sz, _vp)
_sig("fg_module_load", _vp, _i, _vp, _sz, _P(_vp))
_sig("fg_module_unload", _vp)
_sig("fg_device_fft_module", _vp, _P(_vp))
_sig("fg_kernel_get", _vp, ctypes.c_char_p, _P(_vp))
_sig("fg_launch", _vp, _vp, _vp, _P(_u32), _P(_u32), _u32, _P(_vp))
_sig("fg_stream_create", _vp, _P(_vp))
_sig("fg_stream_destroy", _vp, _vp)
_sig("fg_stream_sync", _vp, _vp)
_sig("fg_event_create", _vp, _P(_vp))
_sig("fg_event_destroy", _vp)
_sig("fg_event_record", _vp, _vp)
_sig("fg_event_sync", _vp)
_sig("fg_event_elapsed_ms", _vp, _vp, _P(_f))
_sig("fg_fft_plan_1d", _vp, _u32, _sz, _P(_vp))
_sig("fg_fft_plan_2d", _vp, _u32, _sz, _P(_vp))
_sig("fg_fft_plan_destroy", _vp)
_sig("fg_fft_exec", _vp, _vp, _vp, _i, _i, _vp)
_sig("fg_fft_plan_describe", _vp, _P(_i), ctypes.c_char_p, _sz, _P(_sz))
_sig("fg_fft_exec_events", _vp, _vp, _vp, _i, _i, _vp, _P(_vp), _i)
_sig("fg_fft_plan_kernel", _vp, _i, ctypes.c_char_p, _sz)
_sig("fg_fft_plan_kernel_in_place", _vp, _i, ctypes.c_char_p, _sz)
_sig("fg_fft_set_chunk_bytes", _sz)
_sig("fg_fft_get_chunk_bytes", _P(_sz))
_sig("fg_fft_plan_chunking", _vp, _P(_i), _P(_sz), _P(_i), _P(_i))
_sig("fg_fft_plan_streams", _vp, _P(_i))
_sig("fg_fft_plan_set_streams", _vp, _i)
_sig("fg_fft_1d_c2c_pow2_host", _vp, _vp, _vp, _sz, _u32, _i, _i)
_sig("fg_fft_2d_c2c_pow2_host", _vp, _vp, _vp, _u32, _sz, _i, _i)
_sig("fg_stream_copy", _vp, _vp, _vp, _sz, _vp)
_sig("fg_fft_plan_2d_rect", _vp, _u32, _u32, _sz, _P(_vp))
_sig("fg_fft_2d_rect_host", _vp, _vp, _vp, _u32, _u32, _sz, _i, _i)
_sig("fg_transpose_c64", _vp, _vp, _vp, _u32, _u32, _sz, _vp)
_sig("fg_fft_exec_split", _vp, _vp, _vp, _vp, _vp, _i, _i, _vp)
_sig("fg_fft_exec_split_noalloc", _vp, _vp, _vp, _vp, _vp, _i, _i, _vp)
_sig("fg_cmul_c64", _vp, _vp, _vp, _vp, _sz, _vp)
_sig("fg_cmul_split", _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp)
_sig("fg_deinterleave_c64", _vp, _vp, _vp, _vp, _sz, _vp)
_sig("fg_interleave_c64", _vp, _vp, _vp, _vp, _sz, _vp)
_sig("fg_fill_uniform_c64", _vp, _vp, _sz, ctypes.c_uint64, _vp)
_sig("fg_fill_normal_c64", _vp, _vp, _sz, ctypes.c_uint64, _vp)
_sig("fg_fft_graph_create", _vp, _vp, _vp, _i, _i, _i, _P(_vp))
_sig("fg_graph_launch", _vp, _vp)
_sig("fg_graph_capture_begin", _vp, _P(_vp))
_sig("fg_graph_capture_end", _vp, _vp, _P(_vp))
_sig("fg_graph_node_count", _vp, _P(_sz))
_sig("fg_graph_destroy", _vp)


def last_error() -> str:
    return (lib.fg_last_error() or b"").decode("utf-8", "replace")


def check(rc: int) -> None:
    if rc != FG_OK:
        raise FerrumGpuError(rc, last_error())


def version() -> str:
    """Crate version string (crates/ferrum-gpu-py/src/lib.rs:420-423)."""
    return lib.fg_version().decode()


def backend_id() -> int:
    return lib.fg_backend_id()

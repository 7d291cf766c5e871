"""CPU-side checks of the C ABI library and the Python boundary (no GPU needed).

The library must load, export every entry point include/ferrum_gpu.h
declares, and reject bad arguments with the reference's messages before any
device is touched (crates/ferrum-gpu-py/src/lib.rs:455-477, 537-558).
"""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

import ferrum_gpu
from ferrum_gpu import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ferrum_gpu.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^FG_API\s+[\w\s\*]+?\b(fg_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for must in ("fg_fft_plan_1d", "fg_fft_plan_2d", "fg_fft_exec", "fg_fft_1d_c2c_pow2_host",
                 "fg_fft_2d_c2c_pow2_host", "fg_module_load", "fg_kernel_get", "fg_launch",
                 "fg_alloc_zeros", "fg_copy_h2d", "fg_copy_d2h", "fg_event_elapsed_ms"):
        assert must in syms
    assert len(syms) >= 37


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(N.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_library_exports_nothing_undeclared():
    out = os.popen(f"nm -D --defined-only {N.LIB_PATH}").read()
    exported = sorted(set(re.findall(r" T (fg_\w+)", out)))
    assert exported == declared_symbols()


def test_chunk_limit_round_trip():
    # Process-wide; read by plans when they are created (no device needed).
    saved = ferrum_gpu.fft.get_chunk_bytes()
    try:
        assert saved == 256 << 20 or os.environ.get("FERRUM_GPU_CHUNK_MIB")
        for v in (0, 1, 64 << 20, 1 << 40):
            ferrum_gpu.fft.set_chunk_bytes(v)
            assert ferrum_gpu.fft.get_chunk_bytes() == v
        with pytest.raises(ValueError):
            ferrum_gpu.fft.set_chunk_bytes(-1)
    finally:
        ferrum_gpu.fft.set_chunk_bytes(saved)


def test_version_and_backend():
    assert ferrum_gpu.version() == "0.3.0"          # crates/ferrum-gpu-py/src/lib.rs:420-423
    assert N.backend_id() == N.FG_BACKEND_HIP == 3  # BackendId with Hip added


def instantiated_kernels():
    src = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "kernels", "fft_kernels.hip")).read()
    names = {f"fg_fft_n{m.group(1)}" for m in re.finditer(r"^FG_STOCKHAM\((\d+),", src, flags=re.M)}
    # 8192 / 16384 points: 32 elements per thread, exchanges in halves
    names |= {f"fg_fft_n{m.group(1)}" for m in re.finditer(r"^FG_STOCKHAM_HALVES\((\d+)\)", src, flags=re.M)}
    # 1024 points: two transforms per workgroup, radix list 8 * 16 * 8 (with its _sc variant)
    x2 = re.search(r"^FG_STOCKHAM_X2_1024\(\)", src, flags=re.M) is not None
    if x2:
        names.add("fg_fft_n10")
    names |= {f"{n}_split" for n in names}
    if x2:
        names.add("fg_fft_n10_sc")
    names |= {f"fg_fft_n{m.group(1)}_sc" for m in re.finditer(r"^FG_STOCKHAM_SC\((\d+),", src, flags=re.M)}
    for m in re.finditer(r"^FG_STOCKHAM_LAT\((\d+),", src, flags=re.M):
        names |= {f"fg_fft_n{m.group(1)}_lat", f"fg_fft_n{m.group(1)}_lat_split"}
    for m in re.finditer(r"^FG_TILE(_NARROW)?\((\d+), (\d+), (true|false), ([cr])\)", src, flags=re.M):
        base = f"fg_tile_l{m.group(2)}_g{m.group(3)}_{m.group(5)}"
        # cache policies (FG_TILE_P): all four, or _cc alone for narrow tiles
        names |= {base + "_cc"} if m.group(1) else {base + pol for pol in ("", "_sc", "_cc", "_cs")}
    # one-pass 2D FFTs of small images
    for a, b in re.findall(r"^FG_FFT2D(?:_HALVES)?\((\d+), (\d+)\)", src, flags=re.M):
        names |= {f"fg_fft2d_l{a}_{b}", f"fg_fft2d_l{a}_{b}_split"}
    # first-pass tiles with the exchanges in halves: unchunked and _sc
    for m in re.finditer(r"^FG_TILE_HALVES\((\d+), (\d+)\)", src, flags=re.M):
        names |= {f"fg_tile_l{m.group(1)}_g{m.group(2)}_h{pol}" for pol in ("", "_sc")}
    # the 1024-point column pass in 16-column halves tiles, streamed out
    for m in re.finditer(r"^FG_TILE_HALVES_P\((\d+), (\d+), _cs, true, false\)", src, flags=re.M):
        names.add(f"fg_tile_l{m.group(1)}_g{m.group(2)}_h_cs")
    # the 1D middle pass of 256 points in halves, cached in and out
    for m in re.finditer(r"^FG_TILE_HALVES_P\((\d+), (\d+), _cc, true, true\)", src, flags=re.M):
        names.add(f"fg_tile_l{m.group(1)}_g{m.group(2)}_h_cc")
    # 1D last passes of 512 / 1024 points: rows in, exchanges in halves
    for m in re.finditer(r"^FG_TILE_ROW_HALVES\((\d+), (\d+), (\w*),", src, flags=re.M):
        names.add(f"fg_tile_l{m.group(1)}_g{m.group(2)}_rh{m.group(3)}")
    # row passes over row pairs (2D images of 4096 rows)
    names |= set(re.findall(r"void (fg_fft2d_rowpair_n\d+)\(", src))
    # narrow tiles in halves (2D columns of 2048 / 4096 points): _cc alone
    for m in re.finditer(r"^FG_TILE_HALVES_NARROW\((\d+), (\d+)\)", src, flags=re.M):
        names.add(f"fg_tile_l{m.group(1)}_g{m.group(2)}_h_cc")
    return names


def planned_kernels():
    """Every kernel name FftPlan can request (mirrors fft_plan.cpp via the CPU models)."""
    from test_multipass_model import plan_kernel_names
    from test_stockham_model import LATENCY_GEOM

    names = {f"fg_fft_n{l}" for l in range(2, 16)} | {f"fg_fft_n{l}_split" for l in range(2, 16)}
    names |= {f"fg_fft_n{l}_lat{sfx}" for l in LATENCY_GEOM for sfx in ("", "_split")}
    for cached in (False, True):
        for log_n in range(13, 25):
            names |= set(plan_kernel_names(False, log_n, cached))
            names |= set(plan_kernel_names(False, log_n, cached, streams=2))
        for lr in range(4, 13):
            for lc in range(4, 13):
                names |= set(plan_kernel_names(True, lr, cached, lc))
                if lr + lc <= 14:   # one-pass images: exec_split's twin
                    names.add(f"fg_fft2d_l{lr}_{lc}_split")
    return names


def test_every_planned_kernel_is_instantiated():
    missing = planned_kernels() - instantiated_kernels()
    assert not missing, sorted(missing)


def test_code_object_is_embedded_for_gfx950():
    # The .so carries the gfx950 code object (an ELF for amdgcn) in .rodata,
    # with every instantiated kernel.
    data = open(N.LIB_PATH, "rb").read()
    assert data.count(b"\x7fELF") >= 2
    assert b"gfx950" in data
    for k in sorted(instantiated_kernels()) + ["fg_copy_f4", "fg_vector_add", "fg_transpose_c64", "fg_transpose_c64_t128", "fg_fill_c64"] \
            + POINTWISE:
        assert k.encode() in data, k


POINTWISE = [f"fg_{op}_{w}" for op in ("cmul_c64", "cmul_split", "deinterleave_c64", "interleave_c64")
             for w in ("vec", "elem")]


def test_pointwise_kernels_are_instantiated():
    src = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "kernels", "fft_kernels.hip")).read()
    variants = re.findall(r"^FG_POINTWISE\((\w+), ", src, flags=re.M)
    assert sorted(variants) == ["elem", "vec"]
    host = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "pointwise_ops.cpp")).read()
    for op in ("cmul_c64", "cmul_split", "deinterleave_c64", "interleave_c64"):
        assert f'"fg_{op}"' in host


# --------------------------------------------------- argument validation


def test_fft_1d_argument_errors():
    f = ferrum_gpu.fft.fft_1d_c2c_pow2
    x = np.zeros(1024, np.complex64)
    with pytest.raises(ValueError, match=r"^log_n must be in \[2, 24\], got 1$"):
        f(x, 1)
    with pytest.raises(ValueError, match=r"^log_n must be in \[2, 24\], got 25$"):
        f(x, 25)
    with pytest.raises(ValueError, match=r"^arr len 1000 must be a positive multiple of N = 1024$"):
        f(np.zeros(1000, np.complex64), 10)
    with pytest.raises(ValueError, match=r"^arr len 0 must be a positive multiple of N = 4$"):
        f(np.zeros(0, np.complex64), 2)
    with pytest.raises(ValueError, match=r"^direction must be 'forward' or 'inverse', got \"sideways\"$"):
        f(x, 10, direction="sideways")
    with pytest.raises(TypeError):
        f(np.zeros(1024, np.complex128), 10)        # PyReadonlyArray1<Complex32> dtype check
    with pytest.raises(TypeError):
        f(np.zeros((2, 512), np.complex64), 9)      # rank check
    with pytest.raises(TypeError):
        f(np.zeros(2048, np.complex64)[::2], 10)    # as_slice() needs contiguity
    with pytest.raises(OverflowError):
        f(x, -1)                                    # u32 extraction
    with pytest.raises(TypeError):
        f(x, 10, device="gpu0")


def test_fft_2d_argument_errors():
    f = ferrum_gpu.fft.fft_2d_c2c_pow2
    with pytest.raises(ValueError, match=r"^2D requires log_n in \[4, 12\]; got 3$"):
        f(np.zeros((8, 8), np.complex64), 3)
    with pytest.raises(ValueError, match=r"^2D requires log_n in \[4, 12\]; got 13$"):
        f(np.zeros((16, 16), np.complex64), 13)
    with pytest.raises(ValueError, match=r"^arr shape \[16, 8\] != \(16, 16\)$"):
        f(np.zeros((16, 8), np.complex64), 4)
    with pytest.raises(ValueError, match=r"^direction must be 'forward' or 'inverse'"):
        f(np.zeros((16, 16), np.complex64), 4, direction="back")


def test_argument_types_match_pyo3_extraction():
    # `direction: &str` and `normalize: bool` (crates/ferrum-gpu-py/src/lib.rs:451-452,
    # 533-534): PyO3 0.23 raises TypeError for any other type, before the
    # function body's ValueErrors.
    x = np.zeros(1024, np.complex64)
    img = np.zeros((16, 16), np.complex64)
    for f, a, ln in ((ferrum_gpu.fft.fft_1d_c2c_pow2, x, 10), (ferrum_gpu.fft.fft_2d_c2c_pow2, img, 4)):
        with pytest.raises(TypeError, match=r"^argument 'direction': 'int' object cannot be converted to 'PyString'$"):
            f(a, ln, direction=5)
        with pytest.raises(TypeError, match=r"^argument 'direction': 'NoneType' object cannot be converted"):
            f(a, ln, None)
        with pytest.raises(TypeError, match=r"^argument 'normalize': 'str' object cannot be converted to 'PyBool'$"):
            f(a, ln, "inverse", "yes")
        with pytest.raises(TypeError, match=r"^argument 'normalize': 'int' object cannot be converted to 'PyBool'$"):
            f(a, ln, "inverse", 1)
        with pytest.raises(TypeError, match=r"^argument 'device': 'str' object cannot be converted to 'Device'$"):
            f(a, ln, device="gpu0")
        # extraction comes first: a bad normalize wins over an out-of-range log_n
        with pytest.raises(TypeError, match="normalize"):
            f(a, 40, "forward", 0)
        # numpy.bool_ passes extraction (the log_n ValueError is what stops the call)
        with pytest.raises(ValueError, match="log_n"):
            f(a, 40, "forward", np.bool_(True))
        with pytest.raises(ValueError, match="log_n"):
            f(a, 40, "forward", False)
    # the body's order: the log_n range check runs before as_slice()'s contiguity check
    with pytest.raises(ValueError, match="log_n"):
        ferrum_gpu.fft.fft_1d_c2c_pow2(np.zeros(2048, np.complex64)[::2], 30)
    with pytest.raises(ValueError, match="direction"):
        ferrum_gpu.fft.fft_2d_c2c_pow2(np.zeros((16, 32), np.complex64)[:, ::2], 4, "back")


def _fake_buffer(nbytes, addr=1 << 20):
    # A DeviceBuffer that owns nothing (no device call): only the size and
    # address the Python layer checks.
    b = object.__new__(ferrum_gpu.hip.DeviceBuffer)
    b.nbytes = nbytes
    b._p = ctypes.c_void_p(addr)
    b.device = None
    return b


def test_small_buffers_are_refused_before_any_launch():
    # A plan object with no native plan behind it: every refusal below must
    # come from the size check, before the C ABI is called.
    plan = object.__new__(ferrum_gpu.fft._Plan)
    plan._p = ctypes.c_void_p(None)
    plan.elems, plan.batch, plan._nbytes = 1024, 4, 4 * 1024 * 8
    ok, small = _fake_buffer(plan.nbytes), _fake_buffer(plan.nbytes - 8)
    with pytest.raises(ValueError, match=r"^d_in: buffer of 32760 bytes, the plan reads or writes 32768$"):
        plan.execute(small, ok)
    with pytest.raises(ValueError, match=r"^d_out: buffer of 32760 bytes"):
        plan.execute(ok, small)
    with pytest.raises(ValueError, match="d_out"):
        plan.execute_recording(ok, small, [])
    with pytest.raises(ValueError, match="d_in"):
        plan.capture_graph(small, ok)
    half_ok, half_small = _fake_buffer(plan.nbytes // 2), _fake_buffer(plan.nbytes // 2 - 4)
    with pytest.raises(ValueError, match=r"^out_im: buffer of 16380 bytes, the plan reads or writes 16384$"):
        plan.execute_split(half_ok, half_ok, half_ok, half_small)
    # right-sized buffers reach the C ABI, which refuses the null plan
    with pytest.raises(N.FerrumGpuError, match="plan is null"):
        plan.execute(ok, ok)
    with pytest.raises(N.FerrumGpuError, match="plan is null"):
        plan.execute_split(half_ok, half_ok, half_ok, half_ok)
    n = 100

    class NoDevice:  # a device handle the size checks never reach
        handle = None

    dev = NoDevice()
    with pytest.raises(ValueError, match="^out: buffer of 792 bytes"):
        ferrum_gpu.pointwise.cmul(dev, _fake_buffer(800), _fake_buffer(800), _fake_buffer(792), n)
    with pytest.raises(ValueError, match="^im: buffer of 396 bytes"):
        ferrum_gpu.pointwise.deinterleave(dev, _fake_buffer(800), _fake_buffer(400), _fake_buffer(396), n)
    with pytest.raises(ValueError, match="^re: buffer"):
        ferrum_gpu.pointwise.interleave(dev, _fake_buffer(396), _fake_buffer(400), _fake_buffer(800), n)
    with pytest.raises(ValueError, match="^b_im: buffer"):
        ferrum_gpu.pointwise.cmul_split(dev, *[_fake_buffer(400)] * 3, _fake_buffer(4), *[_fake_buffer(400)] * 2, n)
    with pytest.raises(ValueError, match="^out: buffer of 799 bytes"):
        ferrum_gpu.synthetic.normal(dev, _fake_buffer(799), n, 1)
    with pytest.raises(ValueError, match="^d_out: buffer"):
        ferrum_gpu.fft.transpose(dev, _fake_buffer(8 * 64 * 32), _fake_buffer(8 * 64 * 31), 64, 32)


def test_c_abi_validation_without_device():
    # The host entry points validate before they need a device.
    x = np.zeros(64, np.complex64)
    y = np.empty_like(x)
    rc = N.lib.fg_fft_1d_c2c_pow2_host(None, x.ctypes.data, y.ctypes.data, 64, 30, 1, 0)
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "log_n must be in [2, 24], got 30" in N.last_error()
    rc = N.lib.fg_fft_1d_c2c_pow2_host(None, x.ctypes.data, y.ctypes.data, 60, 4, 1, 0)
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "arr len 60 must be a positive multiple of N = 16" in N.last_error()
    rc = N.lib.fg_fft_1d_c2c_pow2_host(None, x.ctypes.data, y.ctypes.data, 64, 4, 2, 0)
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "direction" in N.last_error()
    rc = N.lib.fg_fft_2d_c2c_pow2_host(None, x.ctypes.data, y.ctypes.data, 2, 1, 1, 0)
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "2D requires log_n in [4, 12]; got 2" in N.last_error()
    # a batch whose element count overflows size_t is refused before any device work
    rc = N.lib.fg_fft_2d_c2c_pow2_host(None, x.ctypes.data, y.ctypes.data, 12, 1 << 40, 1, 0)
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "too large for images of 2^24 points" in N.last_error()
    rc = N.lib.fg_fft_2d_rect_host(None, x.ctypes.data, y.ctypes.data, 12, 11, 1 << 41, 1, 0)
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "too large for images of 2^23 points" in N.last_error()
    rc = N.lib.fg_fft_exec(None, None, None, 1, 0, None)
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "plan is null" in N.last_error()
    rc = N.lib.fg_fft_plan_1d(None, 10, 1, ctypes.byref(ctypes.c_void_p()))
    assert rc == N.FG_ERR_INVALID_ARGUMENT
    streams = ctypes.c_int(-1)
    rc = N.lib.fg_fft_plan_streams(None, ctypes.byref(streams))
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "plan is null" in N.last_error() and streams.value == -1


def test_split_and_pointwise_validation_without_device():
    rc = N.lib.fg_fft_exec_split(None, None, None, None, None, 1, 0, None)
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "plan is null" in N.last_error()
    # (entry point, number of device-pointer arguments between dev and n)
    for fn, nptrs in (("fg_cmul_c64", 3), ("fg_cmul_split", 6), ("fg_deinterleave_c64", 3),
                      ("fg_interleave_c64", 3)):
        rc = getattr(N.lib, fn)(None, *([None] * nptrs), 16, None)
        assert rc == N.FG_ERR_INVALID_ARGUMENT and "device is null" in N.last_error(), fn
    for fn in ("fg_fill_uniform_c64", "fg_fill_normal_c64"):
        rc = getattr(N.lib, fn)(None, None, 16, 1, None)
        assert rc == N.FG_ERR_INVALID_ARGUMENT and "device is null" in N.last_error(), fn


def test_graph_validation_without_device():
    out = ctypes.c_void_p()
    rc = N.lib.fg_fft_graph_create(None, None, None, 1, 0, 1, ctypes.byref(out))
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "plan is null" in N.last_error()
    rc = N.lib.fg_graph_launch(None, None)
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "graph is null" in N.last_error()
    rc = N.lib.fg_graph_node_count(None, ctypes.byref(ctypes.c_size_t()))
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "graph is null" in N.last_error()
    rc = N.lib.fg_graph_capture_begin(None, ctypes.byref(ctypes.c_void_p()))
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "device is null" in N.last_error()
    rc = N.lib.fg_graph_capture_end(None, None, ctypes.byref(out))
    assert rc == N.FG_ERR_INVALID_ARGUMENT and "device is null" in N.last_error()
    assert N.lib.fg_graph_destroy(None) == N.FG_OK


def test_last_error_is_thread_local():
    import threading

    N.lib.fg_fft_exec(None, None, None, 1, 0, None)
    assert N.last_error()
    seen = []
    t = threading.Thread(target=lambda: seen.append(N.last_error()))
    t.start()
    t.join()
    assert seen == [""]


def test_no_device_reports_cleanly():
    if ferrum_gpu.hip.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(ValueError, match=r"^Device::new\(0\): "):
        ferrum_gpu.hip.Device(0)
    with pytest.raises(ValueError, match=r"^ferrum-gpu fft error: "):
        ferrum_gpu.fft.fft_1d_c2c_pow2(np.zeros(16, np.complex64), 4)


# ------------------------------------------------ the C ABI from plain C

EXAMPLES = os.path.join(ROOT, "ferrum-gpu_amd", "examples")


def test_header_is_plain_c(tmp_path):
    # An FFI binding (bindgen, cgo, ctypes) reads the header as C.
    src = tmp_path / "h.c"
    src.write_text('#include "ferrum_gpu.h"\nint main(void) { return 0; }\n')
    cmd = f"gcc -std=c99 -Wall -Wextra -pedantic -Werror -fsyntax-only -I{os.path.join(ROOT, 'include')} {src}"
    assert os.system(cmd) == 0


def test_c_example_is_built_against_the_library():
    # make builds examples/fft_c_abi (executable) and libfft_c_abi.so (the same
    # checks as fft_c_abi_example(), run in-process by the GPU tests).
    exe = os.path.join(EXAMPLES, "fft_c_abi")
    so = os.path.join(EXAMPLES, "libfft_c_abi.so")
    assert os.path.exists(exe) and os.path.exists(so)
    for f in (exe, so):
        needed = os.popen(f"readelf -d {f}").read()
        assert "libferrum_gpu.so" in needed, f
    assert hasattr(ctypes.CDLL(so), "fft_c_abi_example")


def test_host_objects_depend_on_the_shared_geometry_header():
    # fft_plan.hpp includes kernels/tile_geom.h, whose launch geometry the
    # kernels are compiled against: the Makefile must rebuild the host objects
    # when it changes, or a stale host launches a kernel with the old block size
    mk = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "Makefile")).read()
    host_hdr = re.search(r"^HOST_HDR\s*:=(.*)$", mk, flags=re.M).group(1)
    assert "kernels/tile_geom.h" in host_hdr
    plan_hpp = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "fft_plan.hpp")).read()
    assert '#include "kernels/tile_geom.h"' in plan_hpp

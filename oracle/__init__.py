"""CPU oracle for the ferrum-gpu FFT path -- TEST INFRASTRUCTURE ONLY.

This package wraps ``oracle/liboracle.so`` (built from ``oracle/oracle.c`` by
``oracle/Makefile``), a plain-C restatement of the reference's CPU Stockham
FFT (``crates/ferrum-gpu-fft/src/{twiddles,cpu,cpu_2d,cpu_radix4,cpu_radix8,
warp_fft,layout_study}.rs``).  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker or the reported CPU baseline.  The product (``ferrum_gpu``) never
imports it.

Parity pins (what checks each function against something it did not produce):
  or_twiddles / radix4 / radix8 / full_roots -- closed-form lengths and end
      values (tests/twiddles.rs:5-37 of the reference) and fp64 cos/sin.
  or_fft_1d -- DFT([1,2,3,4]) (cpu.rs:142-170), impulse/constant closed forms,
      numpy.fft complex128 golden fixtures, fp64 direct DFT, round trips.
  or_fft_2d -- numpy.fft.fft2 fixtures, separable fp64 DFT, round trips.
  or_radix4/8_forward_lane, or_four_step, or_warp_dif -- direct DFT and the
      radix-2 path (cpu_radix4.rs:105-159, cpu_radix8.rs:153-216,
      warp_fft.rs:211-311).
  or_dft_naive / or_dft_bins_f64 -- DFT([1,2,3,4]) and numpy complex128.
  or_cmul_interleaved / or_cmul_split -- numpy float32 elementwise products
      (each product and the sum rounded to f32), i*i = -1, z*conj(z) = |z|^2.
  or_deinterleave / or_interleave -- numpy .real/.imag views, and each other's inverse.
  or_splitmix64_at / or_fill_* -- splitmix64's published first outputs for
      seed 0, a pure-Python splitmix64, exact value grid and moments (uniform),
      Box-Muller evaluated in Python floats and moments / tails (normal).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None
_lock = threading.Lock()


def build() -> str:
    """Compile liboracle.so with gcc (CPU only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                build()
            L = ctypes.CDLL(_LIB_PATH)
            fp = ctypes.POINTER(ctypes.c_float)
            u32, sz = ctypes.c_uint32, ctypes.c_size_t
            L.or_twiddles.argtypes = [u32, fp]
            L.or_twiddles_radix4_len.argtypes = [u32]
            L.or_twiddles_radix4_len.restype = sz
            L.or_twiddles_radix4.argtypes = [u32, fp]
            L.or_twiddles_radix8_len.argtypes = [u32]
            L.or_twiddles_radix8_len.restype = sz
            L.or_twiddles_radix8.argtypes = [u32, fp]
            L.or_twiddles_full_roots.argtypes = [u32, fp]
            L.or_stage_offsets.argtypes = [u32, ctypes.POINTER(sz)]
            L.or_fft_1d.argtypes = [fp, u32, sz, ctypes.c_int, ctypes.c_int]
            L.or_fft_1d.restype = ctypes.c_int
            L.or_fft_1d_lanes.argtypes = [fp, u32, sz, sz, ctypes.c_int, ctypes.c_int]
            L.or_fft_1d_lanes.restype = ctypes.c_int
            L.or_fft_2d.argtypes = [fp, u32, sz, ctypes.c_int, ctypes.c_int]
            L.or_fft_2d.restype = ctypes.c_int
            L.or_transpose_square.argtypes = [fp, sz]
            L.or_dft4_inplace.argtypes = [fp]
            L.or_dft8_inplace.argtypes = [fp]
            L.or_radix4_forward_lane.argtypes = [fp, fp, u32, fp]
            L.or_radix8_forward_lane.argtypes = [fp, fp, u32, fp]
            L.or_warp_dif.argtypes = [fp, u32]
            L.or_four_step.argtypes = [fp, fp, u32, u32]
            L.or_dft_naive.argtypes = [fp, fp, sz]
            L.or_dft_bins_f64.argtypes = [fp, sz, ctypes.POINTER(ctypes.c_int64), sz,
                                          ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
            L.or_cmul_interleaved.argtypes = [fp, fp, fp, sz]
            L.or_cmul_split.argtypes = [fp, fp, fp, fp, fp, fp, sz]
            L.or_deinterleave.argtypes = [fp, fp, fp, sz]
            L.or_interleave.argtypes = [fp, fp, fp, sz]
            L.or_splitmix64_at.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
            L.or_splitmix64_at.restype = ctypes.c_uint64
            L.or_fill_uniform_c64.argtypes = [fp, sz, ctypes.c_uint64]
            L.or_fill_normal_c64.argtypes = [fp, sz, ctypes.c_uint64]
            _lib = L
    return _lib


def _fptr(a: np.ndarray):
    assert a.dtype in (np.float32, np.complex64) and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _as_c64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.complex64))


def twiddles(log_n: int) -> np.ndarray:
    out = np.empty((1 << log_n) - 1, dtype=np.complex64)
    lib().or_twiddles(log_n, _fptr(out))
    return out


def twiddles_radix4(log_n: int) -> np.ndarray:
    out = np.empty(lib().or_twiddles_radix4_len(log_n), dtype=np.complex64)
    lib().or_twiddles_radix4(log_n, _fptr(out))
    return out


def twiddles_radix8(log_n: int) -> np.ndarray:
    out = np.empty(lib().or_twiddles_radix8_len(log_n), dtype=np.complex64)
    lib().or_twiddles_radix8(log_n, _fptr(out))
    return out


def twiddles_full_roots(log_n: int) -> np.ndarray:
    out = np.empty(1 << log_n, dtype=np.complex64)
    lib().or_twiddles_full_roots(log_n, _fptr(out))
    return out


def stage_offsets(log_n: int) -> list[int]:
    offs = (ctypes.c_size_t * (log_n + 1))()
    lib().or_stage_offsets(log_n, offs)
    return list(offs)


def fft_1d(arr, log_n: int, direction: str = "forward", normalize: bool = False,
           threads: int = 1) -> np.ndarray:
    """Plan::cpu_execute over a flat batch*N complex64 array (returns a copy)."""
    buf = _as_c64(arr).reshape(-1).copy()
    n = 1 << log_n
    if buf.size == 0 or buf.size % n:
        raise ValueError(f"buf.len() ({buf.size}) must be a positive multiple of n ({n})")
    d = 1 if direction == "forward" else -1
    batch = buf.size // n
    if threads <= 1 or batch < 2:
        rc = lib().or_fft_1d(_fptr(buf), log_n, batch, d, int(normalize))
        if rc:
            raise ValueError(f"or_fft_1d failed ({rc})")
        return buf
    # Lanes are independent (cpu.rs:101): split them across threads; ctypes
    # drops the GIL for the duration of each call.
    threads = min(threads, batch)
    bounds = np.linspace(0, batch, threads + 1).astype(int)
    rcs = [0] * threads

    def run(i):
        rcs[i] = lib().or_fft_1d_lanes(_fptr(buf), log_n, int(bounds[i]), int(bounds[i + 1]),
                                       d, int(normalize))

    ts = [threading.Thread(target=run, args=(i,)) for i in range(threads)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    if any(rcs):
        raise ValueError(f"or_fft_1d_lanes failed ({rcs})")
    return buf


def fft_2d(arr, log_n: int, direction: str = "forward", normalize: bool = False) -> np.ndarray:
    """Plan2D::cpu_execute over (batch, N, N) or (N, N) complex64 (returns a copy)."""
    a = _as_c64(arr)
    n = 1 << log_n
    buf = a.reshape(-1).copy()
    if buf.size % (n * n):
        raise ValueError("2D buffer is not a whole number of N x N images")
    d = 1 if direction == "forward" else -1
    rc = lib().or_fft_2d(_fptr(buf), log_n, buf.size // (n * n), d, int(normalize))
    if rc:
        raise ValueError(f"or_fft_2d failed ({rc})")
    return buf.reshape(a.shape)


def dft4(x8: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x8, dtype=np.float32).copy()
    lib().or_dft4_inplace(_fptr(x))
    return x


def dft8(x16: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x16, dtype=np.float32).copy()
    lib().or_dft8_inplace(_fptr(x))
    return x


def radix4_forward_lane(lane, log_n: int, tw: np.ndarray) -> np.ndarray:
    x = _as_c64(lane).copy()
    scratch = np.empty_like(x)
    lib().or_radix4_forward_lane(_fptr(x), _fptr(scratch), log_n, _fptr(_as_c64(tw)))
    return x


def radix8_forward_lane(lane, log_n: int, tw: np.ndarray) -> np.ndarray:
    x = _as_c64(lane).copy()
    scratch = np.empty_like(x)
    lib().or_radix8_forward_lane(_fptr(x), _fptr(scratch), log_n, _fptr(_as_c64(tw)))
    return x


def warp_dif(x, log_n: int) -> np.ndarray:
    y = _as_c64(x).copy()
    lib().or_warp_dif(_fptr(y), log_n)
    return y


def four_step(x, log_n1: int, log_n2: int) -> np.ndarray:
    a = _as_c64(x)
    out = np.empty_like(a)
    lib().or_four_step(_fptr(a), _fptr(out), log_n1, log_n2)
    return out


def dft_naive(x) -> np.ndarray:
    a = _as_c64(x)
    out = np.empty_like(a)
    lib().or_dft_naive(_fptr(a), _fptr(out), a.size)
    return out


def dft_bins_f64(x, bins, sign: int = -1) -> np.ndarray:
    """fp64 DFT of one lane at the given bins (complex128)."""
    a = _as_c64(x)
    b = np.ascontiguousarray(np.asarray(bins, dtype=np.int64))
    out = np.empty(b.size, dtype=np.complex128)
    lib().or_dft_bins_f64(_fptr(a), a.size, b.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                          b.size, sign, out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    return out


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def cmul_interleaved(a, b) -> np.ndarray:
    """a * b elementwise over complex64 arrays (f32, no fused multiply-add)."""
    x, y = _as_c64(a), _as_c64(b)
    assert x.shape == y.shape
    out = np.empty_like(x)
    lib().or_cmul_interleaved(_fptr(x), _fptr(y), _fptr(out), x.size)
    return out


def cmul_split(a_re, a_im, b_re, b_im) -> tuple[np.ndarray, np.ndarray]:
    ar, ai, br, bi = _f32(a_re), _f32(a_im), _f32(b_re), _f32(b_im)
    o_re, o_im = np.empty_like(ar), np.empty_like(ar)
    lib().or_cmul_split(_fptr(ar), _fptr(ai), _fptr(br), _fptr(bi), _fptr(o_re), _fptr(o_im), ar.size)
    return o_re, o_im


def deinterleave(x) -> tuple[np.ndarray, np.ndarray]:
    a = _as_c64(x)
    re, im = np.empty(a.size, np.float32), np.empty(a.size, np.float32)
    lib().or_deinterleave(_fptr(a), _fptr(re), _fptr(im), a.size)
    return re, im


def interleave(re, im) -> np.ndarray:
    r, m = _f32(re), _f32(im)
    out = np.empty(r.size, np.complex64)
    lib().or_interleave(_fptr(r), _fptr(m), _fptr(out), r.size)
    return out


def transpose_square(arr, n: int) -> np.ndarray:
    """In-place transpose of an n x n complex64 matrix (cpu_2d.rs:67-73's swap loop)."""
    a = arr if (isinstance(arr, np.ndarray) and arr.dtype == np.complex64 and arr.flags.c_contiguous) \
        else _as_c64(arr)
    assert a.size == n * n
    lib().or_transpose_square(_fptr(a), n)
    return a


def splitmix64_at(seed: int, j: int) -> int:
    return int(lib().or_splitmix64_at(seed & (2**64 - 1), j & (2**64 - 1)))


def fill_uniform_c64(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.complex64)
    lib().or_fill_uniform_c64(_fptr(out), n, seed & (2**64 - 1))
    return out


def fill_normal_c64(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.complex64)
    lib().or_fill_normal_c64(_fptr(out), n, seed & (2**64 - 1))
    return out

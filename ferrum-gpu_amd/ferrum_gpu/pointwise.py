"""ferrum_gpu.pointwise -- elementwise complex kernels on device arrays.

The reference's cmul_interleaved, cmul_split, deinterleave and interleave
(crates/ferrum-gpu-fft-kernels/src/kernels_body.rs:1612-1672).  ``n`` counts
complex elements; arguments are DeviceBuffers, GPU torch tensors or raw device
addresses, and a DeviceBuffer or tensor smaller than what the call reads or
writes (8 bytes per element interleaved, 4 per f32 part) is refused with a
ValueError before anything is launched.  Products are f32 ``re = ar*br - ai*bi``, ``im = ar*bi + ai*br``
without fused multiply-add, as in the reference.  All calls are stream-ordered
and asynchronous.
"""

from __future__ import annotations

import ctypes

from ferrum_gpu import _native as _n
from ferrum_gpu.fft import _ptr_sized as _p
from ferrum_gpu.hip import Device

__all__ = ["cmul", "cmul_split", "deinterleave", "interleave"]


def _s(stream: int) -> ctypes.c_void_p:
    return ctypes.c_void_p(stream or None)


def cmul(device: Device, a, b, out, n: int, stream: int = 0) -> None:
    """out[i] = a[i] * b[i] over n interleaved complex64 elements (out may be a or b)."""
    n = int(n)
    _n.check(_n.lib.fg_cmul_c64(device.handle, _p(a, 8 * n, "a"), _p(b, 8 * n, "b"), _p(out, 8 * n, "out"), n,
                                _s(stream)))


def cmul_split(device: Device, a_re, a_im, b_re, b_im, o_re, o_im, n: int, stream: int = 0) -> None:
    """(o_re, o_im)[i] = (a_re, a_im)[i] * (b_re, b_im)[i] over n elements of float32 arrays."""
    n = int(n)
    parts = [_p(x, 4 * n, name) for x, name in
             ((a_re, "a_re"), (a_im, "a_im"), (b_re, "b_re"), (b_im, "b_im"), (o_re, "o_re"), (o_im, "o_im"))]
    _n.check(_n.lib.fg_cmul_split(device.handle, *parts, n, _s(stream)))


def deinterleave(device: Device, src, re, im, n: int, stream: int = 0) -> None:
    """re[i], im[i] = src[i] for n complex64 elements."""
    n = int(n)
    _n.check(_n.lib.fg_deinterleave_c64(device.handle, _p(src, 8 * n, "src"), _p(re, 4 * n, "re"),
                                        _p(im, 4 * n, "im"), n, _s(stream)))


def interleave(device: Device, re, im, out, n: int, stream: int = 0) -> None:
    """out[i] = (re[i], im[i]) for n elements."""
    n = int(n)
    _n.check(_n.lib.fg_interleave_c64(device.handle, _p(re, 4 * n, "re"), _p(im, 4 * n, "im"),
                                      _p(out, 8 * n, "out"), n, _s(stream)))

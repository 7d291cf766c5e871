"""ferrum_gpu.synthetic -- seeded complex64 test data generated on the device.

``uniform`` fills re/im iid in [-1, 1) on a 2^-23 grid, ``normal`` with
standard normals (Box-Muller in f64); both are counter-based splitmix64
streams, so a seed gives the same array on any device and run.  The
benchmark's configurations use seed = configuration index.  A DeviceBuffer or
tensor smaller than the n * 8 bytes written is refused with a ValueError.
"""

from __future__ import annotations

import ctypes

from ferrum_gpu import _native as _n
from ferrum_gpu.fft import _ptr_sized
from ferrum_gpu.hip import Device

__all__ = ["uniform", "normal"]


def uniform(device: Device, out, n: int, seed: int, stream: int = 0) -> None:
    """Write n complex64 values with re, im iid uniform in [-1, 1) to ``out``."""
    n = int(n)
    _n.check(_n.lib.fg_fill_uniform_c64(device.handle, _ptr_sized(out, 8 * n, "out"), n, int(seed) & (2**64 - 1),
                                        ctypes.c_void_p(stream or None)))


def normal(device: Device, out, n: int, seed: int, stream: int = 0) -> None:
    """Write n complex64 values with re, im iid standard normal to ``out``."""
    n = int(n)
    _n.check(_n.lib.fg_fill_normal_c64(device.handle, _ptr_sized(out, 8 * n, "out"), n, int(seed) & (2**64 - 1),
                                       ctypes.c_void_p(stream or None)))

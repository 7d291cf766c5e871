"""ferrum-gpu for MI355X: batched power-of-two C2C complex64 FFTs on gfx950.

Package layout mirrors the reference's python/ferrum_gpu/__init__.py:3-6
(``version``, ``fft``), with ``hip`` in place of ``cuda``.
"""

from ferrum_gpu._native import version
from ferrum_gpu import hip, fft, pointwise, synthetic

__all__ = ["version", "hip", "fft", "pointwise", "synthetic"]

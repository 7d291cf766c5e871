"""Writes the golden FFT fixtures in this directory (run from the repo root:
``python tests/golden/make_golden.py``).

The reference cross-checks its CPU Stockham against rustfft 6.4.1
(crates/ferrum-gpu-fft/tests/rustfft_cross_check.rs:21-47,
cpu_2d_vs_rustfft.rs:41-67) and its GPU path against numpy.fft
(crates/ferrum-gpu-py/python/tests/test_fft_vs_numpy.py,
test_fft_2d_vs_numpy.py).  rustfft is not available here, so the library
cross-check is anchored on numpy.fft (pocketfft) evaluated in complex128 on
the reference's own deterministic inputs:

  * ``(sin i, cos i)``           -- test_fft_vs_numpy.py:14-19, rustfft_cross_check.rs:31-35
  * ``(sin 0.013 t, cos 0.021 t)`` -- kernel-cross-check.rs:33-40, cpu_radix4.rs:131-136
  * 2D ``(sin 0.1 i, cos 0.07 i)``  -- test_fft_2d_vs_numpy.py:14-16, cpu_2d_vs_rustfft.rs:96-98

plus seeded uniform lanes.  Inputs are stored as complex64 (what the FFT
consumes), expected outputs as complex128.
"""

from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def sin_cos(n: int, a: float = 1.0, b: float = 1.0) -> np.ndarray:
    i = np.arange(n, dtype=np.float32)
    # f32 arguments, as the reference computes them ((i as f32 * a).sin()).
    return (np.sin(i * np.float32(a)) + 1j * np.cos(i * np.float32(b))).astype(np.complex64)


def main() -> None:
    rng = np.random.default_rng(20251201)
    one_d = {}
    for log_n in range(2, 13):
        n = 1 << log_n
        one_d[f"sincos_n{log_n}"] = sin_cos(n)
        if log_n <= 10:  # keeps the fixture file small
            one_d[f"slow_n{log_n}"] = sin_cos(n, 0.013, 0.021)
            u = (rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)).astype(np.complex64)
            one_d[f"unif_n{log_n}"] = u
    out = {}
    for k, x in one_d.items():
        log_n = int(k.rsplit("_n", 1)[1])
        n = 1 << log_n
        lanes = x.astype(np.complex128).reshape(-1, n)
        out[f"in_{k}"] = x
        out[f"fwd_{k}"] = np.fft.fft(lanes, axis=1).reshape(-1)
        # Unnormalised inverse: numpy's ifft divides by N; multiply back.
        out[f"inv_{k}"] = (np.fft.ifft(lanes, axis=1) * n).reshape(-1)
    np.savez_compressed(os.path.join(HERE, "fft1d_numpy.npz"), **out)

    two_d = {}
    for log_n in (2, 3, 4, 5, 6):
        n = 1 << log_n
        base = np.arange(n * n, dtype=np.float32).reshape(n, n)
        x = (np.sin(base * np.float32(0.1)) + 1j * np.cos(base * np.float32(0.07))).astype(np.complex64)
        two_d[f"in_sincos_n{log_n}"] = x
        two_d[f"fwd_sincos_n{log_n}"] = np.fft.fft2(x.astype(np.complex128))
        two_d[f"inv_sincos_n{log_n}"] = np.fft.ifft2(x.astype(np.complex128)) * (n * n)
    np.savez_compressed(os.path.join(HERE, "fft2d_numpy.npz"), **two_d)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()

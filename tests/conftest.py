"""pytest configuration: the `gpu` marker, import paths and shared helpers."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "ferrum-gpu_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


def rel_l2(a, b) -> float:
    """||a - b||_2 / ||b||_2 in float64 (the north star's accuracy metric)."""
    a = np.asarray(a, dtype=np.complex128).reshape(-1)
    b = np.asarray(b, dtype=np.complex128).reshape(-1)
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (nb if nb > 0 else 1.0))


def uniform_c64(rng, size) -> np.ndarray:
    return (rng.uniform(-1, 1, size) + 1j * rng.uniform(-1, 1, size)).astype(np.complex64)


def normal_c64(rng, size) -> np.ndarray:
    return (rng.standard_normal(size) + 1j * rng.standard_normal(size)).astype(np.complex64)


def _gpu_available() -> bool:
    try:
        import ferrum_gpu

        return ferrum_gpu.hip.device_count() > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu_device():
    """One ferrum_gpu.hip.Device(0) for the whole GPU session.

    Without a visible GPU the GPU tests skip (the analogue of the reference's
    FERRUM_GPU_HAS_CUDA gate, crates/ferrum-gpu/tests/round_trip.rs:8-19)
    unless FERRUM_GPU_REQUIRE_GPU=1, in which case they fail.
    """
    if not _gpu_available():
        if os.environ.get("FERRUM_GPU_REQUIRE_GPU") == "1":
            pytest.fail("FERRUM_GPU_REQUIRE_GPU=1 but no HIP device is visible")
        pytest.skip("no HIP device visible")
    import ferrum_gpu

    dev = ferrum_gpu.hip.Device(0)
    print(f"\n[gpu] {dev.info()}", flush=True)
    yield dev
    dev.sync()

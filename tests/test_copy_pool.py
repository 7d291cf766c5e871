"""CPU test of the host path's parallel memcpy (fg::CopyPool,
ferrum-gpu_amd/csrc/host_stage.cpp): a small C++ program linked with the
product's own source copies buffers of awkward sizes (empty, one byte, just
under and over the parallel threshold, unaligned tails) and, from several
threads at once, many buffers -- every byte must arrive.  No GPU call is made.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "ferrum-gpu_amd", "csrc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

PROGRAM = r"""
#include <stdio.h>
#include <string.h>

#include <thread>
#include <vector>

#include "host_stage.hpp"

static bool check(size_t n, unsigned salt) {
    std::vector<unsigned char> a(n + 1), b(n + 1, 0xEE);
    for (size_t i = 0; i < n; ++i) a[i] = (unsigned char)((i * 131u + salt) & 255u);
    fg::CopyPool::get().copy(b.data(), a.data(), n);
    if (n && memcmp(a.data(), b.data(), n) != 0) return false;
    return b[n] == 0xEE;  // nothing written past the end
}

int main() {
    const size_t sizes[] = {0, 1, 4095, 4096, (4u << 20) - 1, 4u << 20, (4u << 20) + 123,
                            (64u << 20) + 4097, (100u << 20) + 7};
    for (size_t n : sizes)
        if (!check(n, 7)) { printf("FAIL size %zu\n", n); return 1; }
    std::vector<std::thread> ts;
    std::vector<int> ok(6, 1);
    for (int t = 0; t < 6; ++t)
        ts.emplace_back([t, &ok] {
            for (int r = 0; r < 6; ++r)
                if (!check((10u << 20) + 977u * t + r, (unsigned)(t * 17 + r))) ok[t] = 0;
        });
    for (auto& th : ts) th.join();
    for (int t = 0; t < 6; ++t)
        if (!ok[t]) { printf("FAIL thread %d\n", t); return 1; }
    printf("OK threads=%u\n", fg::CopyPool::get().threads());
    return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None or not os.path.exists(os.path.join(ROCM, "lib", "libamdhip64.so")),
                    reason="needs g++ and the ROCm runtime library to link")
def test_copy_pool_copies_every_byte(tmp_path):
    src = tmp_path / "copy_pool_check.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "copy_pool_check"
    cmd = ["g++", "-O2", "-std=c++17", "-pthread", "-D__HIP_PLATFORM_AMD__", f"-I{CSRC}",
           f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(ROCM, 'include')}", str(src),
           os.path.join(CSRC, "host_stage.cpp"), os.path.join(CSRC, "hip_backend.cpp"),
           f"-L{os.path.join(ROCM, 'lib')}", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-lamdhip64",
           "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=180)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=180)
    assert run.returncode == 0 and run.stdout.startswith("OK"), run.stdout + run.stderr

"""CPU checks of the launch-size bound (ferrum-gpu_amd/csrc/launch_limits.h).

One HIP launch covers at most 2^32 - 1 work-items along a dimension (the AQL
dispatch packet's 32-bit grid size) and 2^31 - 1 workgroups; the reference
instead passes `batch as u32` as its grid and wraps silently
(crates/ferrum-gpu-py/src/lib.rs:147).  The header's C functions are compiled
here with gcc and compared with a direct statement of the bound, including the
edge cases a plan meets: N = 4 transforms (64 per 64-thread workgroup), the
largest batch before a second launch, and units that alone exceed a launch.
"""

from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR_DIR = os.path.join(ROOT, "ferrum-gpu_amd", "csrc")

MAX_ITEMS, MAX_BLOCKS = 2**32 - 1, 2**31 - 1

PROG = r"""
#include <stdio.h>
#include <inttypes.h>
#include "launch_limits.h"
int main(void) {
    uint64_t a, b, c;
    while (scanf("%" SCNu64 " %" SCNu64 " %" SCNu64, &a, &b, &c) == 3)
        printf("%d %" PRIu64 "\n", fg_launch_fits(a, c), fg_max_units_per_launch(a, b, c));
    return 0;
}
"""

CASES = [
    # (blocks_per_unit or blocks, units_per_block, threads)
    (1, 64, 64),          # N = 4: 64 transforms per 64-thread workgroup
    (1, 2, 128),          # N = 1024 throughput kernel: two transforms per 128 threads
    (1, 1, 1024),         # N = 32768: one transform per 1024 threads
    (2048, 1, 256),       # a 4096 x 4096 image's row-pair pass: 2048 workgroups per image
    (512, 1, 1024),       # a 2048-row column pass: 512 tiles per image
    (2**31, 1, 1),        # more workgroups than a grid holds
    (2**24, 1, 1024),     # one unit alone exceeds the work-item bound
    (1, 1, 1025),         # beyond the workgroup size
    (0, 1, 64), (1, 0, 64), (1, 1, 0),
]


def fits(blocks, threads):
    return int(1 <= blocks <= MAX_BLOCKS and 1 <= threads <= 1024 and blocks * threads <= MAX_ITEMS)


def max_units(bpu, upb, threads):
    if bpu == 0 or upb == 0 or threads == 0 or threads > 1024:
        return 0
    blocks = min(MAX_ITEMS // threads, MAX_BLOCKS)
    return blocks * upb // bpu


@pytest.fixture(scope="module")
def limits_bin(tmp_path_factory):
    d = tmp_path_factory.mktemp("limits")
    src, exe = d / "limits.c", d / "limits"
    src.write_text(PROG)
    subprocess.run(["gcc", "-std=c99", "-O2", "-Wall", "-Werror", f"-I{HDR_DIR}", str(src), "-o", str(exe)],
                   check=True)
    return str(exe)


def run(exe, cases):
    inp = "".join(f"{a} {b} {c}\n" for a, b, c in cases)
    out = subprocess.run([exe], input=inp, capture_output=True, text=True, check=True).stdout.split("\n")
    return [tuple(int(v) for v in line.split()) for line in out if line.strip()]


def test_header_matches_the_bound(limits_bin):
    got = run(limits_bin, CASES)
    want = [(fits(a, c), max_units(a, b, c)) for a, b, c in CASES]
    assert got == want


def test_largest_batches_in_one_launch(limits_bin):
    # N = 4 at 64 transforms per 64-thread workgroup: 2^32 - 64 transforms
    # fit one launch, 2^32 take two; a launch of the maximum is exactly at
    # the work-item bound's floor
    (fits1, units), = run(limits_bin, [(1, 64, 64)])
    assert units == (MAX_ITEMS // 64) * 64 == 2**32 - 64
    assert -(-2**32 // units) == 2
    assert run(limits_bin, [(units // 64, 1, 64), (units // 64 + 1, 1, 64)]) == [
        (1, max_units(units // 64, 1, 64)), (0, max_units(units // 64 + 1, 1, 64))]


def test_every_work_item_count_below_the_bound_fits(limits_bin):
    # blocks * threads just below, at and above 2^32 for each block size a
    # plan uses
    cases = []
    for threads in (32, 64, 128, 256, 512, 1024):
        top = MAX_ITEMS // threads
        cases += [(top - 1, 1, threads), (top, 1, threads), (top + 1, 1, threads)]
    got = [f for f, _ in run(limits_bin, cases)]
    assert got == [fits(a, c) for a, _, c in cases]
    assert got[1::3] == [1] * 6 and got[2::3] == [0] * 6


def test_plan_and_backend_use_the_header():
    plan = open(os.path.join(HDR_DIR, "fft_plan.cpp")).read()
    backend = open(os.path.join(HDR_DIR, "hip_backend.cpp")).read()
    assert '#include "launch_limits.h"' in plan and "fg_max_units_per_launch" in plan
    assert '#include "launch_limits.h"' in backend and "FG_MAX_LAUNCH_ITEMS" in backend
    # no launch falls back to a plain launch beyond the bound
    assert "Beyond the extension's 32-bit work sizes" not in backend

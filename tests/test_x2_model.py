"""CPU model of the 1024-point throughput kernel (fft1024_x2_body in
ferrum-gpu_amd/csrc/kernels/fft_stockham.hpp: fg_fft_n10, _split, _sc),
checked against the oracle before any launch.

A workgroup of 128 threads holds two transforms; thread t loads position
t + 128 p (p < 8) of each.  The radix list is 8 * 16 * 8:
  stage 0 (R 8, L 1):    butterfly t of each transform, outputs to 8 t + q;
  stage 1 (R 16, L 8):   thread t runs butterfly b = t % 64 of transform
                         t / 64, positions b + 64 m, twiddles W_128^{p (b % 8)};
  stage 2 (R 8, L 128):  butterfly t of each transform, positions t + 128 p,
                         twiddles W_1024^{p t}, outputs to t + 128 q.
The model keeps the kernel's LDS slots (one pad per 16 positions, per
transform 1024 + 64 slots) and the strides it writes them with, checks every
write in bounds and distinct, every read of a slot written in the same phase,
and forms the twiddles from the host's table (fft1024_x2_twiddles in
fft_plan.cpp) the way apply_stage_twiddles does.  Only the DFT-R is numpy's.
"""

from __future__ import annotations

import os
import re

import numpy as np
import pytest

import oracle
from conftest import rel_l2, uniform_c64
from test_stockham_model import lds_pos, stage_twiddles

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SLOTS = 1024 + 64


def x2_table():
    """fft1024_x2_twiddles: 8 rows of W_128^{p k} (p in 1,2,3,4,8,12), then
    128 rows of W_1024^{p k} (p in 1,2,3,4), complex64."""
    k, p = np.meshgrid(np.arange(8), [1, 2, 3, 4, 8, 12], indexing="ij")
    a = np.exp(-2j * np.pi * ((p * k) % 128) / 128).reshape(-1)
    k, p = np.meshgrid(np.arange(128), [1, 2, 3, 4], indexing="ij")
    b = np.exp(-2j * np.pi * ((p * k) % 1024) / 1024).reshape(-1)
    return np.concatenate([a, b]).astype(np.complex64)


def x2_model(x, batch):
    """x: (batch * 1024,) complex; returns the kernel's output for every workgroup."""
    tw = x2_table()
    assert tw.size == 48 + 512
    lanes = x.reshape(batch, 1024).astype(np.complex128)
    t = np.arange(128)
    out = np.zeros_like(lanes)
    for wg in range((batch + 1) // 2):
        f0 = 2 * wg
        has1 = f0 + 1 < batch
        pos = t[:, None] + 128 * np.arange(8)[None, :]             # (t, p)
        regs = [lanes[f0][pos], lanes[f0 + 1][pos] if has1 else np.zeros((128, 8))]
        # stage 0: DFT-8 over p, output q to 8 t + q
        lds = np.zeros((2, SLOTS), np.complex128)
        wr = np.zeros((2, SLOTS), bool)
        for f in range(2):
            y = np.fft.fft(regs[f], axis=1)
            idx = lds_pos(8 * t[:, None] + np.arange(8)[None, :])
            assert idx.max() < SLOTS and not wr[f][idx].any() and len(np.unique(idx)) == idx.size
            wr[f][idx] = True
            lds[f][idx] = y
        assert np.array_equal(wr.sum(axis=1), [1024, 1024])
        # stage 1: thread t reads lds[g][lds_pos(b) + 68 m]
        g, b = t >> 6, t & 63
        k = b & 7
        src = lds_pos(b)[:, None] + 68 * np.arange(16)[None, :]
        assert np.array_equal(src, lds_pos(b[:, None] + 64 * np.arange(16)[None, :]))
        assert wr[g[:, None], src].all()
        u = lds[g[:, None], src]
        u = u * stage_twiddles(tw, 0, k, 16)
        w_exact = np.exp(-2j * np.pi * (k[:, None] * np.arange(16)[None, :]) / 128)
        assert np.max(np.abs(stage_twiddles(tw, 0, k, 16) - w_exact)) < 3e-7
        y = np.fft.fft(u, axis=1)
        lds2 = np.zeros((2, SLOTS), np.complex128)
        wr2 = np.zeros((2, SLOTS), bool)
        d0 = (b >> 3) * 128 + k
        dst = lds_pos(d0)[:, None] + 8 * np.arange(16)[None, :] + (np.arange(16)[None, :] >> 1)
        # the Stockham scatter j L R + k + q L with L = 8, R = 16, j = b / 8
        assert np.array_equal(dst, lds_pos(d0[:, None] + 8 * np.arange(16)[None, :]))
        for gg in range(2):
            sel = g == gg
            d = dst[sel]
            assert d.max() < SLOTS and not wr2[gg][d].any() and len(np.unique(d)) == d.size
            wr2[gg][d] = True
            lds2[gg][d] = y[sel]
        assert wr2.sum() == 2 * 1024
        # stage 2: thread t reads lds[f][lds_pos(t) + 136 p], twiddles W_1024^{p t}
        for f in range(2):
            src = lds_pos(t)[:, None] + 136 * np.arange(8)[None, :]
            assert np.array_equal(src, lds_pos(t[:, None] + 128 * np.arange(8)[None, :]))
            assert wr2[f][src].all()
            u = lds2[f][src] * stage_twiddles(tw, 48, t, 8)
            w_exact = np.exp(-2j * np.pi * (t[:, None] * np.arange(8)[None, :]) / 1024)
            assert np.max(np.abs(stage_twiddles(tw, 48, t, 8) - w_exact)) < 3e-7
            assert 48 + 4 * 127 + 4 <= tw.size
            y = np.fft.fft(u, axis=1)
            if f == 0 or has1:
                out[f0 + f][t[:, None] + 128 * np.arange(8)[None, :]] = y
    return out.reshape(-1)


@pytest.mark.parametrize("batch", [1, 2, 3, 6])
def test_x2_model_matches_oracle(batch):
    # odd batches: the last workgroup holds one transform and stores only it
    rng = np.random.default_rng(batch)
    x = uniform_c64(rng, batch * 1024)
    got = x2_model(x, batch)
    want = oracle.fft_1d(x, 10)
    assert rel_l2(got, want) < 1e-6


def test_x2_table_matches_the_host_builder():
    # fft1024_x2_twiddles in fft_plan.cpp: the same rows, the same exponents
    src = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "fft_plan.cpp")).read()
    body = re.search(r"std::vector<Cf32> fft1024_x2_twiddles\(\) \{(.*?)\n\}", src, flags=re.S).group(1)
    assert "for (uint64_t k = 0; k < 8; ++k)" in body and "{1, 2, 3, 4, 8, 12}" in body and "w(128, p * k)" in body
    assert "for (uint64_t k = 0; k < 128; ++k)" in body and "{1, 2, 3, 4}" in body and "w(1024, p * k)" in body


def test_x2_kernel_shape():
    # 128 threads, two transforms, 2 * (1024 + 64) LDS slots of 8 bytes (17 KiB):
    # kStockham[10] = {4, 2} launches exactly that block
    hip = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "kernels", "fft_stockham.hpp")).read()
    assert "__shared__ float2 lds[2][1024 + 64];" in hip
    assert ((1024 >> 4) * 2) == 128 and 2 * SLOTS * 8 == 17408

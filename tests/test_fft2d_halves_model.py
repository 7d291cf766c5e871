"""CPU model of the one-pass 2D FFT of 2048- to 16384-point images with the
exchanges in halves (fft2d_halves_body in
ferrum-gpu_amd/csrc/kernels/fft_2d_halves.hpp), checked against the oracle
before any launch.

One workgroup of T = N/32 threads holds one image of R x C = 2^lr x 2^lc
points (11 <= lr + lc <= 14) in registers, 32 per thread at positions t + T m of the
row-major image (coalesced loads).  The 2D DFT is a 1D Stockham pass over all
N positions whose radix list is the row-length digits' list for R (16, ..,
16, r), then C's: the first block takes the DFT over the row index (the top
lr bits of a position), twiddles W_{L R_s}^{p k} as in 1D; the second block
takes the DFT over the column index with no twiddle between the two blocks:
its stage twiddles are C's own, W_{Ld R_s}^{p (k >> lr)} (Ld the product of
the block's earlier radices).  The autosort leaves output (k_r, k_c) at
position k_r + R k_c; a last exchange moves it to k_r C + k_c so that the
stores are the same coalesced rows as the loads.  Every exchange runs in two
rounds through N/2 + N/32 LDS slots: round h writes what lands in half h and
every thread then reads its elements m in [16h, 16h + 16).  The model checks
every round's writes inside its half, distinct and in bounds, every read
written in the same round, and the result against the oracle; only the DFT-R
is numpy's, the twiddles come from the host's stage tables.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rel_l2, uniform_c64
from test_stockham_model import stage_twiddles, stockham_table

E = 32


def radices(bits):
    return [16] * (bits // 4) + ([1 << (bits % 4)] if bits % 4 else [])


def stage_list(lr, lc):
    """(dim, R, L, Ld, sd): L over the whole list, Ld and sd within the dimension."""
    out, L = [], 1
    for dim, bits in (("r", lr), ("c", lc)):
        ld = 1
        for sd, r in enumerate(radices(bits)):
            out.append((dim, r, L, ld, sd))
            L *= r
            ld *= r
    return out


def lds_pos(p):
    return p + (p >> 4)


def model(images, lr, lc):
    """images: (B, N) complex, row-major; returns the kernel's (B, N) output."""
    b_, n = images.shape
    assert n == 1 << (lr + lc) and 11 <= lr + lc <= 14
    T, half = n // E, n // 2
    slots = half + half // 16
    nr, nc = 1 << lr, 1 << lc
    twr, offr = stockham_table(lr, 4)
    twc, offc = stockham_table(lc, 4)
    t = np.arange(T)
    natural = t[:, None] + T * np.arange(E)[None, :]
    regs = images.astype(np.complex128)[:, natural]
    stages = stage_list(lr, lc)

    def exchange(out, dst, pos=lds_pos):
        """Two rounds: writes of outputs whose destination lies in half h, then
        reads of positions t + T m, m in [16h, 16h + 16); `pos`: the slot of a
        position within the half."""
        new = np.empty_like(out)
        for h in range(2):
            lds = np.zeros((b_, slots), np.complex128)
            written = np.zeros(slots, dtype=bool)
            sel = (dst >= half * h) & (dst < half * (h + 1))
            # every thread's outputs in half h are exactly its round-h writes
            idx = pos(dst[sel] - half * h)
            assert idx.max() < slots and len(np.unique(idx)) == idx.size == half
            written[idx] = True
            lds[:, idx] = out[:, sel]
            for m in range(E // 2):
                ridx = pos(t + T * m)
                assert written[ridx].all()
                new[:, :, (E // 2) * h + m] = lds[:, ridx]
        return new

    for s, (dim, R, L, ld, sd) in enumerate(stages):
        NB = E // R
        out = np.empty_like(regs)
        dst = np.empty((T, E), dtype=np.int64)
        for i in range(NB):
            u = regs[:, :, [i + NB * p for p in range(R)]]
            b = t + T * i
            k = b & (L - 1)
            if ld > 1:
                if dim == "r":
                    u = u * stage_twiddles(twr, offr[sd], k, R, ld)[None, :, :]
                else:
                    u = u * stage_twiddles(twc, offc[sd], k >> lr, R, ld)[None, :, :]
            y = np.fft.fft(u, axis=2)
            j = b // L
            for q in range(R):
                out[:, :, i + NB * q] = y[:, :, q]
                dst[:, i + NB * q] = j * L * R + k + q * L
            # before the last stage (L R <= N/2), butterflies i < NB/2 write the lower half
            if s + 1 < len(stages):
                assert np.all((dst[:, i + NB * np.arange(R)] < half) == (i < NB // 2))
        assert np.array_equal(np.sort(dst.reshape(-1)), np.arange(n))
        if s + 1 == len(stages):
            assert np.array_equal(dst, natural)
            regs = out
            break
        regs = exchange(out, dst)
    # output (k_r, k_c) sits at position k_r + R k_c; move it to k_r C + k_c
    P = natural
    Q = (P % nr) * nc + P // nr
    regs = exchange(regs, Q, pos=lambda q: q + q // nc)   # one pad slot per output row
    res = np.empty((b_, n), np.complex128)
    res[:, natural] = regs
    return res


SHAPES = [(lr, bits - lr) for bits in (11, 12, 13, 14) for lr in range(4, bits - 3)]


@pytest.mark.parametrize("lr,lc", SHAPES)
def test_model_matches_oracle(lr, lc):
    rng = np.random.default_rng(lr * 16 + lc)
    n = 1 << (lr + lc)
    x = uniform_c64(rng, 2 * n)
    got = model(x.reshape(2, n), lr, lc).reshape(-1)
    want = np.stack([np.fft.fft2(x[i * n:(i + 1) * n].reshape(1 << lr, 1 << lc)).reshape(-1) for i in range(2)])
    assert rel_l2(got, want.reshape(-1)) < 1e-5
    if lr == lc:
        assert rel_l2(got, oracle.fft_2d(x, lr)) < 1e-5


def test_transposing_exchange_round_of_each_output():
    # the kernel's round for output m of thread t in the last exchange:
    # k_r = (t + T m) mod R in the upper half of the rows -> round 1, i.e.
    # Q = k_r C + k_c in the upper half of the image; for R <= T = 512 the
    # round is the same for all 32 outputs of a thread, for R = 1024 it is m's parity
    for lr, lc in SHAPES:
        nr, nc, n = 1 << lr, 1 << lc, 1 << (lr + lc)
        T = n // E
        t = np.arange(T)
        P = t[:, None] + T * np.arange(E)[None, :]
        Q = (P % nr) * nc + P // nr
        rnd = (P % nr) >= nr // 2
        assert np.array_equal(rnd, Q >= n // 2)
        if nr <= T:
            assert np.array_equal(rnd, np.repeat(((t % nr) >= nr // 2)[:, None], E, axis=1))
        else:
            assert np.array_equal(rnd, np.broadcast_to(np.arange(E)[None, :] % 2 == 1, rnd.shape))


def test_transposing_exchange_slots():
    # the kernel's closed forms for the last exchange's slots equal
    # tpos(Q - HALF h) = Q' + Q' / C, and a wave's 16-lane groups of writes
    # hit 16 distinct bank pairs (32 four-byte banks, 8-byte slots)
    for lr, lc in SHAPES:
        nr, nc, n = 1 << lr, 1 << lc, 1 << (lr + lc)
        T = n // E
        t = np.arange(T)
        for h in range(2):
            for m in range(E):
                P = t + T * m
                Q = (P % nr) * nc + P // nr - (n // 2) * h
                mine = ((P % nr) >= nr // 2) == (h == 1)
                if nr <= T:
                    q0 = (t & (nr - 1)) * nc + (t >> lr) - (n // 2) * h
                    slot = q0 + q0 // nc + (T // nr) * m
                else:
                    slot = t * (nc + 1) + (m >> 1)
                assert np.array_equal(slot[mine], (Q + Q // nc)[mine])
                for g in range(0, T, 16):
                    lanes = np.arange(g, g + 16)
                    lanes = lanes[mine[lanes]]
                    if len(lanes) > 1:
                        assert len(set((2 * slot[lanes]) % 32)) == len(lanes), (lr, h, m, g)
        for m in range(E // 2):
            R = t + T * m
            read = t + t // nc + m * (T + T // nc) if nc <= T else t + T * m + m // 2
            assert np.array_equal(read, R + R // nc)

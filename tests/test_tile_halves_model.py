"""CPU model of the tile pass that exchanges in halves (fft_tile_halves_body
in ferrum-gpu_amd/csrc/kernels/fft_tile.hpp), checked against the oracle
before any launch.

A tile holds G columns of L = 2^LOGL points; T = L/32 threads per column
hold 32 elements each, thread t at positions t + T*m.  Stage s (radix
R = 16, ..., 16, r; L_s = the product of the earlier radices) runs NB = 32/R
butterflies b = t + T*i per thread.  Butterfly b writes to
j*L_s*R + k + q*L_s (j = b / L_s, k = b % L_s), which lies below L/2 exactly
when i < NB/2, so each exchange runs in two rounds through an LDS tile of
L/2 positions: round h writes butterflies i in [h*NB/2, (h+1)*NB/2), then
every thread reads its elements m in [16h, 16h + 16).  The model keeps that
bookkeeping with the kernel's LDS layout (positions x columns, pitch G + 1;
G >= 16) and checks every write in bounds and distinct
within its round, every read written in the same round, and the last
stage's outputs at the thread's own positions t + T*m.  Only the DFT-R is
numpy's; the stage twiddles come from the host's table for the radix list.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rel_l2, uniform_c64
from test_stockham_model import stage_twiddles, stockham_table

E = 32


def radices(log_l):
    return [16] * (log_l // 4) + ([1 << (log_l % 4)] if log_l % 4 else [])


def lds_index(pos, c, g):
    """TileLayout<LOGL - 1, G>::at for G >= 16."""
    assert g >= 16
    return pos * (g + 1) + c


def lds_elems(log_l, g):
    return (1 << (log_l - 1)) * (g + 1)


def halves_model(cols, log_l):
    """cols: (G, L) complex; returns the kernel's (G, L) output."""
    g, n = cols.shape
    assert n == 1 << log_l
    T, half = n // E, n // 2
    tw, offs = stockham_table(log_l, 4)
    t = np.arange(T)
    natural = t[:, None] + T * np.arange(E)[None, :]
    regs = cols.astype(np.complex128)[:, natural]          # regs[c, t, m]: position t + T*m
    rs = radices(log_l)
    L = 1
    for s, R in enumerate(rs):
        NB = E // R
        out = np.empty_like(regs)
        dst = np.empty((T, E), dtype=np.int64)
        for i in range(NB):
            u = regs[:, :, [i + NB * p for p in range(R)]]
            b = t + T * i
            k = b & (L - 1)
            if L > 1:
                u = u * stage_twiddles(tw, offs[s], k, R)[None, :, :]
            y = np.fft.fft(u, axis=2)
            j = b // L
            for q in range(R):
                out[:, :, i + NB * q] = y[:, :, q]
                dst[:, i + NB * q] = j * L * R + k + q * L
        assert np.array_equal(np.sort(dst.reshape(-1)), np.arange(n))
        if s + 1 == len(rs):
            assert np.array_equal(dst, natural)
            regs = out
            break
        new = np.empty_like(regs)
        lds = np.zeros(lds_elems(log_l, g), np.complex128)
        for h in range(2):
            written = np.zeros(lds.size, dtype=bool)
            for i in range(h * NB // 2, (h + 1) * NB // 2):
                for q in range(R):
                    d = dst[:, i + NB * q]
                    assert np.all((d >= half * h) & (d < half * (h + 1))), (log_l, s, i, q)
                    for c in range(g):
                        idx = lds_index(d - half * h, c, g)
                        assert idx.max() < lds.size
                        assert not written[idx].any()
                        written[idx] = True
                        lds[idx] = out[c, :, i + NB * q]
            assert written.sum() == half * g
            for m in range(E // 2):
                for c in range(g):
                    idx = lds_index(t + T * m, c, g)
                    assert written[idx].all()
                    new[c, :, (E // 2) * h + m] = lds[idx]
        regs = new
        L *= R
    res = np.empty((g, n), np.complex128)
    res[:, natural] = regs
    return res


# (log_l, G): the instantiated kernels (FG_TILE_HALVES), the widths of the
# passes that read HBM
CASES = [(7, 64), (8, 32), (9, 16), (10, 16)]


@pytest.mark.parametrize("log_l,g", CASES)
def test_halves_model_matches_oracle(log_l, g):
    rng = np.random.default_rng(log_l * 100 + g)
    n = 1 << log_l
    cols = uniform_c64(rng, g * n).reshape(g, n)
    got = halves_model(cols, log_l)
    want = oracle.fft_1d(cols.reshape(-1), log_l).reshape(g, n)
    assert rel_l2(got, want) < 1e-5


@pytest.mark.parametrize("log_l,g", [(7, 64), (8, 32), (9, 16), (10, 16)])
def test_halves_tiles_halve_the_lds(log_l, g):
    # the LDS of a half tile, against the whole-tile layout of the 16-element kernel
    whole = (1 << log_l) * (g + 1) * 8
    assert lds_elems(log_l, g) * 8 * 2 == whole
    assert g * ((1 << log_l) // E) <= 1024

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
bookkeeping with the kernel's LDS layouts (TileLayout<LOGL - 1, G>: positions
x columns with pitch G + 1 for G >= 16; pitch G with one pad row per 16
positions for the narrow 1024- to 4096-point tiles, G = 8), forms every write
address the way halves_exchange does (a base at the butterfly's first output
plus q times a compile-time step) and every read address as a base plus m
times step<T>, checks each against the layout's own index of the position,
every write in bounds and distinct within its round, every read written in
the same round, and the last stage's outputs at the thread's own positions
t + T*m.  Only the DFT-R is numpy's; the stage twiddles come from the host's
table for the radix list.
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
    """TileLayout<LOGL - 1, G>::at: pitch G + 1 for G >= 16, else lds_pos(pos) * G."""
    if g < 16:
        return (pos + (pos >> 4)) * g + c
    return pos * (g + 1) + c


def lds_elems(log_l, g):
    half = 1 << (log_l - 1)
    return (half + half // 16) * g if g < 16 else half * (g + 1)


def layout_step(d, g):
    """TileLayout::step<D>: at(pos + D, c) - at(pos, c) for D a multiple of 16."""
    if g < 16:
        assert d % 16 == 0
        return (d + d // 16) * g
    return d * (g + 1)


def scatter_step(L, g):
    """halves_scatter_step: the step between a butterfly's outputs q and q + 1."""
    return g if (g < 16 and L == 1) else layout_step(L, g)


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
        assert g >= 16 or L > 1 or R == 16
        for h in range(2):
            written = np.zeros(lds.size, dtype=bool)
            for i in range(h * NB // 2, (h + 1) * NB // 2):
                b = t + T * i
                d0 = (b >> (4 * s)) * L * R + (b & (L - 1)) - half * h
                for q in range(R):
                    d = dst[:, i + NB * q]
                    assert np.all((d >= half * h) & (d < half * (h + 1))), (log_l, s, i, q)
                    for c in range(g):
                        idx = lds_index(d0, c, g) + q * scatter_step(L, g)
                        assert np.array_equal(idx, lds_index(d - half * h, c, g))
                        assert idx.max() < lds.size
                        assert not written[idx].any()
                        written[idx] = True
                        lds[idx] = out[c, :, i + NB * q]
            assert written.sum() == half * g
            for m in range(E // 2):
                for c in range(g):
                    idx = lds_index(t, c, g) + m * layout_step(T, g)
                    assert np.array_equal(idx, lds_index(t + T * m, c, g))
                    assert written[idx].all()
                    new[c, :, (E // 2) * h + m] = lds[idx]
        regs = new
        L *= R
    res = np.empty((g, n), np.complex128)
    res[:, natural] = regs
    return res


def row_halves_model(lanes, log_n):
    """The single-pass 8192 / 16384 / 32768-point kernel (fft_row_halves_body): the same
    stages on one contiguous transform per workgroup, the LDS holding L/2
    positions with one pad slot per 16 (lds_pos); lanes: (B, L) complex."""
    b_, n = lanes.shape
    T, half = n // E, n // 2
    tw, offs = stockham_table(log_n, 4)
    t = np.arange(T)
    natural = t[:, None] + T * np.arange(E)[None, :]
    regs = lanes.astype(np.complex128)[:, natural]
    rs = radices(log_n)
    slots = half + half // 16
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
                u = u * stage_twiddles(tw, offs[s], k, R, L)[None, :, :]
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
        assert R == 16
        new = np.empty_like(regs)
        for h in range(2):
            lds = np.zeros((b_, slots), np.complex128)
            written = np.zeros(slots, dtype=bool)
            for i in range(h * NB // 2, (h + 1) * NB // 2):
                b = t + T * i
                for q in range(R):
                    d = dst[:, i + NB * q]
                    assert np.all((d >= half * h) & (d < half * (h + 1))), (log_n, s, i, q)
                    # the kernel's slot: stage 0 writes 17 * (b - HALF/16 * h) + q,
                    # later stages lds_pos(d0) + q * (L + L/16)
                    if L == 1:
                        idx = 17 * (b - (half // 16) * h) + q
                    else:
                        d0 = (b >> (4 * s)) * L * 16 + (b & (L - 1)) - half * h
                        idx = d0 + (d0 >> 4) + q * (L + L // 16)
                    assert np.array_equal(idx, (d - half * h) + ((d - half * h) >> 4))
                    assert idx.max() < slots and not written[idx].any()
                    written[idx] = True
                    lds[:, idx] = out[:, :, i + NB * q]
            assert written.sum() == half
            for m in range(E // 2):
                idx = (t + t // 16) + m * (T + T // 16)
                assert np.array_equal(idx, (t + T * m) + ((t + T * m) >> 4))
                assert written[idx].all()
                new[:, :, (E // 2) * h + m] = lds[:, idx]
        regs = new
        L *= R
    res = np.empty((b_, n), np.complex128)
    res[:, natural] = regs
    return res


@pytest.mark.parametrize("log_n", [13, 14, 15])
def test_row_halves_model_matches_oracle(log_n):
    rng = np.random.default_rng(log_n)
    n = 1 << log_n
    lanes = uniform_c64(rng, 2 * n).reshape(2, n)
    got = row_halves_model(lanes, log_n)
    want = oracle.fft_1d(lanes.reshape(-1), log_n).reshape(2, n)
    assert rel_l2(got, want) < 1e-5


@pytest.mark.parametrize("log_n", [13, 14, 15])
def test_row_halves_fit_the_hardware(log_n):
    # N/32 threads (at most 1024), N/2 + N/32 LDS slots: at least two
    # workgroups per CU up to 16384 points, one (136 KB) at 32768
    n = 1 << log_n
    assert n // E <= 1024
    lds = (n // 2 + n // 32) * 8
    assert (2 if log_n < 15 else 1) * lds <= 160 * 1024, lds


# (log_l, G): the instantiated kernels, FG_TILE_HALVES (the widths of the
# passes that read HBM), the 1D middle pass of 256 points (16 columns) and
# FG_TILE_HALVES_NARROW (2D columns of 1024 .. 4096 points)
CASES = [(7, 64), (8, 32), (8, 16), (9, 16), (10, 16), (10, 8), (11, 8), (12, 8)]


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


@pytest.mark.parametrize("log_l,g,threads,kib", [(10, 8, 256, 34), (11, 8, 512, 68), (12, 8, 1024, 136)])
def test_narrow_halves_tiles_fit_a_cu(log_l, g, threads, kib):
    # twice the columns of the 16-element narrow tiles (8 / 4) in the same or
    # half the LDS; the layout is injective and inside its array
    assert g * ((1 << log_l) // E) == threads
    assert lds_elems(log_l, g) * 8 == kib * 1024 <= 160 * 1024
    half = 1 << (log_l - 1)
    pos, c = np.meshgrid(np.arange(half), np.arange(g), indexing="ij")
    idx = lds_index(pos, c, g)
    assert len(np.unique(idx)) == half * g and idx.max() < lds_elems(log_l, g)


def test_narrow_halves_kernels_are_instantiated():
    import os
    import re
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = open(os.path.join(root, "ferrum-gpu_amd", "csrc", "kernels", "fft_kernels.hip")).read()
    got = {(int(a), int(b)) for a, b in re.findall(r"^FG_TILE_HALVES_NARROW\((\d+), (\d+)\)", src, flags=re.M)}
    assert got == {(11, 8), (12, 8)}
    hpp = open(os.path.join(root, "ferrum-gpu_amd", "csrc", "kernels", "fft_tile.hpp")).read()
    assert "if constexpr (Lay::PADPOS && L == 1) return G;" in hpp


def row_tile_load_model(rows, log_l, g):
    """The row-wise input of fft_tile_halves_body (ROWWISE = true, the 1D last
    passes fg_tile_l{9,10}_g16_rh): thread tid = c + G t issues all E loads
    along the rows first -- y[m] is linear element li = tid + THREADS (m mod
    E/2) of half h = m / (E/2), i.e. row li / HALF at position HALF h + li mod
    HALF -- then each half goes through the LDS tile (TileLayout<LOGL - 1, G>)
    into x[E/2 h + m] = position t + T (E/2 h + m) of column c.  Checks every
    write in bounds and distinct within its half, every read written in the
    same half, each read address formed as the kernel forms it, and each
    wave's loads in at most two contiguous runs; returns regs[c, t, m]."""
    n = 1 << log_l
    T, half = n // E, n // 2
    threads = g * T
    assert g * half == threads * (E // 2)
    tid = np.arange(threads)
    y = np.empty((threads, E), np.complex64)
    for m in range(E):
        h = m // (E // 2)
        li = tid + threads * (m % (E // 2))
        row, pos = li >> (log_l - 1), half * h + (li & (half - 1))
        assert row.max() < g and pos.max() < n
        for w in range(0, threads, 64):
            flat = row[w:w + 64] * n + pos[w:w + 64]
            assert np.count_nonzero(np.diff(flat) != 1) <= 1   # one row end per wave at most
        y[:, m] = rows[row, pos]
    c, t = tid % g, tid // g
    regs = np.empty((g, T, E), np.complex64)
    for h in range(2):
        lds = np.zeros(lds_elems(log_l, g), np.complex64)
        written = np.zeros(lds.size, dtype=bool)
        for m in range(E // 2):
            li = tid + threads * m
            idx = lds_index(li & (half - 1), li >> (log_l - 1), g)
            assert idx.max() < lds.size and len(np.unique(idx)) == threads
            assert not written[idx].any()
            written[idx] = True
            lds[idx] = y[:, (E // 2) * h + m]
        assert written.sum() == half * g
        for m in range(E // 2):
            idx = lds_index(t, c, g) + m * layout_step(T, g)
            assert np.array_equal(idx, lds_index(t + T * m, c, g))
            assert written[idx].all()
            regs[c, t, (E // 2) * h + m] = lds[idx]
    return regs


@pytest.mark.parametrize("log_l,g", [(8, 32), (9, 16), (10, 16)])
def test_row_tile_load_transposes_each_half(log_l, g):
    # the transposed load hands each thread its Stockham positions t + T m
    # bit for bit, so the stages are those of the column tile above
    n = 1 << log_l
    rng = np.random.default_rng(log_l)
    rows = uniform_c64(rng, g * n).reshape(g, n)
    T = n // E
    natural = np.arange(T)[:, None] + T * np.arange(E)[None, :]
    assert np.array_equal(row_tile_load_model(rows, log_l, g), rows[:, natural])
    got = halves_model(rows, log_l)
    assert rel_l2(got, oracle.fft_1d(rows.reshape(-1), log_l).reshape(g, n)) < 1e-5


def test_row_halves_tiles_fit_and_are_instantiated():
    import os
    import re
    from test_multipass_model import use_row_halves_tile
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = open(os.path.join(root, "ferrum-gpu_amd", "csrc", "kernels", "fft_kernels.hip")).read()
    got = set(re.findall(r"^FG_TILE_ROW_HALVES\((\d+), (\d+), (\w*),", src, flags=re.M))
    assert got == {(l, g, p) for l, g in (("8", "32"), ("9", "16"), ("10", "16")) for p in ("", "_cs")}
    for log_l, g in ((8, 32), (9, 16), (10, 16)):
        assert use_row_halves_tile(log_l, g, True)
        assert not use_row_halves_tile(log_l, 8, True) and not use_row_halves_tile(log_l, g, False)
        # four / four / two workgroups per CU; the whole-tile layout of the
        # 16-element kernel takes twice the LDS
        lds = lds_elems(log_l, g) * 8
        whole = (1 << log_l) * (g + 1) * 8
        assert 2 * lds == whole and (160 * 1024) // lds == (2 if log_l == 10 else 4)
        assert g * (1 << log_l) // E <= 1024
    assert not use_row_halves_tile(8, 16, True)


def test_rowpair_cross_exchange_model():
    # fft2d_rowpair_fused_body (4096-point rows, 128 threads per row): the
    # exchange before the last stage writes each row's stage-1 outputs into
    # its own LDS region in two rounds (the row exchange's writes) and reads,
    # in round h, inputs p in [8h, 8h + 8) of last-stage butterfly
    # b = 128 s + t of both rows from both regions.  Every read slot holds, in
    # that round, position b + 256 p of its row; slots stay in bounds and no
    # slot is written twice in a round; each thread's 2 x 16 inputs are
    # exactly its butterfly's positions b + 256 p, p < 16.
    N, T, HALF = 4096, 128, 2048
    NB, L, S = 2, 16, 1

    def lds_pos(p):
        return p + (p >> 4)

    got = {}
    for h in range(2):
        written = {}
        for s in range(2):
            for t in range(T):
                for ii in range(NB // 2):
                    bb = t + T * (h * (NB // 2) + ii)
                    d0 = (bb >> (4 * S)) * L * 16 + (bb & (L - 1)) - HALF * h
                    for q in range(16):
                        slot = lds_pos(d0) + q * (L + L // 16)
                        assert slot == lds_pos(d0 + q * L) and 0 <= d0 + q * L < HALF
                        assert (s, slot) not in written
                        written[(s, slot)] = d0 + q * L + HALF * h
        assert len(written) == 2 * HALF
        for s in range(2):
            for t in range(T):
                b = T * s + t
                for pp in range(8):
                    slot = lds_pos(b) + pp * (256 + 16)
                    assert slot < HALF + HALF // 16
                    for row in range(2):
                        got.setdefault((s, t, row), []).append(written[(row, slot)])
    for (s, t, row), positions in got.items():
        b = T * s + t
        assert positions == [b + 256 * p for p in range(16)]
    assert len(got) == 2 * T * 2

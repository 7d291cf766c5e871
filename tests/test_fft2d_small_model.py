"""CPU model of the one-pass 2D FFT of small images (fft2d_small_body,
ferrum-gpu_amd/csrc/kernels/fft_2d_small.hpp), checked against the oracle
before any launch.

Per image the workgroup's LDS holds R rows of pitch P; the column exchanges
use regions of CP slots (both from the shape's Small2DLayout, read from the
header).  The model replays the kernel's index bookkeeping: the coalesced load
and store cover the workgroup's FPI images exactly once, both lane orders
give every (line, thread) pair once and keep a line's threads in one wave,
each row's Stockham exchanges stay in its own P slots and each column's in its
own CP slots of the image, all inside the image, and the data flow (rows, then
columns, each by the Stockham model of tests/test_stockham_model.py, which
checks the exchanges' own indices) gives the 2D DFT.  The host's launch
geometry (FG_SMALL2D_* in kernels/tile_geom.h) is mirrored here and checked
against the sources.
"""

from __future__ import annotations

import os
import re

import numpy as np
import pytest

import oracle
from conftest import rel_l2, uniform_c64
from test_stockham_model import model as stockham_model

MAX_LOG = 14
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def layouts():
    """small2d_layout's table: (lr, lc) -> (dp, dc, shr, shc, row_tm, col_tm)."""
    src = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "kernels", "fft_2d_small.hpp")).read()
    pat = r"case (\d+) \* 16 \+ (\d+): return \{(\d+), (\d+), (\d+), (\d+), (true|false), (true|false)\};"
    tab = {}
    for m in re.finditer(pat, src):
        g = m.groups()
        tab[(int(g[0]), int(g[1]))] = tuple(int(v) for v in g[2:6]) + (g[6] == "true", g[7] == "true")
    assert "default: return {1, 0, 4, 4, false, false};" in src
    return tab


LAYOUTS = layouts()


def layout(lr, lc):
    dp, dc, shr, shc, row_tm, col_tm = LAYOUTS.get((lr, lc), (1, 0, 4, 4, False, False))
    R, C = 1 << lr, 1 << lc
    return dict(P=C + (C >> shr) + dp, CP=R + (R >> shc) + dc, shr=shr, shc=shc, row_tm=row_tm, col_tm=col_tm)


def lanes(timg, threads_per_line, thread_major):
    """The kernel's (line, thread) of each local thread id."""
    local = np.arange(timg)
    k = min(64, timg)
    part, l = local // k, local % k
    per = k // threads_per_line
    if thread_major:
        return part * per + l % per, l // per
    return part * per + l // threads_per_line, l % threads_per_line


def loge(lr, lc):
    """FG_SMALL2D_LOGE: 8 elements per thread for the LDS-resident shapes (4:
    the radix-16 tables of the register-resident 8192- / 16384-point kernel)."""
    return 4 if lr + lc >= HALVES_LOG else 3


def fpi(lr, lc):
    """FG_SMALL2D_FPI: images per workgroup (256 threads, or one image)."""
    t = (1 << (lr + lc)) >> loge(lr, lc)
    return 1 if t >= 256 else 256 // t


HALVES_LOG = 11


def shapes():
    """The LDS-resident kernel's shapes: up to 1024 points (2048- to
    16384-point images run fft2d_halves_body, tests/test_fft2d_halves_model.py)."""
    return [(lr, lc) for lr in range(4, 11) for lc in range(4, 11) if lr + lc < HALVES_LOG]


def halves_shapes():
    return [(lr, bits - lr) for bits in range(HALVES_LOG, MAX_LOG + 1) for lr in range(4, bits - 3)]


def small2d_model(images, lr, lc):
    """images: (FPI, R, C) complex; returns the kernel's output, checking indices."""
    R, C = 1 << lr, 1 << lc
    LOGE = loge(lr, lc)
    N, E = R * C, 1 << LOGE
    F = images.shape[0]
    lay = layout(lr, lc)
    P, CP = lay["P"], lay["CP"]
    IMG = R * P
    block = F * (N // E)
    # 1. load: e = tid + BLOCK*j -> LDS is*IMG + r*P + c
    lds = np.full(F * IMG, np.nan + 0j)
    e = (np.arange(block)[:, None] + block * np.arange(E)[None, :]).reshape(-1)
    assert np.array_equal(np.sort(e), np.arange(F * N))
    img_of, n = e >> (lr + lc), e & (N - 1)
    idx = img_of * IMG + (n >> lc) * P + (n & (C - 1))
    assert idx.max() < lds.size and len(np.unique(idx)) == idx.size
    lds[idx] = images.reshape(-1)[e]
    out = np.empty((F, R, C), np.complex128)
    for s in range(F):
        img = lds[s * IMG:(s + 1) * IMG]
        # 2. rows: row r's exchanges in [r*P, r*P + C + C/2^shr)
        assert C + (C >> lay["shr"]) <= P and (R - 1) * P + C + (C >> lay["shr"]) <= IMG
        rows = np.stack([img[r * P:r * P + C] for r in range(R)])
        rows = stockham_model(rows.reshape(-1), lc, LOGE, lay["shr"]).reshape(R, C)
        for r in range(R):
            img[r * P:r * P + C] = rows[r]
        # 3. columns: column c read at k*P + c; its exchanges in [c*CP, c*CP + R + R/2^shc)
        cols = np.stack([img[np.arange(R) * P + c] for c in range(C)])
        assert R + (R >> lay["shc"]) <= CP and C * CP <= IMG
        cols = stockham_model(cols.reshape(-1), lr, LOGE, lay["shc"]).reshape(C, R)
        for c in range(C):
            img[np.arange(R) * P + c] = cols[c]
        out[s] = np.stack([img[r * P:r * P + C] for r in range(R)])
    return out


@pytest.mark.parametrize("lr,lc", shapes())
def test_small2d_model_matches_oracle(lr, lc):
    R, C = 1 << lr, 1 << lc
    F = min(fpi(lr, lc), 3)
    x = uniform_c64(np.random.default_rng(lr * 16 + lc), F * R * C).reshape(F, R, C)
    got = small2d_model(x, lr, lc)
    want = np.fft.fft2(x.astype(np.complex128))
    if lr == lc:
        assert rel_l2(got, oracle.fft_2d(x, lr)) < 1e-5
    assert rel_l2(got, want) < 1e-5


@pytest.mark.parametrize("lr,lc", shapes())
def test_small2d_geometry_fits(lr, lc):
    R, C = 1 << lr, 1 << lc
    N, E = R * C, 1 << loge(lr, lc)
    block = fpi(lr, lc) * N // E
    assert block <= 1024 and block % 64 == 0
    tc, tr = C // E, R // E
    assert tc <= 64 and tr <= 64 and 64 % tc == 0 and 64 % tr == 0   # rows / columns within a wave
    lay = layout(lr, lc)
    lds = fpi(lr, lc) * R * lay["P"] * 8
    assert lds <= 160 * 1024
    timg = N // E
    for tpl, tm, lines in ((tc, lay["row_tm"], R), (tr, lay["col_tm"], C)):
        line, t = lanes(timg, tpl, tm)
        assert np.array_equal(np.sort(line * tpl + t), np.arange(timg))   # every (line, thread) once
        assert line.max() == lines - 1
        wave = np.arange(timg) // 64
        for ln in range(lines):                                         # a line's threads in one wave
            assert len(set(wave[line == ln])) == 1


def test_small2d_mirror_matches_the_sources():
    geom = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "kernels", "tile_geom.h")).read()
    m = re.search(r"#define FG_SMALL2D_LOGE\(lr, lc\) \(\(\(lr\) \+ \(lc\)\) >= FG_SMALL2D_HALVES_LOG \? (\d+) : (\d+)\)", geom)
    assert m and m.groups() == ("4", "3")
    assert re.search(r"#define FG_SMALL2D_HALVES_LOG (\d+)", geom).group(1) == str(HALVES_LOG)
    assert re.search(r"#define FG_SMALL2D_MAX_LOG (\d+)", geom).group(1) == str(MAX_LOG)
    hip = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "kernels", "fft_kernels.hip")).read()
    inst = {(int(a), int(b)) for a, b in re.findall(r"^FG_FFT2D\((\d+), (\d+)\)", hip, flags=re.M)}
    assert inst == set(shapes())
    halves = {(int(a), int(b)) for a, b in re.findall(r"^FG_FFT2D_HALVES\((\d+), (\d+)\)", hip, flags=re.M)}
    assert halves == set(halves_shapes())
    # N/32 threads per image of 2048 points and more (FG_SMALL2D_TPI), one image per workgroup
    assert "(((lr) + (lc)) >= FG_SMALL2D_HALVES_LOG ? (1 << ((lr) + (lc))) / 32 :" in geom

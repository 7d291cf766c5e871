"""CPU model of the multi-pass decompositions used for N > 4096 (1D) and 2D,
checked against the oracle before any kernel exists for them.

1D, N = N_1 * ... * N_P (digit 1 slowest, S_i = N_{i+1} * ... * N_P):
  pass i < P: for every value of the faster digits r_i and the already
      transformed slower digits k_1..k_{i-1}: DFT over n_i (stride S_i),
      multiply by W_{S_{i-1}}^{r_i * k_i} (S_0 = N), store in place;
  pass P:  DFT over n_P (contiguous rows), store to the digit-reversed output
      position k_1 + N_1 k_2 + N_1 N_2 k_3 + ...
2D, N x N image: row FFTs, then the column FFT of length N split the same
  way (N = C_1 * C_2 with both passes over the slow axis).

`tile_geometry` builds the per-pass geometry (strides, tile counts, twiddle
coefficients) exactly as FftPlan does on the host; `run_geometry` executes it
with numpy so the index arithmetic is proven here.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
from conftest import rel_l2, uniform_c64

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def tile_columns(log_l):
    """Columns per tile of a pass that reads HBM (tile_columns in fft_plan.cpp):
    16..64 up to 1024 points, 8 (narrow tiles) for 2048 / 4096."""
    if log_l > 10:
        return 8
    return max(16, min(64, 8192 >> log_l))


def cached_tile_columns(log_l, rowwise):
    """Columns (row-wise: rows) per tile of a pass that reads cache-resident data
    (cached_tile_columns in fft_plan.cpp)."""
    if log_l < 7:
        return tile_columns(log_l)
    if rowwise:
        return {9: 8, 8: 32}.get(log_l, 16)
    return 16 if log_l == 8 else 8


def split_1d(log_n):
    """Digit sizes (log2) for N = 2^log_n, slowest first (split_1d in fft_plan.cpp)."""
    if log_n <= 20:
        b = min(10, log_n - 8) if log_n >= 16 else log_n // 2
        return [log_n - b, b]
    base = log_n // 3
    rest = log_n - 3 * base
    return [base + (1 if rest > 0 else 0), base + (1 if rest > 1 else 0), base]


def tile_geometry_1d(log_n, batch, cached=True, streams=1):
    """Per-pass geometry dicts (TileGeom), built as FftPlan::make_1d builds them;
    ``cached``: the plan is chunked, so passes after the first read the caches;
    ``chunks``: how many chunks the batch takes (two or more: the last pass
    takes at least 16 rows, for the plan's two chunks in flight)."""
    logs = split_1d(log_n)
    P = len(logs)
    N = 1 << log_n
    sizes = [1 << l for l in logs]
    S = [N]
    for s in sizes:
        S.append(S[-1] // s)          # S[i] = stride of digit i (1-based), S[P] = 1
    passes = []
    for i in range(1, P):
        L = sizes[i - 1]
        cols = S[i]                   # r_i ranges over [0, S_i): the faster digits
        g = cached_tile_columns(logs[i - 1], False) if (cached and i > 1) else tile_columns(logs[i - 1])
        assert cols >= g
        t0n = cols // g               # column groups
        t1n = N // (S[i - 1])         # values of the slower transformed digits k_1..k_{i-1}
        passes.append(dict(log_l=logs[i - 1], g=g, rowwise=False,
                           t0n=t0n, t1n=t1n,
                           is0=g, is1=S[i - 1], is2=N, ics=1, ies=S[i],
                           os0=g, os1=S[i - 1], os2=N, ocs=1, oes=S[i],
                           twc=1, tw0=g, tw1=0, log_m=int(np.log2(S[i - 1]))))
    # last pass: rows of length N_P, grouped by G' consecutive values of k_1
    L = sizes[-1]
    n1 = sizes[0]
    gp = cached_tile_columns(logs[-1], True) if cached else tile_columns(logs[-1])
    if cached and streams == 2:
        gp = max(gp, 16)
    assert n1 >= gp
    inner = N // (n1 * L)             # values of k_2..k_{P-1}
    # the row for (k_1, kmid) starts at k_1*S_1 + sum k_j S_j = k_1*S_1 + kmid*L
    passes.append(dict(log_l=logs[-1], g=gp, rowwise=True,
                       t0n=n1 // gp, t1n=inner,
                       is0=gp * S[1], is1=L, is2=N, ics=S[1], ies=1,
                       os0=gp, os1=n1, os2=N, ocs=1, oes=N // L,
                       twc=0, tw0=0, tw1=0, log_m=0))
    return passes


def rowpair_2d(log_rows, log_cols):
    """FftPlan::make_2d: images of 2048 / 4096 rows of 1024 .. 4096 points and
    of 1024 rows of 2048 / 4096 points split their column DFT radix-2 over the
    row index (kernels/fft_2d_rowpair.hpp) when run out of place; in place
    they keep the row pass + R-row columns."""
    return (log_rows >= 11 and log_cols >= 10) or (log_rows == 10 and log_cols >= 11)


def rowpair_model(x):
    """numpy model of the split: x (B, R, C) -> the 2D DFT.  Row DFTs; rows r
    and r + R/2 combined as A + B to row 2r and (A - B) W_R^r to row 2r + 1;
    then, in place, R/2-point DFTs down the rows of each parity h (a strided
    tile geometry: is1 = os1 = C, ies = oes = 2 C), X[2k + h] at row 2k + h."""
    b, R, C = x.shape
    half = R // 2
    rows = np.fft.fft(x.astype(np.complex128), axis=2)
    a, bb = rows[:, :half, :], rows[:, half:, :]
    w = np.exp(-2j * np.pi * np.arange(half) / R)[None, :, None]
    out = np.empty_like(rows)
    out[:, 0::2, :] = a + bb              # the row pass's output, rows as stored
    out[:, 1::2, :] = (a - bb) * w
    for h in range(2):
        out[:, h::2, :] = np.fft.fft(out[:, h::2, :], axis=1)
    return out


def two_in_flight_shape(two_d, log_rows, log_cols=None):
    """FftPlan::make_1d / make_2d: the multi-pass shapes that run two chunks at
    a time when the batch makes two or more (1D; every 2D plan runs one)."""
    return not two_d


def choose_chunk(unit, batch, limit, two_in_flight):
    """FftPlan::choose_chunk (fft_plan.cpp): (units per chunk, cached, two chunks
    in flight).  The limit bounds the bytes in flight: chunks of limit / 2 for
    shapes that run two at a time when a unit fits and the batch makes two or
    more, else chunks of the limit; 0 or a unit above the limit: one
    streaming chunk."""
    def units_for(lim):
        if lim == 0 or unit > lim:
            return batch, False
        return min(lim // unit, batch), True

    if two_in_flight and unit <= limit // 2:
        per, cached = units_for(limit // 2)
        if -(-batch // per) > 1:
            return per, cached, True
    per, cached = units_for(limit)
    return per, cached, False


def tile_geometry_2d(log_n, batch, log_cols=None, cached=True):
    """Column FFT of each R x C image after the row pass, as FftPlan::make_2d builds it
    (R = 2^log_n rows, C = 2^log_cols columns, square by default): one tile pass over
    min(width, C) adjacent columns of length R, in place; the width is the
    cache-resident one for chunked plans of 2048 and 4096 rows, else the HBM
    one."""
    R = 1 << log_n
    C = R if log_cols is None else 1 << log_cols
    narrow = cached and log_n > 10
    g = min(cached_tile_columns(log_n, False) if narrow else tile_columns(log_n), C)
    return [dict(log_l=log_n, g=g, rowwise=False, t0n=C // g, t1n=1,
                 is0=g, is1=0, is2=R * C, ics=1, ies=C,
                 os0=g, os1=0, os2=R * C, ocs=1, oes=C,
                 twc=0, tw0=0, tw1=0, log_m=0)]


def pass_policy(i, n, cached, g):
    """Cache-policy suffix of pass i of n (FftPlan::policy / add_tile): narrow
    tiles always _cc; unchunked plans stream; chunked: _sc, _cc..., _cs."""
    if g < 16:
        return "_cc"
    if not cached:
        return ""
    return "_sc" if i == 0 else ("_cs" if i == n - 1 else "_cc")


def use_halves_tile(log_l, g, rowwise):
    """use_halves_tile in fft_plan.cpp: column passes at the HBM width of 128 ..
    1024 points and the 8-column passes of 2048 / 4096 points run the
    32-element kernel with the exchanges in halves."""
    if rowwise:
        return False
    if log_l > 10:
        return True
    if log_l == 8 and g == 16:      # the cache-resident 1D middle pass
        return True
    return 7 <= log_l and g == tile_columns(log_l)


def use_row_halves_tile(log_l, g, rowwise):
    """use_row_halves_tile in fft_plan.cpp: the 1D last passes of 256 points
    in 32-row tiles and of 512 / 1024 points in 16-row tiles run the
    32-element kernel with the exchanges in halves (fg_tile_l*_g*_rh)."""
    return rowwise and ((g == 16 and log_l in (9, 10)) or (g == 32 and log_l == 8))


def plan_kernel_names(two_d, log_n, cached=True, log_cols=None, streams=1):
    """The kernel of every pass of a plan of 1D length 2^log_n (one pass up to
    16384 points, several beyond) or of 2D images with 2^log_n rows and
    2^log_cols columns, in launch order; ``streams``: 2 for plans with two
    chunks in flight (the two-stream widths)."""
    def tile(p, pol):
        kind = "h" if use_halves_tile(p["log_l"], p["g"], p["rowwise"]) else \
            "rh" if use_row_halves_tile(p["log_l"], p["g"], p["rowwise"]) else \
            ("r" if p["rowwise"] else "c")
        return f"fg_tile_l{p['log_l']}_g{p['g']}_{kind}{pol}"

    if not two_d:
        if log_n <= 15:
            # single pass: the Stockham kernel (fg_fft_n13 / n14 / n15: 32
            # elements per thread, exchanges in halves; test_tile_halves_model)
            return [f"fg_fft_n{log_n}"]
        passes = tile_geometry_1d(log_n, 1, cached, streams)
        return [tile(p, pass_policy(i, len(passes), cached, p["g"]))
                for i, p in enumerate(passes)]
    lc = log_n if log_cols is None else log_cols
    if log_n + lc <= 14:
        # images of up to 16384 points: one pass (fg_fft2d_*, test_fft2d_small_model)
        return [f"fg_fft2d_l{log_n}_{lc}"]
    if rowpair_2d(log_n, lc):
        # row pairs, then R/2-row halves tiles over each row parity: 8
        # columns at 4096 rows (narrow: always _cc), 16 at 1024 / 2048 rows
        if log_n == 12:
            return [f"fg_fft2d_rowpair_n{lc}", "fg_tile_l11_g8_h_cc"]
        return [f"fg_fft2d_rowpair_n{lc}", f"fg_tile_l{log_n - 1}_g16_h" + ("_cs" if cached else "")]
    passes = tile_geometry_2d(log_n, 1, lc, cached)
    n = len(passes) + 1
    return [f"fg_fft_n{lc}" + ("_sc" if cached else "")] + \
        [tile(p, pass_policy(i + 1, n, cached, p["g"])) for i, p in enumerate(passes)]


def xcd_remap(b, grid):
    """Tile handled by workgroup b under the XCD-range order (FG_TILE_ORDER_XCD_RANGES,
    tile_coords in kernels/fft_tile.hpp)."""
    return (b & 7) * (grid >> 3) + (b >> 3)


def line_group_order(b, g):
    """Tile handled by workgroup b under the line-group order
    (FG_TILE_ORDER_LINE_GROUPS): groups of s = 16 / g tiles dealt over the XCDs."""
    s = 16 // g if g < 16 else 1
    j = b >> 3
    return ((j // s) * 8 + (b & 7)) * s + j % s


def tile_order(log_l, g, rowwise, tiles):
    """TileGeom::remap of a pass (add_tile / exec in fft_plan.cpp): narrow tiles
    take the line-group order in halves, the XCD-range order otherwise, each
    only when the grid is a multiple of its unit; wide tiles the natural one."""
    if g >= 16:
        return 0
    if use_halves_tile(log_l, g, rowwise):
        return 2 if tiles % (8 * (16 // g)) == 0 else 0
    return 1 if tiles % 8 == 0 else 0


def tile_lds_index(log_l, g, pos, c):
    """TileLayout<LOGL, G>::at: position-padded for g < 16, column-padded otherwise."""
    if g < 16:
        return (pos + (pos >> 4)) * g + c
    return pos * (g + 1) + c


def tile_lds_elems(log_l, g):
    n = 1 << log_l
    return (n + n // 16) * g if g < 16 else n * (g + 1)


def run_geometry(buf_in, passes, batch, elems):
    """numpy execution of tile passes: out(c, k) = DFT_L over n of in(c, n), times the
    four-step twiddle, with the affine tile addressing of the kernel."""
    src = buf_in.astype(np.complex128).copy()
    for p in passes:
        L = 1 << p["log_l"]
        dst = np.zeros_like(src)
        n = np.arange(L)
        touched = np.zeros(src.size, dtype=np.int64)
        for t2 in range(batch):
            for t1 in range(p["t1n"]):
                for t0 in range(p["t0n"]):
                    ib = t0 * p["is0"] + t1 * p["is1"] + t2 * p["is2"]
                    ob = t0 * p["os0"] + t1 * p["os1"] + t2 * p["os2"]
                    c = np.arange(p["g"])
                    iaddr = ib + c[:, None] * p["ics"] + n[None, :] * p["ies"]
                    oaddr = ob + c[:, None] * p["ocs"] + n[None, :] * p["oes"]
                    assert iaddr.max() < src.size and oaddr.max() < src.size
                    y = np.fft.fft(src[iaddr], axis=1)
                    if p["log_m"]:
                        M = 1 << p["log_m"]
                        r = (p["twc"] * c + p["tw0"] * t0 + p["tw1"] * t1) % M
                        e = (r[:, None] * n[None, :]) % M
                        y = y * np.exp(-2j * np.pi * e / M)
                    dst[oaddr] = y
                    touched[oaddr] += 1
        # every output position is written exactly once
        assert np.all(touched == 1)
        src = dst
    return src


@pytest.mark.parametrize("cached", [True, False], ids=["chunked", "unchunked"])
@pytest.mark.parametrize("log_n", [15, 16, 17, 18, 20])
def test_1d_multipass_matches_oracle(log_n, cached):
    rng = np.random.default_rng(log_n)
    batch = 2
    x = uniform_c64(rng, batch << log_n)
    got = run_geometry(x, tile_geometry_1d(log_n, batch, cached), batch, 1 << log_n)
    assert rel_l2(got, oracle.fft_1d(x, log_n)) < 1e-5


@pytest.mark.parametrize("cached", [True, False], ids=["chunked", "unchunked"])
def test_1d_three_pass_small(cached):
    # exercise the 3-pass geometry at a size numpy loops finish quickly
    log_n = 21
    passes = tile_geometry_1d(log_n, 1, cached)
    assert len(passes) == 3
    rng = np.random.default_rng(0)
    x = uniform_c64(rng, 1 << log_n)
    got = run_geometry(x, passes, 1, 1 << log_n)
    assert rel_l2(got, np.fft.fft(x.astype(np.complex128))) < 1e-5


@pytest.mark.parametrize("cached", [True, False], ids=["chunked", "unchunked"])
@pytest.mark.parametrize("log_n", [4, 5, 6, 7, 8, 10, 11, 12])
def test_2d_column_passes_match_oracle(log_n, cached):
    rng = np.random.default_rng(log_n + 100)
    n = 1 << log_n
    batch = 2 if log_n <= 10 else 1
    x = uniform_c64(rng, batch * n * n).reshape(batch, n, n)
    rows = np.fft.fft(x.astype(np.complex128), axis=2).reshape(-1)
    got = run_geometry(rows, tile_geometry_2d(log_n, batch, cached=cached), batch, n * n).reshape(batch, n, n)
    assert rel_l2(got, oracle.fft_2d(x, log_n)) < 1e-5


@pytest.mark.parametrize("lr,lc", [(4, 9), (9, 4), (6, 12), (11, 4), (11, 6), (5, 7)])
def test_2d_rectangular_column_passes(lr, lc):
    rng = np.random.default_rng(lr * 13 + lc)
    R, C = 1 << lr, 1 << lc
    x = uniform_c64(rng, R * C).reshape(1, R, C)
    rows = np.fft.fft(x.astype(np.complex128), axis=2).reshape(-1)
    got = run_geometry(rows, tile_geometry_2d(lr, 1, lc), 1, R * C).reshape(1, R, C)
    assert rel_l2(got, np.fft.fft2(x.astype(np.complex128))) < 1e-5


@pytest.mark.parametrize("grid", [8, 16, 64, 1024, 4096, 8 * 1000])
def test_xcd_remap_is_a_permutation_grouping_neighbours(grid):
    tiles = [xcd_remap(b, grid) for b in range(grid)]
    assert sorted(tiles) == list(range(grid))
    per = grid // 8
    for b in range(grid):
        # every tile of XCD b % 8 lies in that XCD's contiguous range
        assert (b & 7) * per <= tiles[b] < ((b & 7) + 1) * per


@pytest.mark.parametrize("grid,g", [(16, 8), (32, 8), (512, 8), (1024, 8), (8 * 1000, 8), (32, 4), (4096, 4)])
def test_line_group_order_is_a_permutation_keeping_lines_on_one_xcd(grid, g):
    s = 16 // g
    assert grid % (8 * s) == 0
    tiles = [line_group_order(b, g) for b in range(grid)]
    assert sorted(tiles) == list(range(grid))
    for b in range(grid):
        # the tiles sharing a 128-byte line (one group of s) run on one XCD,
        # as consecutive workgroups of that XCD
        grp, r = divmod(tiles[b], s)
        assert grp % 8 == b % 8
        assert (b >> 3) % s == r
    # each dispatch round of 8 s workgroups covers 8 neighbouring line groups
    for base in range(0, grid, 8 * s):
        assert sorted(tiles[base:base + 8 * s]) == list(range(base, base + 8 * s))


def test_tile_orders_of_the_2d_column_passes():
    # 4096 / 2048 rows: 8 columns in halves, line groups when the grid allows
    for log_rows in (11, 12):
        for log_cols in range(4, 13):
            p = tile_geometry_2d(log_rows, 1, log_cols)[0]
            assert p["g"] == 8 and use_halves_tile(log_rows, 8, False)
            # a full 256 MiB chunk (the default limit, one chunk at a time):
            # 2^22 / R tiles whatever C, so always line groups
            unit = 8 << (log_rows + log_cols)
            units, _, two = choose_chunk(unit, 1 << 20, 256 << 20, two_in_flight_shape(True, log_rows, log_cols))
            tiles = p["t0n"] * units
            assert not two and tiles == (1 << 22) >> log_rows
            assert tile_order(log_rows, 8, False, tiles) == 2
    # a short last chunk whose grid is no multiple of 16 keeps the natural order
    assert tile_order(12, 8, False, 2 * 3) == 0
    # 512 rows: the 16-element narrow tile in XCD ranges
    assert tile_order(9, 8, False, 4096) == 1


@pytest.mark.parametrize("log_l,g", [(11, 8), (10, 16), (10, 8), (9, 8), (8, 32), (8, 16), (8, 8),
                                     (7, 8), (6, 64), (6, 16)])
def test_tile_lds_layout_is_injective_and_fits(log_l, g):
    n = 1 << log_l
    pos, c = np.meshgrid(np.arange(n), np.arange(g), indexing="ij")
    idx = tile_lds_index(log_l, g, pos, c)
    assert len(np.unique(idx)) == n * g
    assert idx.max() < tile_lds_elems(log_l, g)
    assert tile_lds_elems(log_l, g) * 8 <= 160 * 1024   # one CU's LDS


def test_long_column_widths():
    # 2048 / 4096-point columns: 8 per tile, 32 elements per thread (512 / 1024
    # threads), the halves of a 4096-point tile in 136 KB of LDS
    for log_n, threads in ((11, 512), (12, 1024)):
        assert tile_columns(log_n) == 8 == cached_tile_columns(log_n, False)
        assert 8 * (1 << log_n) // 32 == threads
    assert tile_lds_elems(11, 8) * 8 == 136 * 1024


def test_split_sizes_fit_the_tile_kernel():
    for log_n in range(15, 25):
        logs = split_1d(log_n)
        assert sum(logs) == log_n
        assert all(4 <= l <= 10 for l in logs), (log_n, logs)   # wide tiles only


@pytest.mark.parametrize("R,C", [(4096, 16), (64, 32), (16, 8)])
def test_rowpair_split_matches_fft2(R, C):
    # the radix-2 split of the column DFT reproduces the 2D DFT (any R; the
    # plan uses it at 4096 rows)
    rng = np.random.default_rng(R + C)
    x = uniform_c64(rng, 2 * R * C).reshape(2, R, C)
    assert rel_l2(rowpair_model(x), np.fft.fft2(x.astype(np.complex128))) < 1e-12


def test_rowpair_geometry_stays_in_bounds():
    # the column pass's tiles (8 / 16 columns, the rows of one parity) read and
    # write the image's elements, each exactly once and each in its own tile
    # (so the pass runs in place); the row pass's workgroups write rows 2r and
    # 2r + 1 of what they read from rows r and r + R/2, every row once
    for R, C in ((4096, 4096), (4096, 2048), (4096, 1024), (2048, 2048), (2048, 4096), (2048, 1024),
                 (1024, 2048), (1024, 4096)):
        g = 8 if R == 4096 else 16
        t0n, t1n, L = C // g, 2, R // 2
        t0 = np.arange(t0n)[:, None, None, None]
        t1 = np.arange(t1n)[None, :, None, None]
        c = np.arange(g)[None, None, :, None]
        k = np.arange(L)[None, None, None, :]
        idx = t0 * g + t1 * C + c + k * (2 * C)
        assert idx.min() == 0 and idx.max() == R * C - 1 and len(np.unique(idx)) == R * C
        r = np.arange(R // 2)
        assert sorted(np.concatenate([r, r + R // 2])) == list(range(R))
        assert sorted(np.concatenate([2 * r, 2 * r + 1])) == list(range(R))


def rowpair_index(b, pairs, log_rows):
    """rowpair_index in kernels/fft_2d_rowpair.hpp: 4096-row images in reverse
    order within a launch, rows in order; other heights in the natural order."""
    lh = log_rows - 1
    if log_rows != 12 or pairs & ((1 << lh) - 1):
        return b
    images = pairs >> lh
    return ((images - 1 - (b >> lh)) << lh) | (b & ((1 << lh) - 1))


@pytest.mark.parametrize("log_rows,images", [(12, 1), (12, 2), (12, 5), (11, 3)])
def test_rowpair_order_is_a_permutation(log_rows, images):
    # every workgroup of a launch takes a different pair of the launch's
    # images; 4096-row launches start with their last image and end with the
    # first (the image the column pass starts with), rows ascending in each
    half = 1 << (log_rows - 1)
    pairs = images * half
    b = np.arange(pairs)
    p = rowpair_index(b, pairs, log_rows)
    assert sorted(p.tolist()) == list(range(pairs))
    assert np.array_equal(p & (half - 1), b & (half - 1))
    if log_rows == 12:
        assert p[0] == (images - 1) * half and p[-1] == half - 1
    else:
        assert np.array_equal(p, b)
    src = open(os.path.join(ROOT, "ferrum-gpu_amd", "csrc", "kernels", "fft_2d_rowpair.hpp")).read()
    assert "if (log_rows != 12 || (pairs & ((1ull << lh) - 1)) != 0) return b;" in src
    # a count that is not whole images (no plan launches one) keeps the natural order
    assert np.array_equal(rowpair_index(b[:-1], pairs - 1, log_rows), b[:-1])
    assert "return ((images - 1 - (b >> lh)) << lh) | (b & ((1ull << lh) - 1));" in src
    assert src.count("const uint64_t p = rowpair_index(blockIdx.x, pairs, log_rows);") == 2


def test_chunk_choice_bounds_the_bytes_in_flight():
    MIB = 1 << 20
    # config 4: four 128 MiB transforms, two chunks of one in flight
    assert choose_chunk(128 * MIB, 4, 256 * MIB, True) == (1, True, True)
    # config 5: two 128 MiB images on one stream, one chunk of both
    assert choose_chunk(128 * MIB, 2, 256 * MIB, False) == (2, True, False)
    # a batch that fits half the limit: one chunk, one stream
    assert choose_chunk(MIB, 100, 256 * MIB, True) == (100, True, False)
    # 512 MiB of 2D 256 x 256 images: 128 MiB chunks, two in flight
    assert choose_chunk(512 * 1024, 1024, 256 * MIB, True) == (256, True, True)
    # a unit above half the limit: one chunk at a time of the whole limit
    assert choose_chunk(3 * MIB, 5, 4 * MIB, True) == (1, True, False)
    # chunking off, or a unit above the limit: one streaming chunk
    assert choose_chunk(MIB, 7, 0, True) == (7, False, False)
    assert choose_chunk(8 * MIB, 7, 4 * MIB, False) == (7, False, False)
    for unit in (1, 3, 64, 1000):
        for batch in (1, 2, 5, 64):
            for limit in (0, unit, 2 * unit, 3 * unit, 7 * unit, 1000 * unit):
                for shape in (False, True):
                    per, cached, two = choose_chunk(unit, batch, limit, shape)
                    assert 1 <= per <= batch
                    assert cached == (limit > 0 and unit <= limit)
                    if two:  # two chunks in flight stay within the limit
                        assert shape and 2 * per * unit <= limit and per < batch
                    elif cached:
                        assert per * unit <= limit

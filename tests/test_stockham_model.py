"""CPU model of the LDS-resident Stockham kernel's data movement
(ferrum-gpu_amd/csrc/kernels/fft_stockham.hpp), checked against the oracle.

The model keeps the kernel's register bookkeeping exactly -- thread t holds
positions t + T*m, butterfly i of stage s reads x[i + NB*p], scatters output q
to j*L*R + k + q*L, the next stage gathers t + T*m -- and its twiddle table is
built the way fft_plan.cpp builds it.  Only the in-register DFT-R is replaced
by numpy's, so this pins the indexing (the part a GPU fault would come from)
on the CPU before any launch.  It also checks every LDS index stays inside the
padded allocation the kernel declares.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rel_l2, uniform_c64

# kStockham in fft_plan.cpp / FG_STOCKHAM in fft_kernels.hip: (log_e, fpb)
GEOM = {2: (2, 64), 3: (3, 64), 4: (3, 32), 5: (3, 16), 6: (2, 4), 7: (3, 4), 8: (4, 4),
        9: (4, 2), 10: (4, 2), 11: (4, 1), 12: (4, 1)}
# kStockham[10] = {4, 2} launches the 1024-point kernel with two transforms per
# 128-thread workgroup and the radix list 8 * 16 * 8 (FG_STOCKHAM_X2_1024;
# modelled in test_x2_model.py); GEOM keeps it for the launch shape.
X2_GEOM = {10: (4, 2)}
# kStockham entries of the 32-element kernels with the exchanges in halves
# (FG_STOCKHAM_HALVES, one transform per workgroup; modelled in
# test_tile_halves_model.py)
HALVES_GEOM = {13: (5, 1), 14: (5, 1), 15: (5, 1)}
# kStockhamLatency / FG_STOCKHAM_LAT: single-pass plans too small to fill the GPU
LATENCY_GEOM = {8: (2, 1), 10: (3, 1), 12: (3, 1)}


def row_exponents(r):
    """Exponents p of W^{p*k} stored per table row for a radix-r stage."""
    return [1, 2, 3, 4, 8, 12] if r == 16 else [1, 2, 3, 4] if r == 8 else list(range(r))


def two_level(L):
    """A stage spanning L >= 1024 stores W^{64 h} (h < L/64; radix 8: h < 8L/64),
    then W^l (l < 64)."""
    return L >= 1024


def two_level_high(L, R):
    """Entries W^{64 h} of a two-level block (tw_two_level_high)."""
    return L * R // 64 if R == 8 else L // 64


def stockham_table(log_n, log_e):
    nfull, rem = divmod(log_n, log_e)
    nst = nfull + (1 if rem else 0)
    out, offs = [], [0, 0]
    for s in range(1, nst):
        logl, logr = s * log_e, (log_e if s < nfull else rem)
        L, R = 1 << logl, 1 << logr
        if two_level(L):
            hi = two_level_high(L, R)
            e = np.concatenate([(64 * np.arange(hi)) % (L * R), np.arange(64)])
            out.append(np.exp(-2j * np.pi * e / (L * R)).astype(np.complex64))
            offs.append(offs[-1] + hi + 64)
            continue
        ps = np.array(row_exponents(R))
        k, p = np.meshgrid(np.arange(L), ps, indexing="ij")
        e = (p * k) % (L * R)
        out.append(np.exp(-2j * np.pi * e / (L * R)).astype(np.complex64).reshape(-1))
        offs.append(offs[-1] + L * len(ps))
    return (np.concatenate(out) if out else np.ones(1, np.complex64)), offs


def stage_twiddles(tw, off, k, r, L=None):
    """(T, r) twiddles W^{p*k} as the kernel forms them from the table rows at
    off + k * row_len: a stored entry, or for radix 16 / 8 the product
    W^{k*(p & 3)} * W^{k*4*(p >> 2)} of two stored entries.  A two-level stage
    (L >= 1024) forms W^k = A[k >> 6] * B[k & 63]; radix 4 forms W^2k and
    W^3k as products of it, radix 8 looks up W^2k and W^4k the same way and
    forms W^3k = W^k W^2k, W^5k = W^k W^4k, W^6k = W^2k W^4k,
    W^7k = W^3k W^4k -- all in f32, as apply_stage_twiddles_at does."""
    if L is not None and two_level(L):
        assert r in (2, 4, 8)
        hi = two_level_high(L, r)

        def look(e):
            return (tw[off + (e >> 6)] * tw[off + hi + (e & 63)]).astype(np.complex64)

        def mul(a, b):
            return (a * b).astype(np.complex64)

        w1 = look(k)
        cols = [np.ones(k.shape, np.complex64), w1]
        if r == 4:
            w2 = mul(w1, w1)
            cols += [w2, mul(w2, w1)]
        if r == 8:
            w2, w4 = look(2 * k), look(4 * k)
            w3 = mul(w1, w2)
            cols += [w2, w3, w4, mul(w1, w4), mul(w2, w4), mul(w3, w4)]
        return np.stack(cols, axis=1).astype(np.complex128)
    ps = row_exponents(r)
    rows = tw[off + k[:, None] * len(ps) + np.arange(len(ps))[None, :]].astype(np.complex128)
    if r not in (8, 16):
        return rows
    ent = {p: rows[:, i] for i, p in enumerate(ps)}
    ent[0] = np.ones(k.shape, np.complex128)
    cols = []
    for p in range(r):
        lo, hi = p & 3, 4 * (p >> 2)
        cols.append(ent[p] if (lo == 0 or hi == 0) else ent[lo] * ent[hi])
    return np.stack(cols, axis=1)


def lds_pos(p, sh=4):
    return p + (p >> sh)


def model(x, log_n, log_e, sh=4):
    """sh: the exchanges' padding, one slot per 2**sh positions (lds_pos<SH>)."""
    n, e = 1 << log_n, 1 << log_e
    t_per = n // e
    nfull, rem = divmod(log_n, log_e)
    logrs = [log_e] * nfull + ([rem] if rem else [])
    tw, offs = stockham_table(log_n, log_e)
    lanes = x.reshape(-1, n)
    t = np.arange(t_per)
    regs = lanes[:, t[:, None] + t_per * np.arange(e)[None, :]]   # regs[b, t, m] = x[t + T m]
    lds_elems = n + (n >> sh)
    for s, logr in enumerate(logrs):
        r = 1 << logr
        nb = e // r
        L = 1 << (s * log_e)
        new = np.empty_like(regs)
        dst_pos = np.empty((t_per, e), dtype=np.int64)
        for i in range(nb):
            u = regs[:, :, [i + nb * p for p in range(r)]].astype(np.complex128)   # (B, T, R)
            b = t + t_per * i
            k = b & (L - 1)
            if L > 1:
                w = stage_twiddles(tw, offs[s], k, r, L)
                used = (L // 64 + 64) if two_level(L) else (k.max() + 1) * len(row_exponents(r))
                assert offs[s] + used <= offs[s + 1] <= tw.size
                u = u * w[None, :, :]
            y = np.fft.fft(u, axis=2)
            j = b >> (s * log_e)
            for q in range(r):
                new[:, :, i + nb * q] = y[:, :, q]
                dst_pos[:, i + nb * q] = j * L * r + k + q * L
        # every thread writes a distinct position and all N positions are covered
        assert np.array_equal(np.sort(dst_pos.reshape(-1)), np.arange(n))
        if s + 1 < len(logrs):
            lds = np.zeros((lanes.shape[0], lds_elems), np.complex128)
            assert lds_pos(dst_pos, sh).max() < lds_elems
            lds[:, lds_pos(dst_pos, sh)] = new
            gather = lds_pos(t[:, None] + t_per * np.arange(e)[None, :], sh)
            assert gather.max() < lds_elems
            regs = lds[:, gather]
        else:
            # the last stage's scatter is exactly the coalesced t + T*m store
            assert np.array_equal(dst_pos, t[:, None] + t_per * np.arange(e)[None, :])
            regs = new
    out = np.empty((lanes.shape[0], n), np.complex128)
    out[:, t[:, None] + t_per * np.arange(e)[None, :]] = regs
    return out.reshape(-1)


@pytest.mark.parametrize("log_n", list(range(2, 13)))
def test_model_matches_oracle(log_n):
    rng = np.random.default_rng(log_n)
    x = uniform_c64(rng, 3 << log_n)
    log_e, _ = GEOM[log_n]
    assert rel_l2(model(x, log_n, log_e), oracle.fft_1d(x, log_n)) < 1e-5


@pytest.mark.parametrize("log_n", sorted(LATENCY_GEOM))
def test_model_matches_oracle_latency_geometry(log_n):
    rng = np.random.default_rng(log_n + 50)
    x = uniform_c64(rng, 3 << log_n)
    log_e, _ = LATENCY_GEOM[log_n]
    assert rel_l2(model(x, log_n, log_e), oracle.fft_1d(x, log_n)) < 1e-5


@pytest.mark.parametrize("log_n,log_e", [(10, 3), (12, 3), (11, 2), (9, 5), (12, 6)])
def test_model_other_radices(log_n, log_e):
    rng = np.random.default_rng(log_n * 7 + log_e)
    x = uniform_c64(rng, 2 << log_n)
    assert rel_l2(model(x, log_n, log_e), oracle.fft_1d(x, log_n)) < 1e-5


def test_twiddle_rows_are_16_byte_aligned():
    # The kernel loads table rows as float4 pairs: every block offset and row
    # length must be even (8-byte entries -> 16-byte aligned rows).
    for log_n, (log_e, _) in list(GEOM.items()) + list(LATENCY_GEOM.items()):
        _, offs = stockham_table(log_n, log_e)
        assert all(o % 2 == 0 for o in offs), log_n
    assert all(len(row_exponents(r)) % 2 == 0 for r in (2, 4, 8, 16))


def test_factored_twiddles_equal_the_full_rows():
    # the products the kernel forms reproduce W^{p*k} for every p (to f32 rounding)
    for log_n, log_e in [(12, 4), (11, 4), (10, 4), (9, 3), (12, 3), (13, 4), (14, 4), (15, 4)]:
        tw, offs = stockham_table(log_n, log_e)
        nfull, rem = divmod(log_n, log_e)
        for s in range(1, nfull + (1 if rem else 0)):
            L, R = 1 << (s * log_e), 1 << (log_e if s < nfull else rem)
            k = np.arange(L)
            w = stage_twiddles(tw, offs[s], k, R, L)
            exact = np.exp(-2j * np.pi * ((k[:, None] * np.arange(R)[None, :]) % (L * R)) / (L * R))
            # stored or one product: 3e-7; two-level (W^k from two entries, then
            # W^2k and W^3k as products): up to five f32 roundings, 6e-7 (radix
            # 8 at 32768 points, W^7k from three lookups: 2.4e-7)
            tol = 6e-7 if two_level(L) else 3e-7
            assert np.max(np.abs(w - exact)) < tol, (log_n, s)


def test_stage_table_sizes():
    # N = 4096, radix 16: stage 1 holds 16 rows, stage 2 256 rows of 6 entries
    _, offs = stockham_table(12, 4)
    assert offs == [0, 0, 16 * 6, 16 * 6 + 256 * 6]
    # N = 1024 (16, 16, 4): 16 rows of 6, then 256 full rows of 4
    _, offs = stockham_table(10, 4)
    assert offs == [0, 0, 96, 96 + 1024]
    # N = 16384 (16, 16, 16, 4): the last stage (L = 4096) is two-level, 64 + 64
    # entries instead of 4096 rows of 4
    tw, offs = stockham_table(14, 4)
    assert offs == [0, 0, 96, 96 + 1536, 96 + 1536 + 128] and tw.size == offs[-1]
    # N = 32768 (16, 16, 16, 8): the radix-8 two-level stage holds W^{64 h} for
    # every exponent below L*R = 32768 (512 entries), then 64
    tw, offs = stockham_table(15, 4)
    assert offs == [0, 0, 96, 96 + 1536, 96 + 1536 + 512 + 64] and tw.size == offs[-1]
    # no stage of the kernels up to 4096 points is two-level (their tables are
    # unchanged): the single-pass geometries, the tile passes (log_e 4, up to
    # 4096 points) and the one-pass 2D kernels (log_e 3 or 4, up to 1024 points)
    geoms = set(GEOM.items()) | set(LATENCY_GEOM.items())
    geoms = {(n, g[0]) for n, g in geoms} | {(n, 4) for n in range(4, 13)} | \
        {(n, e) for n in range(4, 11) for e in (3, 4)}
    for log_n, log_e in geoms:
        nstages = log_n // log_e + (1 if log_n % log_e else 0)
        assert all(not two_level(1 << (s * log_e)) for s in range(1, nstages)), (log_n, log_e)


def test_staged_block_mapping_covers_each_element_once():
    # Sizes with T < 8 threads per transform stage their FPB transforms
    # through LDS: element e = tid + BLOCK*j of the block -> transform e >> log_n,
    # position e & (N-1).  Every element once, every LDS index in its slot.
    for log_n, (log_e, fpb) in GEOM.items():
        n, t_per = 1 << log_n, (1 << log_n) >> log_e
        if not (t_per < 8 and fpb > 1):
            continue
        block, e_per = fpb * t_per, 1 << log_e
        e = (np.arange(block)[:, None] + block * np.arange(e_per)[None, :]).reshape(-1)
        assert np.array_equal(np.sort(e), np.arange(fpb * n))
        assert (e >> log_n).max() < fpb
        assert lds_pos(e & (n - 1)).max() < n + n // 16


def test_geometry_fits_hardware():
    for log_n, (log_e, fpb) in list(GEOM.items()) + list(LATENCY_GEOM.items()):
        threads = ((1 << log_n) >> log_e) * fpb
        assert 1 <= threads <= 1024
        lds = fpb * ((1 << log_n) + (1 << log_n) // 16) * 8
        assert lds <= 64 * 1024, (log_n, lds)


def test_geometry_tables_match_the_sources():
    # the mirrors above equal the host tables and the kernel instantiations
    import os
    import re

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    plan = open(os.path.join(root, "ferrum-gpu_amd", "csrc", "fft_plan.cpp")).read()
    hip = open(os.path.join(root, "ferrum-gpu_amd", "csrc", "kernels", "fft_kernels.hip")).read()

    def table(name):
        body = re.search(name + r"\[kMaxLogNSingle \+ 1\] = \{(.*?)\};", plan, flags=re.S).group(1)
        body = re.sub(r"//[^\n]*", "", body)
        return [tuple(int(v) for v in m) for m in re.findall(r"\{(\d+), (\d+)\}", body)]

    assert {n: g for n, g in enumerate(table("kStockham")) if g != (0, 0)} == {**GEOM, **HALVES_GEOM}
    halves = {int(a): (5, 1) for a in re.findall(r"^FG_STOCKHAM_HALVES\((\d+)\)", hip, flags=re.M)}
    assert halves == HALVES_GEOM
    assert {n: g for n, g in enumerate(table("kStockhamLatency")) if g != (0, 0)} == LATENCY_GEOM
    inst = {int(a): (int(b), int(c)) for a, b, c in re.findall(r"^FG_STOCKHAM\((\d+), (\d+), (\d+)\)", hip, flags=re.M)}
    if re.search(r"^FG_STOCKHAM_X2_1024\(\)", hip, flags=re.M):
        inst.update(X2_GEOM)
    assert inst == GEOM
    lat = {int(a): (int(b), 1) for a, b in re.findall(r"^FG_STOCKHAM_LAT\((\d+), (\d+)\)", hip, flags=re.M)}
    assert lat == LATENCY_GEOM

"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each check compares the oracle with something it did not produce: the
reference's own known-answer tests (cited), textbook closed forms, an fp64
direct DFT, numpy.fft complex128 golden fixtures, and cross-algorithm
agreement.  The last section plants plausible mistakes in oracle outputs and
shows the same checks reject them.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
from conftest import rel_l2, uniform_c64

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ------------------------------------------------------------------ twiddles


def test_twiddles_total_count_is_n_minus_one():
    # crates/ferrum-gpu-fft/tests/twiddles.rs:23-37
    for log_n in (2, 3, 6, 8, 10, 12):
        assert oracle.twiddles(log_n).size == (1 << log_n) - 1


def test_twiddles_first_and_last_are_one():
    # twiddles.rs:5-21: first entry of stage log_n and the single W_2^0 entry.
    for log_n in (2, 3, 10):
        tw = oracle.twiddles(log_n)
        assert abs(tw[0] - 1) < 1e-6 and abs(tw[-1] - 1) < 1e-6


def test_twiddles_match_fp64_roots():
    # Stage s (descending) holds W_{2^s}^k, k < 2^(s-1).
    for log_n in (4, 9, 12):
        tw = oracle.twiddles(log_n).astype(np.complex128)
        exp = np.concatenate([np.exp(-2j * np.pi * np.arange(1 << (s - 1)) / (1 << s))
                              for s in range(log_n, 0, -1)])
        assert np.max(np.abs(tw - exp)) < 4e-7


def test_radix_tables_match_fp64_roots():
    for log_r, fn in ((2, oracle.twiddles_radix4), (3, oracle.twiddles_radix8)):
        r = 1 << log_r
        for log_n in (log_r, 2 * log_r, 4 * log_r if log_r == 2 else 3 * log_r):
            tw = fn(log_n).astype(np.complex128)
            exp, m_r = [], 1
            for _ in range(log_n // log_r):
                m = m_r * r
                k, p = np.meshgrid(np.arange(m_r), np.arange(r), indexing="ij")
                exp.append(np.exp(-2j * np.pi * ((p * k) % m) / m).reshape(-1))
                m_r = m
            exp = np.concatenate(exp)
            assert tw.size == exp.size
            assert np.max(np.abs(tw - exp)) < 4e-7
    assert oracle.twiddles_radix4(10).size == 4 * (1024 - 1) // 3  # 1364: 4·m entries per stage, m = 1, 4, ..., 256
    assert oracle.twiddles_radix8(12).size == 4680


def test_full_roots():
    tw = oracle.twiddles_full_roots(8).astype(np.complex128)
    assert np.max(np.abs(tw - np.exp(-2j * np.pi * np.arange(256) / 256))) < 4e-7


def test_stage_offsets_log_n_3():
    # crates/ferrum-gpu-fft/src/cpu.rs:131-139
    offs = oracle.stage_offsets(3)
    assert (offs[3], offs[2], offs[1]) == (0, 4, 6)


# ------------------------------------------------------ 1D radix-2 Stockham


def test_forward_n4_matches_hand_dft():
    # cpu.rs:141-170: DFT([1,2,3,4]) = [10, -2+2i, -2, -2-2i]
    y = oracle.fft_1d(np.array([1, 2, 3, 4], dtype=np.complex64), 2)
    assert np.max(np.abs(y - np.array([10, -2 + 2j, -2, -2 - 2j]))) < 1e-5


def test_dft_naive_matches_known_4pt():
    # crates/ferrum-gpu-fft/src/layout_study.rs:58-66
    y = oracle.dft_naive(np.array([1, 2, 3, 4], dtype=np.complex64))
    assert np.max(np.abs(y - np.array([10, -2 + 2j, -2, -2 - 2j]))) < 1e-4


@pytest.mark.parametrize("log_n", [2, 5, 9, 12])
def test_impulse_and_constant_closed_forms(log_n):
    n = 1 << log_n
    d = np.zeros(n, np.complex64)
    d[0] = 1
    assert np.max(np.abs(oracle.fft_1d(d, log_n) - 1)) < 1e-6          # delta -> ones
    c = np.ones(n, np.complex64)
    exp = np.zeros(n)
    exp[0] = n
    assert np.max(np.abs(oracle.fft_1d(c, log_n) - exp)) < 1e-6 * n     # ones -> N delta
    s = np.zeros(n, np.complex64)
    s[1] = 1                                                             # shifted delta -> W^k
    assert np.max(np.abs(oracle.fft_1d(s, log_n) - np.exp(-2j * np.pi * np.arange(n) / n))) < 1e-5


def test_golden_numpy_1d():
    g = _golden("fft1d_numpy.npz")
    keys = sorted(k[3:] for k in g if k.startswith("in_"))
    assert len(keys) == 29  # 11 sin/cos lanes + 9 slow + 9 uniform
    for k in keys:
        log_n = int(k.rsplit("_n", 1)[1])
        x = g["in_" + k]
        assert rel_l2(oracle.fft_1d(x, log_n), g["fwd_" + k]) < 1e-6, k
        assert rel_l2(oracle.fft_1d(x, log_n, "inverse"), g["inv_" + k]) < 1e-6, k
        n = 1 << log_n
        assert rel_l2(oracle.fft_1d(x, log_n, "inverse", True), g["inv_" + k] / n) < 1e-6, k


def test_rustfft_cross_check_inputs():
    # crates/ferrum-gpu-fft/tests/rustfft_cross_check.rs:21-47, metric and bound
    # kept: (|dre|+|dim|)/(|re|+|im|+1) < 1e-4 against a library FFT.
    for log_n in (2, 3, 6):
        n = 1 << log_n
        i = np.arange(n, dtype=np.float32)
        x = (np.sin(i) + 1j * np.cos(i)).astype(np.complex64)
        exp = np.fft.fft(x.astype(np.complex128))
        got = oracle.fft_1d(x, log_n)
        rel = (np.abs(got.real - exp.real) + np.abs(got.imag - exp.imag)) / (np.abs(exp.real) + np.abs(exp.imag) + 1)
        assert rel.max() < 1e-4


def test_fp64_dft_bins_match_numpy():
    rng = np.random.default_rng(7)
    x = uniform_c64(rng, 512)
    bins = [0, 1, 17, 255, 256, 511]
    got = oracle.dft_bins_f64(x, bins)
    exp = np.fft.fft(x.astype(np.complex128))[bins]
    assert np.max(np.abs(got - exp)) < 1e-9 * 512
    got_inv = oracle.dft_bins_f64(x, bins, sign=+1)
    assert np.max(np.abs(got_inv - np.fft.ifft(x.astype(np.complex128))[bins] * 512)) < 1e-9 * 512


def test_batched_lanes_are_independent_and_threaded_split_is_identical():
    rng = np.random.default_rng(3)
    x = uniform_c64(rng, 256 * 37)
    one = oracle.fft_1d(x, 8)
    many = oracle.fft_1d(x, 8, threads=4)
    assert np.array_equal(one, many)
    lanes = x.reshape(37, 256)
    for j in (0, 20, 36):
        assert np.array_equal(one.reshape(37, 256)[j], oracle.fft_1d(lanes[j], 8))


@pytest.mark.parametrize("log_n,tol", [(2, 1e-4), (3, 1e-4), (8, 1e-3)])
def test_roundtrip(log_n, tol):
    # crates/ferrum-gpu-fft/tests/cpu_roundtrip.rs:5-69
    n = 1 << log_n
    if log_n == 2:
        x = np.array([complex(i + 1, 2 * i - 1) for i in range(n)], np.complex64)
    else:
        x = np.array([complex(i, n - i) for i in range(n)], np.complex64)
    y = oracle.fft_1d(oracle.fft_1d(x, log_n), log_n, "inverse", True)
    assert np.max(np.abs(y - x)) < tol


def test_parseval_and_linearity_large():
    rng = np.random.default_rng(11)
    n = 1 << 16
    a, b = uniform_c64(rng, n), uniform_c64(rng, n)
    fa, fb = oracle.fft_1d(a, 16), oracle.fft_1d(b, 16)
    assert abs(np.vdot(fa, fa).real / n - np.vdot(a, a).real) / np.vdot(a, a).real < 1e-5
    fab = oracle.fft_1d((a + 2 * b).astype(np.complex64), 16)
    assert rel_l2(fab, fa + 2 * fb) < 1e-5


# -------------------------------------------------------------------- 2D


def test_golden_numpy_2d():
    g = _golden("fft2d_numpy.npz")
    for k in sorted(k[3:] for k in g if k.startswith("in_")):
        log_n = int(k.rsplit("_n", 1)[1])
        x = g["in_" + k]
        assert rel_l2(oracle.fft_2d(x, log_n), g["fwd_" + k]) < 1e-6, k
        assert rel_l2(oracle.fft_2d(x, log_n, "inverse"), g["inv_" + k]) < 1e-6, k


def test_2d_rustfft_cross_check_metric():
    # crates/ferrum-gpu-fft/tests/cpu_2d_vs_rustfft.rs:90-116 (N = 8, 64)
    for log_n in (3, 6):
        n = 1 << log_n
        i = np.arange(n * n, dtype=np.float32)
        x = (np.sin(i * np.float32(0.1)) + 1j * np.cos(i * np.float32(0.07))).astype(np.complex64).reshape(n, n)
        exp = np.fft.fft2(x.astype(np.complex128))
        got = oracle.fft_2d(x, log_n)
        rel = (np.abs(got.real - exp.real) + np.abs(got.imag - exp.imag)) / (np.abs(exp.real) + np.abs(exp.imag) + 1)
        assert rel.max() < 1e-4


@pytest.mark.parametrize("log_n,tol", [(2, 1e-4), (6, 1e-3)])
def test_2d_roundtrip(log_n, tol):
    # crates/ferrum-gpu-fft/tests/cpu_2d_roundtrip.rs:5-49
    n = 1 << log_n
    if log_n == 2:
        x = np.array([complex(i + 1, 2 * i - 0.5) for i in range(n * n)], np.complex64).reshape(n, n)
    else:
        x = np.array([complex(np.sin(i % n), np.cos(i // n)) for i in range(n * n)], np.complex64).reshape(n, n)
    y = oracle.fft_2d(oracle.fft_2d(x, log_n), log_n, "inverse", True)
    assert np.max(np.abs(y - x)) < tol


def test_2d_is_separable_fp64():
    rng = np.random.default_rng(5)
    x = uniform_c64(rng, 128 * 128).reshape(128, 128)
    got = oracle.fft_2d(x, 7)
    # separable fp64 DFT at sampled (k1, k2)
    n = 128
    idx = np.arange(n)
    for k1, k2 in [(0, 0), (3, 77), (127, 1), (64, 64)]:
        v = np.sum(x.astype(np.complex128) * np.exp(-2j * np.pi * k1 * idx[:, None] / n)
                   * np.exp(-2j * np.pi * k2 * idx[None, :] / n))
        assert abs(got[k1, k2] - v) < 1e-4 * np.sqrt(n * n)


def test_2d_batch_matches_single_images():
    rng = np.random.default_rng(9)
    x = uniform_c64(rng, 3 * 32 * 32).reshape(3, 32, 32)
    got = oracle.fft_2d(x, 5)
    for b in range(3):
        assert np.array_equal(got[b], oracle.fft_2d(x[b], 5))


# --------------------------------------------------- radix-4/8, four-step


def _direct(x):
    n = x.size
    k = np.arange(n)
    return np.exp(-2j * np.pi * np.outer(k, k) / n) @ x.astype(np.complex128)


def test_dft4_dft8_match_direct():
    # cpu_radix4.rs:105-123 (sin 0.41 i), cpu_radix8.rs:153-174 (sin 0.37 i)
    for fn, r, a in ((oracle.dft4, 4, 0.41), (oracle.dft8, 8, 0.37)):
        inp = np.sin(np.arange(2 * r, dtype=np.float32) * np.float32(a)).astype(np.float32)
        got = fn(inp)
        c = inp[0::2].astype(np.float64) + 1j * inp[1::2]
        exp = _direct(c)
        assert np.max(np.abs(got[0::2] - exp.real)) < 1e-4 and np.max(np.abs(got[1::2] - exp.imag)) < 1e-4


def _slow_input(n, batch=3):
    t = (np.arange(n * batch) % n).astype(np.float32)
    return (np.sin(t * np.float32(0.013)) + 1j * np.cos(t * np.float32(0.021))).astype(np.complex64)


def _per_bin_rel(got, ref):
    err = np.abs(got.astype(np.complex128) - ref)
    return np.max(err / np.maximum(np.abs(ref), 1.0))


@pytest.mark.parametrize("log_r,log_ns", [(2, (2, 4, 6, 8, 10)), (3, (3, 6, 9, 12))])
def test_radix4_radix8_match_radix2(log_r, log_ns):
    # cpu_radix4.rs:125-159, cpu_radix8.rs:176-216: batch 3, per-bin rel < 1e-3
    for log_n in log_ns:
        n = 1 << log_n
        x = _slow_input(n)
        ref = oracle.fft_1d(x, log_n)
        tw = oracle.twiddles_radix4(log_n) if log_r == 2 else oracle.twiddles_radix8(log_n)
        lane_fn = oracle.radix4_forward_lane if log_r == 2 else oracle.radix8_forward_lane
        got = np.concatenate([lane_fn(x[j * n:(j + 1) * n], log_n, tw) for j in range(3)])
        assert _per_bin_rel(got, ref) < 1e-3, log_n


def test_warp_dif_matches_direct_32_and_64():
    # warp_fft.rs:211-233
    for log_n in (5, 6):
        n = 1 << log_n
        i = np.arange(n, dtype=np.float32)
        x = (np.sin(i * np.float32(0.29)) + 1j * np.cos(i * np.float32(0.13))).astype(np.complex64)
        got = oracle.warp_dif(x, log_n)
        assert _per_bin_rel(got, _direct(x)) < 1e-4


@pytest.mark.parametrize("l1,l2", [(6, 6), (5, 3), (3, 7)])
def test_four_step_matches_radix2(l1, l2):
    # warp_fft.rs:235-287 (64 x 64 and 32 x 8)
    n = 1 << (l1 + l2)
    i = np.arange(n, dtype=np.float32)
    x = (np.sin(i * np.float32(0.013)) + 1j * np.cos(i * np.float32(0.021))).astype(np.complex64)
    got = oracle.four_step(x, l1, l2)
    assert _per_bin_rel(got, oracle.fft_1d(x, l1 + l2).astype(np.complex128)) < 1e-3


# ------------------------------------------------- planted-mistake checks


def test_checks_reject_planted_mistakes():
    """Plausible oracle bugs (sign, index, transposition, dropped twiddle,
    missing scale) each fail the golden comparison used above."""
    g = _golden("fft1d_numpy.npz")
    x, exp = g["in_unif_n8"], g["fwd_unif_n8"]
    good = oracle.fft_1d(x, 8)
    assert rel_l2(good, exp) < 1e-6
    assert rel_l2(np.conj(good), exp) > 1e-2                     # wrong sign of the exponent
    assert rel_l2(np.roll(good, 1), exp) > 1e-2                  # off-by-one output index
    assert rel_l2(good[::-1], exp) > 1e-2                        # reversed bins
    buf = x.copy()
    buf[3] = 0                                                   # dropped input term
    assert rel_l2(oracle.fft_1d(buf, 8), exp) > 1e-3
    inv = oracle.fft_1d(good, 8, "inverse", True)
    assert rel_l2(inv * 256, x) > 1e-2                           # scale applied twice/missing
    g2 = _golden("fft2d_numpy.npz")
    x2, exp2 = g2["in_sincos_n5"], g2["fwd_sincos_n5"]
    good2 = oracle.fft_2d(x2, 5)
    assert rel_l2(good2, exp2) < 1e-6
    assert rel_l2(good2.T, exp2) > 1e-2                          # transposed operand
    # a radix-2 stage with its twiddles dropped (all ones) differs from the DFT
    lane = _slow_input(16, 1)
    no_tw = oracle.radix4_forward_lane(lane, 4, np.ones_like(oracle.twiddles_radix4(4)))
    assert _per_bin_rel(no_tw, np.fft.fft(lane.astype(np.complex128))) > 1e-2


# ------------------------------------------------------- pointwise kernels


def _numpy_cmul_f32(ar, ai, br, bi):
    # float32 numpy arithmetic rounds each product and the sum to f32: the
    # reference's unfused `ar * br - ai * bi`, `ar * bi + ai * br`.
    return ar * br - ai * bi, ar * bi + ai * br


@pytest.mark.parametrize("n", [1, 7, 4096, 100003])
def test_cmul_matches_numpy_f32_exactly(n):
    rng = np.random.default_rng(n)
    a, b = uniform_c64(rng, n), uniform_c64(rng, n)
    re, im = _numpy_cmul_f32(a.real.copy(), a.imag.copy(), b.real.copy(), b.imag.copy())
    got = oracle.cmul_interleaved(a, b)
    assert np.array_equal(got.real, re) and np.array_equal(got.imag, im)
    s_re, s_im = oracle.cmul_split(a.real, a.imag, b.real, b.imag)
    assert np.array_equal(s_re, re) and np.array_equal(s_im, im)
    # complex128 product rounded once differs from the f32 formula by at most
    # a few ulps of the operands' magnitude (sanity of the operand roles)
    ref = (a.astype(np.complex128) * b.astype(np.complex128))
    assert np.max(np.abs(got - ref)) < 1e-6


def test_cmul_closed_forms():
    z = np.array([0.5 - 1.25j, 3 + 4j, -2.5 + 0.125j], np.complex64)
    i = np.full(3, 1j, np.complex64)
    assert np.array_equal(oracle.cmul_interleaved(i, i), np.full(3, -1, np.complex64))
    zz = oracle.cmul_interleaved(z, np.conj(z))
    assert np.array_equal(zz.imag, np.zeros(3, np.float32))      # ar*(-ai) + ai*ar = 0 exactly
    assert np.array_equal(zz.real, np.array([1.8125, 25, 6.265625], np.float32))
    one = np.ones(3, np.complex64)
    assert np.array_equal(oracle.cmul_interleaved(z, one), z)


def test_deinterleave_interleave_are_views_and_inverses():
    x = uniform_c64(np.random.default_rng(5), 1001)
    re, im = oracle.deinterleave(x)
    assert np.array_equal(re, x.real) and np.array_equal(im, x.imag)
    assert np.array_equal(oracle.interleave(re, im), x)
    assert np.array_equal(oracle.interleave(x.real, x.imag), x)


def test_pointwise_checks_reject_planted_mistakes():
    rng = np.random.default_rng(9)
    a, b = uniform_c64(rng, 64), uniform_c64(rng, 64)
    re, im = _numpy_cmul_f32(a.real.copy(), a.imag.copy(), b.real.copy(), b.imag.copy())
    wrong = [oracle.cmul_interleaved(a, np.conj(b)),                 # conjugated operand
             oracle.cmul_interleaved(a, b[::-1].copy()),              # wrong index
             oracle.cmul_interleaved(np.conj(a), np.conj(b)),         # sign of the imaginary part
             oracle.interleave(*oracle.deinterleave(a * 1j)) * b]     # swapped parts
    for w in wrong:
        assert not (np.array_equal(w.real, re) and np.array_equal(w.imag, im))
    sw_re, sw_im = oracle.deinterleave(a)
    assert not np.array_equal(oracle.interleave(sw_im, sw_re), a)   # re/im swapped


# ------------------------------------------------------- synthetic data

M64 = 2**64 - 1


def _splitmix64_py(seed, j):
    z = (seed + (j + 1) * 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def test_splitmix64_known_answers():
    # the generator's published first outputs for seed 0 (splitmix64.c)
    assert [oracle.splitmix64_at(0, j) for j in range(4)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    rng = np.random.default_rng(0)
    for seed, j in zip(rng.integers(0, 2**63, 20), rng.integers(0, 2**40, 20)):
        assert oracle.splitmix64_at(int(seed), int(j)) == _splitmix64_py(int(seed), int(j))


def test_fill_uniform_grid_and_moments():
    x = oracle.fill_uniform_c64(1000, 7).view(np.float32)
    exp = np.array([(_splitmix64_py(7, j) >> 40) * 2.0**-23 - 1 for j in range(2000)])
    assert np.array_equal(x.astype(np.float64), exp)       # exact: 24-bit values on a 2^-23 grid
    big = oracle.fill_uniform_c64(1 << 20, 1).view(np.float32).astype(np.float64)
    assert big.min() >= -1 and big.max() < 1
    assert abs(big.mean()) < 5 * np.sqrt(1 / 3 / big.size)
    assert abs(big.var() - 1 / 3) < 0.002


def test_fill_normal_box_muller_and_moments():
    import math

    x = oracle.fill_normal_c64(500, 3)
    for i in range(500):
        u1 = ((_splitmix64_py(3, 2 * i) >> 11) + 1) * 2.0**-53
        u2 = (_splitmix64_py(3, 2 * i + 1) >> 11) * 2.0**-53
        r = math.sqrt(-2.0 * math.log(u1))
        assert x[i].real == np.float32(r * math.cos(2 * math.pi * u2))
        assert x[i].imag == np.float32(r * math.sin(2 * math.pi * u2))
    big = oracle.fill_normal_c64(1 << 20, 4).view(np.float32).astype(np.float64)
    assert abs(big.mean()) < 5 / np.sqrt(big.size)
    assert abs(big.var() - 1) < 0.005
    assert abs(np.mean(np.abs(big) > 3) - 0.0026998) < 0.0005   # two-sided 3-sigma tail


def test_fill_checks_reject_planted_mistakes():
    known = 0xE220A8397B1DCDAF

    def mix(z, s1=30, s2=27, s3=31):
        z = ((z ^ (z >> s1)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> s2)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> s3)

    gamma = 0x9E3779B97F4A7C15
    assert mix(gamma) == known                                   # the formula as restated
    assert mix(0) != known                                       # counter j instead of j + 1
    assert mix(gamma, 31, 27, 30) != known                       # shifts swapped
    assert mix((gamma << 1) & M64) != known                      # stride doubled (interleaving bug)
    # uniform mapping: a 23-bit field or a missing offset leaves the grid / range
    z = oracle.splitmix64_at(7, 0)
    good = (z >> 40) * 2.0**-23 - 1
    assert oracle.fill_uniform_c64(1, 7).real[0] == np.float32(good)
    assert (z >> 41) * 2.0**-23 - 1 != good and (z >> 40) * 2.0**-23 != good

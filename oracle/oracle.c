/*
 * oracle.c -- TEST INFRASTRUCTURE ONLY.  CPU restatement of the reference's
 * FFT host library (the .rs files of crates/ferrum-gpu-fft/src in the reference tree).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it, as the checker; the product path never does.
 *
 * Rules kept from the reference so results agree to the last bit where the
 * reference is deterministic:
 *   - f32 arithmetic everywhere except the fp64 direct DFT;
 *   - complex multiply as (a.re*b.re - a.im*b.im, a.re*b.im + a.im*b.re)
 *     with no fused multiply-add (complex.rs:27-32; built -ffp-contract=off);
 *   - twiddle angles formed in f32 as (-2*PI/m as f32) * (k as f32) and
 *     evaluated with libm cosf/sinf, which is what Rust's f32::cos/sin call
 *     on Linux (twiddles.rs:14-20).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct { float re, im; } c32;

static const float PI_F = 3.14159265358979323846f; /* core::f32::consts::PI */

/* complex.rs:27-32 */
static inline c32 cmul(c32 a, c32 b) {
    c32 r;
    r.re = a.re * b.re - a.im * b.im;
    r.im = a.re * b.im + a.im * b.re;
    return r;
}
static inline c32 cadd(c32 a, c32 b) { c32 r = {a.re + b.re, a.im + b.im}; return r; }
static inline c32 csub(c32 a, c32 b) { c32 r = {a.re - b.re, a.im - b.im}; return r; }

/* ---------------------------------------------------------------- twiddles */

/* twiddles.rs:10-23: stages log_n..1 descending; W_{2^s}^k for k < 2^(s-1). */
void or_twiddles(uint32_t log_n, float *out) {
    size_t o = 0;
    for (uint32_t stage = log_n; stage >= 1; --stage) {
        uint64_t n_stage = 1ull << stage;
        size_t half = (size_t)(n_stage / 2);
        float scale = -2.0f * PI_F / (float)n_stage;
        for (size_t k = 0; k < half; ++k) {
            float theta = scale * (float)k;
            out[o++] = cosf(theta);
            out[o++] = sinf(theta);
        }
    }
}

/* Shared body of twiddles_radix4 (twiddles.rs:33-54) and twiddles_radix8
 * (twiddles.rs:83-104): ascending stages, [k][p] = W_m^((p*k) mod m). */
static size_t radix_table_len(uint32_t log_n, uint32_t log_r) {
    size_t r = (size_t)1 << log_r, m_r = 1, len = 0;
    for (uint32_t s = 1; s <= log_n / log_r; ++s) { len += r * m_r; m_r *= r; }
    return len;
}
static void radix_table(uint32_t log_n, uint32_t log_r, float *out) {
    size_t r = (size_t)1 << log_r, m_r = 1, o = 0;
    for (uint32_t s = 1; s <= log_n / log_r; ++s) {
        size_t m = m_r * r;
        float scale = -2.0f * PI_F / (float)m;
        for (size_t k = 0; k < m_r; ++k) {
            for (size_t p = 0; p < r; ++p) {
                size_t e = (p * k) % m;
                float theta = scale * (float)e;
                out[o++] = cosf(theta);
                out[o++] = sinf(theta);
            }
        }
        m_r = m;
    }
}
size_t or_twiddles_radix4_len(uint32_t log_n) { return radix_table_len(log_n, 2); }
void or_twiddles_radix4(uint32_t log_n, float *out) { radix_table(log_n, 2, out); }
size_t or_twiddles_radix8_len(uint32_t log_n) { return radix_table_len(log_n, 3); }
void or_twiddles_radix8(uint32_t log_n, float *out) { radix_table(log_n, 3, out); }

/* twiddles.rs:60-69 */
void or_twiddles_full_roots(uint32_t log_n, float *out) {
    size_t n = (size_t)1 << log_n;
    float scale = -2.0f * PI_F / (float)n;
    for (size_t e = 0; e < n; ++e) {
        float theta = scale * (float)e;
        out[2 * e] = cosf(theta);
        out[2 * e + 1] = sinf(theta);
    }
}

/* ------------------------------------------------------- radix-2 Stockham */

/* cpu.rs:15-23 */
void or_stage_offsets(uint32_t log_n, size_t *offs) {
    size_t off = 0;
    for (uint32_t i = 0; i <= log_n; ++i) offs[i] = 0;
    for (uint32_t s = log_n; s >= 1; --s) {
        offs[s] = off;
        off += (size_t)1 << (s - 1);
    }
}

/* cpu.rs:30-45: one radix-2 Stockham stage src -> dst. */
static void stockham_stage(const c32 *src, c32 *dst, size_t n, uint32_t s, const c32 *tw) {
    size_t m = (size_t)1 << s, m_half = (size_t)1 << (s - 1);
    size_t l = n / m, half_n = n / 2;
    for (size_t j = 0; j < l; ++j) {
        for (size_t k = 0; k < m_half; ++k) {
            c32 w = tw[k];
            c32 a = src[j * m_half + k];
            c32 b = src[j * m_half + k + half_n];
            c32 wb = cmul(w, b);
            dst[j * m + k] = cadd(a, wb);
            dst[j * m + k + m_half] = csub(a, wb);
        }
    }
}

/* cpu.rs:51-81: ping-pong buf <-> scratch, copy back when log_n is odd. */
static void forward_lane(c32 *buf, c32 *scratch, uint32_t log_n, const c32 *tw,
                         const size_t *offs) {
    size_t n = (size_t)1 << log_n;
    int from_buf_to_scratch = 1;
    for (uint32_t s = 1; s <= log_n; ++s) {
        const c32 *t = tw + offs[s];
        if (from_buf_to_scratch) stockham_stage(buf, scratch, n, s, t);
        else stockham_stage(scratch, buf, n, s, t);
        from_buf_to_scratch = !from_buf_to_scratch;
    }
    if (log_n % 2 == 1) memcpy(buf, scratch, n * sizeof(c32));
}

/* Plan::new (plan.rs:57-68) builds twiddles(log_n); Plan::cpu_execute
 * (cpu.rs:90-124) runs every lane; the inverse is conj -> forward -> conj and
 * then x (1.0f32 / n as f32) when normalize is set.  The reference asserts
 * log_n in [2, 12] (plan.rs:58); the algorithm is generic, so this
 * restatement accepts [1, 30]. */
int or_fft_1d_lanes(float *bufp, uint32_t log_n, size_t lane_begin, size_t lane_end,
                    int dir, int normalize) {
    if (log_n < 1 || log_n > 30 || (dir != 1 && dir != -1)) return -1;
    size_t n = (size_t)1 << log_n;
    c32 *buf = (c32 *)bufp;
    c32 *tw = (c32 *)malloc((n - 1 + 1) * sizeof(c32));
    c32 *scratch = (c32 *)malloc(n * sizeof(c32));
    size_t offs[32];
    if (!tw || !scratch) { free(tw); free(scratch); return -2; }
    or_twiddles(log_n, (float *)tw);
    or_stage_offsets(log_n, offs);
    for (size_t lane_i = lane_begin; lane_i < lane_end; ++lane_i) {
        c32 *lane = buf + lane_i * n;
        if (dir == 1) {
            forward_lane(lane, scratch, log_n, tw, offs);
        } else {
            for (size_t i = 0; i < n; ++i) lane[i].im = -lane[i].im;
            forward_lane(lane, scratch, log_n, tw, offs);
            for (size_t i = 0; i < n; ++i) lane[i].im = -lane[i].im;
            if (normalize) {
                float inv_n = 1.0f / (float)n;
                for (size_t i = 0; i < n; ++i) { lane[i].re *= inv_n; lane[i].im *= inv_n; }
            }
        }
    }
    free(tw);
    free(scratch);
    return 0;
}

int or_fft_1d(float *buf, uint32_t log_n, size_t batch, int dir, int normalize) {
    if (batch == 0) return -1; /* cpu.rs:92-97: positive multiple of n */
    return or_fft_1d_lanes(buf, log_n, 0, batch, dir, normalize);
}

/* ------------------------------------------------------------------- 2D */

/* cpu_2d.rs:67-73 */
void or_transpose_square(float *bufp, size_t n) {
    c32 *buf = (c32 *)bufp;
    for (size_t i = 0; i < n; ++i)
        for (size_t j = i + 1; j < n; ++j) {
            c32 t = buf[i * n + j];
            buf[i * n + j] = buf[j * n + i];
            buf[j * n + i] = t;
        }
}

/* cpu_2d.rs:9-64: optional conj, row pass (1D plan, batch n, normalize off),
 * transpose, row pass, transpose back, optional conj and x 1/(n*n). */
int or_fft_2d(float *bufp, uint32_t log_n, size_t batch, int dir, int normalize) {
    if (log_n < 1 || log_n > 15 || (dir != 1 && dir != -1) || batch == 0) return -1;
    size_t n = (size_t)1 << log_n, total = n * n;
    for (size_t b = 0; b < batch; ++b) {
        c32 *buf = (c32 *)bufp + b * total;
        if (dir == -1)
            for (size_t i = 0; i < total; ++i) buf[i].im = -buf[i].im;
        int rc = or_fft_1d((float *)buf, log_n, n, 1, 0);
        if (rc) return rc;
        or_transpose_square((float *)buf, n);
        rc = or_fft_1d((float *)buf, log_n, n, 1, 0);
        if (rc) return rc;
        or_transpose_square((float *)buf, n);
        if (dir == -1) {
            for (size_t i = 0; i < total; ++i) buf[i].im = -buf[i].im;
            if (normalize) {
                float scale = 1.0f / ((float)n * (float)n);
                for (size_t i = 0; i < total; ++i) { buf[i].re *= scale; buf[i].im *= scale; }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------ radix-4 / radix-8 */

/* cpu_radix4.rs:16-35 */
void or_dft4_inplace(float x[8]) {
    float x0r = x[0], x0i = x[1], x1r = x[2], x1i = x[3];
    float x2r = x[4], x2i = x[5], x3r = x[6], x3i = x[7];
    float ar = x0r + x2r, ai = x0i + x2i;
    float br = x0r - x2r, bi = x0i - x2i;
    float cr = x1r + x3r, ci = x1i + x3i;
    float dr = x1r - x3r, di = x1i - x3i;
    x[0] = ar + cr; x[1] = ai + ci;
    x[2] = br + di; x[3] = bi - dr;
    x[4] = ar - cr; x[5] = ai - ci;
    x[6] = br - di; x[7] = bi + dr;
}

/* cpu_radix8.rs:25-79 */
void or_dft8_inplace(float x[16]) {
    const float C = 0.70710678118654752440f; /* FRAC_1_SQRT_2 */
    float x0r = x[0], x0i = x[1], x1r = x[2], x1i = x[3];
    float x2r = x[4], x2i = x[5], x3r = x[6], x3i = x[7];
    float x4r = x[8], x4i = x[9], x5r = x[10], x5i = x[11];
    float x6r = x[12], x6i = x[13], x7r = x[14], x7i = x[15];
    float a0r = x0r + x4r, a0i = x0i + x4i, a1r = x0r - x4r, a1i = x0i - x4i;
    float b0r = x2r + x6r, b0i = x2i + x6i, b1r = x2r - x6r, b1i = x2i - x6i;
    float e0r = a0r + b0r, e0i = a0i + b0i, e2r = a0r - b0r, e2i = a0i - b0i;
    float e1r = a1r + b1i, e1i = a1i - b1r, e3r = a1r - b1i, e3i = a1i + b1r;
    float c0r = x1r + x5r, c0i = x1i + x5i, c1r = x1r - x5r, c1i = x1i - x5i;
    float d0r = x3r + x7r, d0i = x3i + x7i, d1r = x3r - x7r, d1i = x3i - x7i;
    float o0r = c0r + d0r, o0i = c0i + d0i, o2r = c0r - d0r, o2i = c0i - d0i;
    float o1r = c1r + d1i, o1i = c1i - d1r, o3r = c1r - d1i, o3i = c1i + d1r;
    float w0r = o0r, w0i = o0i;
    float w1r = C * (o1r + o1i), w1i = C * (o1i - o1r);
    float w2r = o2i, w2i = -o2r;
    float w3r = C * (o3i - o3r), w3i = -C * (o3r + o3i);
    x[0] = e0r + w0r;  x[1] = e0i + w0i;  x[2] = e1r + w1r;  x[3] = e1i + w1i;
    x[4] = e2r + w2r;  x[5] = e2i + w2i;  x[6] = e3r + w3r;  x[7] = e3i + w3i;
    x[8] = e0r - w0r;  x[9] = e0i - w0i;  x[10] = e1r - w1r; x[11] = e1i - w1i;
    x[12] = e2r - w2r; x[13] = e2i - w2i; x[14] = e3r - w3r; x[15] = e3i - w3i;
}

/* Shared Stockham driver of radix4_forward_lane (cpu_radix4.rs:40-97) and
 * radix8_forward_lane (cpu_radix8.rs:86-145): gather src[j*m_r+k+p*(n/r)],
 * twiddle tw[stage_off + r*k + p] (p > 0), DFT-r, scatter dst[j*m+k+q*m_r]. */
static void radix_r_forward_lane(float *lane, float *scratch, uint32_t log_n,
                                 const float *twf, uint32_t log_r) {
    const c32 *tw = (const c32 *)twf;
    size_t n = (size_t)1 << log_n, r = (size_t)1 << log_r;
    uint32_t stages = log_n / log_r;
    size_t nr = n / r, butterflies = n / r;
    int src_is_lane = 1;
    size_t m_r = 1, stage_off = 0;
    for (uint32_t s = 1; s <= stages; ++s) {
        size_t m = m_r * r;
        for (size_t b = 0; b < butterflies; ++b) {
            size_t j = b / m_r, k = b - j * m_r, src_base = j * m_r + k;
            float x[16];
            for (size_t p = 0; p < r; ++p) {
                size_t si = 2 * (src_base + p * nr);
                const float *src = src_is_lane ? lane : scratch;
                float re = src[si], im = src[si + 1];
                if (p == 0) { x[0] = re; x[1] = im; }
                else {
                    c32 w = tw[stage_off + r * k + p];
                    x[2 * p] = re * w.re - im * w.im;
                    x[2 * p + 1] = re * w.im + im * w.re;
                }
            }
            if (log_r == 2) or_dft4_inplace(x); else or_dft8_inplace(x);
            size_t dst_base = j * m + k;
            float *dst = src_is_lane ? scratch : lane;
            for (size_t q = 0; q < r; ++q) {
                size_t di = 2 * (dst_base + q * m_r);
                dst[di] = x[2 * q];
                dst[di + 1] = x[2 * q + 1];
            }
        }
        stage_off += r * m_r;
        m_r = m;
        src_is_lane = !src_is_lane;
    }
    if (stages % 2 == 1) memcpy(lane, scratch, 2 * n * sizeof(float));
}
void or_radix4_forward_lane(float *lane, float *scratch, uint32_t log_n, const float *tw) {
    radix_r_forward_lane(lane, scratch, log_n, tw, 2);
}
void or_radix8_forward_lane(float *lane, float *scratch, uint32_t log_n, const float *tw) {
    radix_r_forward_lane(lane, scratch, log_n, tw, 3);
}

/* ------------------------------------------------------- four-step model */

/* warp_fft.rs:21-25: W_n^e with the angle formed in f32. */
static c32 twiddle_f32(size_t e, size_t n) {
    float theta = -2.0f * PI_F * (float)e / (float)n;
    c32 w = {cosf(theta), sinf(theta)};
    return w;
}

static size_t bitrev(size_t i, uint32_t log_n) {
    size_t r = 0;
    for (uint32_t b = 0; b < log_n; ++b)
        if (i & ((size_t)1 << b)) r |= (size_t)1 << (log_n - 1 - b);
    return r;
}

/* warp_fft.rs:56-77: radix-2 DIF with partner g^d, twiddle on the upper
 * element, bit-reversal unscramble at the end. */
void or_warp_dif(float *xp, uint32_t log_n) {
    c32 *x = (c32 *)xp;
    size_t n = (size_t)1 << log_n;
    c32 *cur = (c32 *)malloc(n * sizeof(c32));
    for (uint32_t s = 0; s < log_n; ++s) {
        size_t d = (n >> 1) >> s;
        memcpy(cur, x, n * sizeof(c32));
        for (size_t g = 0; g < n; ++g) {
            c32 partner = cur[g ^ d];
            if ((g & d) == 0) x[g] = cadd(cur[g], partner);
            else {
                c32 diff = csub(partner, cur[g]);
                size_t e = (g & (d - 1)) * ((size_t)1 << s);
                x[g] = cmul(diff, twiddle_f32(e, n));
            }
        }
    }
    memcpy(cur, x, n * sizeof(c32));
    for (size_t g = 0; g < n; ++g) x[bitrev(g, log_n)] = cur[g];
    free(cur);
}

/* warp_fft.rs:122-155: n = n1 + N1*n2, k = N2*k1 + k2. */
void or_four_step(const float *inp, float *outp, uint32_t log_n1, uint32_t log_n2) {
    const c32 *in = (const c32 *)inp;
    c32 *out = (c32 *)outp;
    size_t n1 = (size_t)1 << log_n1, n2 = (size_t)1 << log_n2, n = n1 * n2;
    c32 *b = (c32 *)malloc(n * sizeof(c32));
    c32 *col = (c32 *)malloc((n1 > n2 ? n1 : n2) * sizeof(c32));
    for (size_t a = 0; a < n1; ++a) {
        for (size_t c = 0; c < n2; ++c) col[c] = in[a + n1 * c];
        or_warp_dif((float *)col, log_n2);
        for (size_t k2 = 0; k2 < n2; ++k2) b[a * n2 + k2] = col[k2];
    }
    for (size_t a = 0; a < n1; ++a)
        for (size_t k2 = 0; k2 < n2; ++k2)
            b[a * n2 + k2] = cmul(b[a * n2 + k2], twiddle_f32(a * k2, n));
    for (size_t k2 = 0; k2 < n2; ++k2) {
        for (size_t a = 0; a < n1; ++a) col[a] = b[a * n2 + k2];
        or_warp_dif((float *)col, log_n1);
        for (size_t k1 = 0; k1 < n1; ++k1) out[n2 * k1 + k2] = col[k1];
    }
    free(b);
    free(col);
}

/* ------------------------------------------------------ fp64 direct DFT */

/* layout_study.rs:5-21 */
void or_dft_naive(const float *in, float *out, size_t n) {
    for (size_t k = 0; k < n; ++k) {
        double sr = 0.0, si = 0.0;
        for (size_t t = 0; t < n; ++t) {
            double ang = -2.0 * 3.14159265358979323846 * (double)k * (double)t / (double)n;
            double c = cos(ang), s = sin(ang);
            double xr = in[2 * t], xi = in[2 * t + 1];
            sr += xr * c - xi * s;
            si += xr * s + xi * c;
        }
        out[2 * k] = (float)sr;
        out[2 * k + 1] = (float)si;
    }
}

/* The layout_study.rs:5-21 sum at selected bins, fp64 result.  The exponent
 * k*t is reduced mod n in integers first so the angle stays exact for the
 * 2^24-point spot checks. */
void or_dft_bins_f64(const float *in, size_t n, const int64_t *bins, size_t nbins,
                     int sign, double *out) {
    const double two_pi = 2.0 * 3.14159265358979323846;
    for (size_t bi = 0; bi < nbins; ++bi) {
        uint64_t k = (uint64_t)bins[bi] % n;
        double sr = 0.0, si = 0.0;
        uint64_t e = 0; /* (k*t) mod n, advanced incrementally */
        for (size_t t = 0; t < n; ++t) {
            double ang = (sign < 0 ? -two_pi : two_pi) * (double)e / (double)n;
            double c = cos(ang), s = sin(ang);
            double xr = in[2 * t], xi = in[2 * t + 1];
            sr += xr * c - xi * s;
            si += xr * s + xi * c;
            e += k;
            if (e >= n) e -= n;
        }
        out[2 * bi] = sr;
        out[2 * bi + 1] = si;
    }
}

/* ---- pointwise kernels ----------------------------------------------------
 * One element per kernel thread in the reference; the products are written
 * ar*br - ai*bi and ar*bi + ai*br, two f32 roundings and a rounded sum (the
 * file is built with -ffp-contract=off, as Rust does not contract). */

void or_cmul_interleaved(const float *a, const float *b, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float ar = a[2 * i], ai = a[2 * i + 1];
        const float br = b[2 * i], bi = b[2 * i + 1];
        out[2 * i] = ar * br - ai * bi;
        out[2 * i + 1] = ar * bi + ai * br;
    }
}

void or_cmul_split(const float *a_re, const float *a_im, const float *b_re, const float *b_im,
                   float *o_re, float *o_im, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float ar = a_re[i], ai = a_im[i], br = b_re[i], bi = b_im[i];
        o_re[i] = ar * br - ai * bi;
        o_im[i] = ar * bi + ai * br;
    }
}

void or_deinterleave(const float *in, float *re, float *im, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        re[i] = in[2 * i];
        im[i] = in[2 * i + 1];
    }
}

void or_interleave(const float *re, const float *im, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        out[2 * i] = re[i];
        out[2 * i + 1] = im[i];
    }
}

/* ---- seeded synthetic data ------------------------------------------------- */

uint64_t or_splitmix64_at(uint64_t seed, uint64_t j) {
    uint64_t z = seed + (j + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void or_fill_uniform_c64(float *out, size_t n, uint64_t seed) {
    for (size_t j = 0; j < 2 * n; ++j) {
        uint32_t u = (uint32_t)(or_splitmix64_at(seed, j) >> 40);
        out[j] = (float)u * 0x1p-23f - 1.0f;
    }
}

void or_fill_normal_c64(float *out, size_t n, uint64_t seed) {
    for (size_t i = 0; i < n; ++i) {
        double u1 = (double)((or_splitmix64_at(seed, 2 * i) >> 11) + 1) * 0x1p-53;
        double u2 = (double)(or_splitmix64_at(seed, 2 * i + 1) >> 11) * 0x1p-53;
        double r = sqrt(-2.0 * log(u1));
        double a = 6.283185307179586476925286766559 * u2;
        out[2 * i] = (float)(r * cos(a));
        out[2 * i + 1] = (float)(r * sin(a));
    }
}

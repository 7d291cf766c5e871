/*
 * oracle.h -- CPU restatement of ferrum-gpu's FFT host library, used ONLY as
 * test infrastructure (the checker in tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py).  Nothing in the product links or calls it.
 *
 * Every function restates one function of the reference Rust crate
 * `crates/ferrum-gpu-fft` (paths relative to the reference root) with the
 * same f32 operation order.  Complex values are interleaved (re, im) float
 * pairs, exactly the layout of `Complex32` (crates/ferrum-gpu-fft/src/complex.rs:10-53).
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off: the Rust source has no
 * fused multiply-adds, so contraction is disabled to keep the op order).
 */
#ifndef FERRUM_ORACLE_H
#define FERRUM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- twiddle tables (crates/ferrum-gpu-fft/src/twiddles.rs) ------------- */

/* Radix-2 stage table, stages descending, length 2^log_n - 1 (twiddles.rs:10-23). */
void or_twiddles(uint32_t log_n, float *out);
/* Radix-4 per-stage [k][p] input twiddles, length 4(N-1)/3 (twiddles.rs:33-54). */
size_t or_twiddles_radix4_len(uint32_t log_n);
void or_twiddles_radix4(uint32_t log_n, float *out);
/* Flat W_N^e table, e < N (twiddles.rs:60-69). */
void or_twiddles_full_roots(uint32_t log_n, float *out);
/* Radix-8 per-stage [k][p] input twiddles (twiddles.rs:83-104). */
size_t or_twiddles_radix8_len(uint32_t log_n);
void or_twiddles_radix8(uint32_t log_n, float *out);

/* ---- radix-2 Stockham reference (crates/ferrum-gpu-fft/src/cpu.rs) ------ */

/* stage_offsets (cpu.rs:15-23): offs[s] for s in 1..=log_n; offs has log_n+1 slots. */
void or_stage_offsets(uint32_t log_n, size_t *offs);
/* Plan::new(log_n, batch, normalize) + Plan::cpu_execute(buf, dir) (plan.rs:57-68,
 * cpu.rs:90-124).  buf holds batch*N complex, processed in place.  dir: +1
 * forward, -1 inverse.  Returns 0, or -1 on a bad argument. */
int or_fft_1d(float *buf, uint32_t log_n, size_t batch, int dir, int normalize);
/* Same over lanes [lane_begin, lane_end) only, so callers can split a batch
 * across threads (each lane is independent in cpu.rs:101). */
int or_fft_1d_lanes(float *buf, uint32_t log_n, size_t lane_begin, size_t lane_end,
                    int dir, int normalize);

/* ---- 2D (crates/ferrum-gpu-fft/src/cpu_2d.rs) --------------------------- */

/* Plan2D::new(log_n, normalize) + Plan2D::cpu_execute (cpu_2d.rs:9-64) on one
 * N x N row-major image; `batch` images back to back. */
int or_fft_2d(float *buf, uint32_t log_n, size_t batch, int dir, int normalize);
/* transpose_square (cpu_2d.rs:67-73). */
void or_transpose_square(float *buf, size_t n);

/* ---- radix-4 / radix-8 executable specs (cpu_radix4.rs, cpu_radix8.rs) -- */

void or_dft4_inplace(float x[8]);                 /* cpu_radix4.rs:16-35 */
void or_radix4_forward_lane(float *lane, float *scratch, uint32_t log_n,
                            const float *tw);     /* cpu_radix4.rs:40-97 */
void or_dft8_inplace(float x[16]);                /* cpu_radix8.rs:25-79 */
void or_radix8_forward_lane(float *lane, float *scratch, uint32_t log_n,
                            const float *tw);     /* cpu_radix8.rs:86-145 */

/* ---- four-step model (crates/ferrum-gpu-fft/src/warp_fft.rs) ------------ */

void or_warp_dif(float *x, uint32_t log_n);       /* warp_fft.rs:56-77 */
/* four_step_model(input, log_n1, log_n2) (warp_fft.rs:122-155): out[N2*k1+k2]. */
void or_four_step(const float *in, float *out, uint32_t log_n1, uint32_t log_n2);

/* ---- fp64 direct DFT (crates/ferrum-gpu-fft/src/layout_study.rs:5-21) --- */

/* O(N^2) forward DFT of n points, f64 angle and accumulation, rounded to f32. */
void or_dft_naive(const float *in, float *out, size_t n);
/* The same sum evaluated only at the listed bins; out is double (re, im)
 * pairs so spot checks keep the fp64 accuracy.  sign = -1 forward, +1 inverse
 * (unnormalised). */
void or_dft_bins_f64(const float *in, size_t n, const int64_t *bins, size_t nbins,
                     int sign, double *out);

/* ---- pointwise kernels (crates/ferrum-gpu-fft-kernels/src/kernels_body.rs) -- */

/* out = a * b over n interleaved complex (cmul_interleaved, :1612-1627). */
void or_cmul_interleaved(const float *a, const float *b, float *out, size_t n);
/* (o_re, o_im) = (a_re, a_im) * (b_re, b_im) over n elements (cmul_split, :1629-1645). */
void or_cmul_split(const float *a_re, const float *a_im, const float *b_re, const float *b_im,
                   float *o_re, float *o_im, size_t n);
/* re[i], im[i] = in[2i], in[2i+1] (deinterleave, :1647-1659). */
void or_deinterleave(const float *in, float *re, float *im, size_t n);
/* out[2i], out[2i+1] = re[i], im[i] (interleave, :1661-1671). */
void or_interleave(const float *re, const float *im, float *out, size_t n);

/* ---- seeded synthetic data (the generator of the benchmark configurations) --
 * Float j of the output uses splitmix64 at state seed + (j+1)*0x9E3779B97F4A7C15
 * (Steele, Lea, Flood, OOPSLA 2014; Vigna's splitmix64.c constants).
 * uniform: (z >> 40) * 2^-23 - 1; normal: f64 Box-Muller on (z(2i), z(2i+1)). */
uint64_t or_splitmix64_at(uint64_t seed, uint64_t j);
void or_fill_uniform_c64(float *out, size_t n, uint64_t seed);
void or_fill_normal_c64(float *out, size_t n, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif

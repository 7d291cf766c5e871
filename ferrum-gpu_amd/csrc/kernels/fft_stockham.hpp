// fft_stockham.hpp -- LDS-resident batched power-of-two C2C FFT for
// N = 2^LOGN <= 4096, one (or several) transforms per workgroup.
//
// Algorithm: mixed-radix Stockham autosort, the same stage recurrence as the
// reference's radix-4/radix-8 specs (crates/ferrum-gpu-fft/src/cpu_radix4.rs:6-9,
// cpu_radix8.rs:11-15) generalised to a radix list (E, E, ..., E, r) with
// E = 2^LOGE elements held in VGPRs per thread:
//   stage s, radix R, L = product of earlier radices, butterfly b = j*L + k:
//     gather  src[b + p*(N/R)]              p in [0, R)
//     twiddle t_p = W_{L*R}^{p*k} * src_p    (factored table; none when L == 1)
//     DFT-R   X = DFT_R(t)
//     scatter dst[j*L*R + k + q*L] = X_q    q in [0, R)
// Thread t of a transform always gathers positions t + T*m (m in [0, E)), so
// the first stage reads global memory coalesced; the last stage has j == 0 and
// scatters to positions t + T*m as well, so it writes global memory coalesced.
// Intermediate stages exchange through LDS with one pad slot per 16 entries,
// which breaks the stride-E pattern of the first scatter across LDS banks.
//
// Inverse: conjugate on load, conjugate (and scale) on store (runtime flags,
// so a multi-pass plan can apply each half in a different pass).
#pragma once
#include "fft_common.hpp"
#include "tile_geom.h"

namespace fg {

template <int LOGN, int LOGE>
struct StockhamShape {
    static constexpr int N = 1 << LOGN;
    static constexpr int E = 1 << LOGE;                  // elements per thread
    static constexpr int T = N / E;                      // threads per transform
    static constexpr int NFULL = LOGN / LOGE;            // radix-E stages
    static constexpr int REM = LOGN % LOGE;              // log2 of the tail radix
    static constexpr int NSTAGES = NFULL + (REM ? 1 : 0);
    static constexpr int LDS_ELEMS = N + N / 16;         // padded transform
    static_assert(LOGE <= LOGN, "more elements per thread than points");
};

// Padded LDS slot of logical position p: one pad slot per 2^SH positions
// (16 unless a caller's bank pattern wants another spacing).
template <int SH = 4>
__device__ __forceinline__ int lds_pos(int p) { return p + (p >> SH); }

// Stage twiddle table, built by the host for this radix list (stage 0 has no
// block).  The block of stage s (radix R, L = product of earlier radices,
// M = L*R) holds one row per k < L of W_M^{p*k} for the exponents
//   R = 16: p in {1, 2, 3, 4, 8, 12}   (the other nine are one product each,
//           W^{k*p} = W^{k*(p & 3)} * W^{k*4*(p >> 2)}, following the 4 x 4
//           split of the radix-16 butterfly)
//   R = 8:  p in {1, 2, 3, 4}          (p = 5..7: W^{k*(p-4)} * W^{4k})
//   R <= 4: p in [0, R)                (the full row)
// Rows are 16-byte multiples so they load as float4 pairs.  The factored rows
// keep a radix-16 stage's table at 6/16 of the full [k][p] block: at N = 4096
// the last stage's 32 KB table fell out of L1 and cost 19 % of the kernel time
// against 12 KB factored.
__host__ __device__ constexpr int tw_row_len(int R) { return R == 16 ? 6 : (R == 8 ? 4 : R); }

// A stage whose butterflies span L >= 1024 (the last, radix-2 or radix-4 stage
// of N = 2^13 and 2^14) would need L rows -- 64 / 128 KB that every
// workgroup streams through its L1.  Such a stage stores a two-level table
// instead, A[h] = W_M^{64 h} for h < L/64 followed by B[l] = W_M^l for
// l < 64 (M = L*R), and forms W^k = A[k >> 6] * B[k & 63], W^{2k} = (W^k)^2,
// W^{3k} = W^{2k} * W^k (up to five f32 roundings, under 6e-7).
__host__ __device__ constexpr bool tw_two_level(int L) { return L >= 1024; }
// Entries W^{64 h} of a two-level block: h < L/64 covers the exponents k < L
// of radix 2 and 4 (their W^2k, W^3k are products of W^k); radix 8 looks up
// W^2k and W^4k as well, so its block covers every exponent below L*R.
__host__ __device__ constexpr int tw_two_level_high(int L, int R) { return R == 8 ? L * R / 64 : L / 64; }
__host__ __device__ constexpr int tw_stage_entries(int L, int R) {
    return tw_two_level(L) ? tw_two_level_high(L, R) + 64 : L * tw_row_len(R);
}

template <int LOGN, int LOGE>
__host__ __device__ constexpr int stockham_tw_offset(int s) {
    int off = 0;
    for (int i = 1; i < s; ++i) {
        int logl = i * LOGE;
        int logr = (i < LOGN / LOGE) ? LOGE : (LOGN % LOGE);
        off += tw_stage_entries(1 << logl, 1 << logr);
    }
    return off;
}

// Multiplies input p of a radix-R butterfly by W^{p*k}, p >= 1, reading the
// row w of the table above.
template <int R>
__device__ __forceinline__ void apply_stage_twiddles(float2* u, const float2* __restrict__ w) {
    const float4* w4 = reinterpret_cast<const float4*>(w);
    if constexpr (R == 16 || R == 8) {
        const float4 a = w4[0], b = w4[1];
        const float2 lo[4] = {make_float2(1.f, 0.f), make_float2(a.x, a.y), make_float2(a.z, a.w),
                              make_float2(b.x, b.y)};
        float2 hi[4] = {make_float2(1.f, 0.f), make_float2(b.z, b.w), make_float2(1.f, 0.f),
                        make_float2(1.f, 0.f)};
        if constexpr (R == 16) {
            const float4 c = w4[2];
            hi[2] = make_float2(c.x, c.y);
            hi[3] = make_float2(c.z, c.w);
        }
#pragma unroll
        for (int p = 1; p < R; ++p) {
            const int pl = p & 3, ph = p >> 2;
            const float2 wp = (pl == 0) ? hi[ph] : (ph == 0 ? lo[pl] : cmul(lo[pl], hi[ph]));
            u[p] = cmul(u[p], wp);
        }
    } else if constexpr (R >= 2) {
#pragma unroll
        for (int p2 = 0; p2 < R / 2; ++p2) {
            const float4 ww = w4[p2];
            if (p2 > 0) u[2 * p2] = cmul(u[2 * p2], make_float2(ww.x, ww.y));
            u[2 * p2 + 1] = cmul(u[2 * p2 + 1], make_float2(ww.z, ww.w));
        }
    }
}

// Multiplies input p of a radix-R butterfly with k = b mod L by W_{L*R}^{p*k},
// from the block of the stage's table at `stage`.
template <int R, int L>
__device__ __forceinline__ void apply_stage_twiddles_at(float2* u, const float2* __restrict__ stage, int k) {
    if constexpr (tw_two_level(L)) {
        static_assert(R == 2 || R == 4 || R == 8, "two-level stages are radix 2, 4 or 8");
        constexpr int HI = tw_two_level_high(L, R);
        const float2 w1 = cmul(stage[k >> 6], stage[HI + (k & 63)]);
        u[1] = cmul(u[1], w1);
        if constexpr (R == 8) {
            // W^2k and W^4k looked up too, the other powers one product away:
            // at most three roundings from the table (2.4e-7 at 32768 points,
            // against 7e-7 for W^7k by repeated products of W^k)
            const float2 w2 = cmul(stage[(2 * k) >> 6], stage[HI + ((2 * k) & 63)]);
            const float2 w4 = cmul(stage[(4 * k) >> 6], stage[HI + ((4 * k) & 63)]);
            const float2 w3 = cmul(w1, w2);
            u[2] = cmul(u[2], w2);
            u[3] = cmul(u[3], w3);
            u[4] = cmul(u[4], w4);
            u[5] = cmul(u[5], cmul(w1, w4));
            u[6] = cmul(u[6], cmul(w2, w4));
            u[7] = cmul(u[7], cmul(w3, w4));
        }
        if constexpr (R == 4) {
            const float2 w2 = cmul(w1, w1);
            u[2] = cmul(u[2], w2);
            u[3] = cmul(u[3], cmul(w2, w1));
        }
    } else {
        apply_stage_twiddles<R>(u, stage + k * tw_row_len(R));
    }
}

// Processes one stage's butterflies for a thread: x holds the E gathered
// elements (position t + T*m at index m); on return x holds the outputs laid
// out so that output q of butterfly i sits at index i + NB*q.
template <int LOGN, int LOGE, int S>
__device__ __forceinline__ void stockham_stage_regs(float2* x, int t, const float2* __restrict__ tw) {
    using Sh = StockhamShape<LOGN, LOGE>;
    constexpr int LOGR = (S < Sh::NFULL) ? LOGE : Sh::REM;
    constexpr int R = 1 << LOGR;
    constexpr int NB = Sh::E / R;       // butterflies per thread
    constexpr int LOGL = S * LOGE;
    constexpr int L = 1 << LOGL;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        float2 u[R];
#pragma unroll
        for (int p = 0; p < R; ++p) u[p] = x[i + NB * p];
        if constexpr (L > 1) {
            const int b = t + Sh::T * i;
            const int k = b & (L - 1);
            apply_stage_twiddles_at<R, L>(u, tw + stockham_tw_offset<LOGN, LOGE>(S), k);
        }
        Dft<R>::run(u);
#pragma unroll
        for (int q = 0; q < R; ++q) x[i + NB * q] = u[q];
    }
}

// Destination position of output (i, q) of stage S for thread t.
template <int LOGN, int LOGE, int S>
__device__ __forceinline__ int stockham_dst(int t, int i, int q) {
    using Sh = StockhamShape<LOGN, LOGE>;
    constexpr int LOGR = (S < Sh::NFULL) ? LOGE : Sh::REM;
    constexpr int R = 1 << LOGR;
    constexpr int L = 1 << (S * LOGE);
    const int b = t + Sh::T * i;
    const int j = b >> (S * LOGE);
    const int k = b & (L - 1);
    return j * L * R + k + q * L;
}

// LDS addresses as a per-thread base plus compile-time offsets, using
// lds_pos(a + K*c) = lds_pos(a) + (K+1)*c for K = 2^SH: the gather of position
// t + T*m and the scatter of output q of butterfly i then need no per-element
// index arithmetic (ds_read/ds_write take the offset as an immediate).
template <int LOGN, int LOGE, int SH = 4>
__device__ __forceinline__ void lds_gather(float2* x, const float2* __restrict__ lds, int t) {
    using Sh = StockhamShape<LOGN, LOGE>;
    constexpr int K = 1 << SH;
    if constexpr (Sh::T % K == 0) {
        const float2* base = lds + lds_pos<SH>(t);
#pragma unroll
        for (int m = 0; m < Sh::E; ++m) x[m] = base[m * (Sh::T + Sh::T / K)];
    } else {
#pragma unroll
        for (int m = 0; m < Sh::E; ++m) x[m] = lds[lds_pos<SH>(t + Sh::T * m)];
    }
}

template <int LOGN, int LOGE, int S, int SH = 4>
__device__ __forceinline__ void lds_scatter(const float2* x, float2* __restrict__ lds, int t) {
    using Sh = StockhamShape<LOGN, LOGE>;
    constexpr int LOGR = (S < Sh::NFULL) ? LOGE : Sh::REM;
    constexpr int NB = Sh::E >> LOGR;
    constexpr int R = 1 << LOGR;
    constexpr int L = 1 << (S * LOGE);
    constexpr int K = 1 << SH;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if constexpr (L == 1 && R == K) {
            // dst = K*b + q, q < K  ->  lds_pos = (K+1)*b + q
            float2* base = lds + (K + 1) * (t + Sh::T * i);
#pragma unroll
            for (int q = 0; q < R; ++q) base[q] = x[i + NB * q];
        } else if constexpr (L % K == 0) {
            // dst = (j*L*R + k) + q*L with L a multiple of K
            float2* base = lds + lds_pos<SH>(stockham_dst<LOGN, LOGE, S>(t, i, 0));
#pragma unroll
            for (int q = 0; q < R; ++q) base[q * (L + L / K)] = x[i + NB * q];
        } else {
#pragma unroll
            for (int q = 0; q < R; ++q) lds[lds_pos<SH>(stockham_dst<LOGN, LOGE, S>(t, i, q))] = x[i + NB * q];
        }
    }
}

// SH: the exchanges' padding (lds_pos<SH>); the exchange buffer holds
// N + N/2^SH positions.
template <int LOGN, int LOGE, int S, int SH = 4>
struct StockhamStages {
    using Sh = StockhamShape<LOGN, LOGE>;
    // Runs stage S (already gathered in x) and every later stage.
    template <bool ONE_WAVE>
    __device__ __forceinline__ static void run(float2* x, int t, const float2* __restrict__ tw,
                                               float2* __restrict__ lds) {
        stockham_stage_regs<LOGN, LOGE, S>(x, t, tw);
        if constexpr (S + 1 < Sh::NSTAGES) {
            lds_scatter<LOGN, LOGE, S, SH>(x, lds, t);
            if constexpr (ONE_WAVE) wave_sync(); else __syncthreads();
            lds_gather<LOGN, LOGE, SH>(x, lds, t);
            if constexpr (S + 2 < Sh::NSTAGES) {
                if constexpr (ONE_WAVE) wave_sync(); else __syncthreads();
            }
            StockhamStages<LOGN, LOGE, S + 1, SH>::template run<ONE_WAVE>(x, t, tw, lds);
        }
    }
};

// Kernel body: FPB transforms per workgroup of FPB*T threads; IO is the global
// layout (InterleavedIO or SplitIO).  flags take FG_PASS_CONJ_IN /
// FG_PASS_CONJ_SCALE_OUT (tile_geom.h): the inverse is both.
template <int LOGN, int LOGE, int FPB, class IO>
__device__ __forceinline__ void fft_stockham_body(const IO io, const float2* __restrict__ tw,
                                                  uint64_t batch, float scale, uint32_t flags) {
    using Sh = StockhamShape<LOGN, LOGE>;
    constexpr int BLOCK = FPB * Sh::T;
    // Whole workgroup in one wave: its block-wide LDS staging needs only
    // wave-scope ordering.
    constexpr bool ONE_WAVE = BLOCK <= 64;
    // Each transform's T threads lie in one wave (T <= 64 divides the 64
    // lanes), so its stage exchanges need only wave-scope ordering, however
    // many transforms the workgroup holds.
    constexpr bool WAVE_LOCAL = Sh::T <= 64;
    // With fewer than 8 threads per transform a thread's positions t + T*m
    // give each wave only T*8-byte pieces per load; such sizes move the
    // workgroup's FPB contiguous transforms through LDS instead, 64 lanes x 8
    // contiguous bytes per instruction.
    constexpr bool STAGED = Sh::T < 8 && FPB > 1;  // measured: N = 128 (T = 8) is faster direct
    __shared__ float2 lds_all[FPB][Sh::LDS_ELEMS];
    const int tid = threadIdx.x;
    const int slot = tid / Sh::T;
    const int t = tid - slot * Sh::T;
    const uint64_t f0 = (uint64_t)blockIdx.x * FPB;
    const uint64_t f = f0 + slot;
    const bool valid = f < batch;
    const bool cs = (flags & FG_PASS_CONJ_SCALE_OUT) != 0;

    float2 x[Sh::E];
    if constexpr (STAGED) {
#pragma unroll
        for (int j = 0; j < Sh::E; ++j) {
            const int e = tid + BLOCK * j;  // element of the block's FPB*N
            const int fs = e >> LOGN;
            float2 v = make_float2(0.f, 0.f);
            if (f0 + fs < batch) v = io.load(f0 * Sh::N + e);
            lds_all[fs][lds_pos<>(e & (Sh::N - 1))] = v;
        }
        if constexpr (ONE_WAVE) wave_sync(); else __syncthreads();
#pragma unroll
        for (int m = 0; m < Sh::E; ++m) x[m] = lds_all[slot][lds_pos<>(t + Sh::T * m)];
        if constexpr (ONE_WAVE) wave_sync(); else __syncthreads();
    } else if (valid) {
#pragma unroll
        for (int m = 0; m < Sh::E; ++m) x[m] = io.load(f * Sh::N + t + Sh::T * m);
    } else {
#pragma unroll
        for (int m = 0; m < Sh::E; ++m) x[m] = make_float2(0.f, 0.f);
    }
    if (flags & FG_PASS_CONJ_IN) {
#pragma unroll
        for (int m = 0; m < Sh::E; ++m) x[m] = cconj(x[m]);
    }
    StockhamStages<LOGN, LOGE, 0>::template run<WAVE_LOCAL>(x, t, tw, lds_all[slot]);
    if constexpr (STAGED) {
        if constexpr (ONE_WAVE) wave_sync(); else __syncthreads();
#pragma unroll
        for (int m = 0; m < Sh::E; ++m) {
            float2 v = x[m];
            if (cs) v = cscale(cconj(v), scale);
            lds_all[slot][lds_pos<>(t + Sh::T * m)] = v;
        }
        if constexpr (ONE_WAVE) wave_sync(); else __syncthreads();
#pragma unroll
        for (int j = 0; j < Sh::E; ++j) {
            const int e = tid + BLOCK * j;
            const int fs = e >> LOGN;
            if (f0 + fs < batch) io.store(f0 * Sh::N + e, lds_all[fs][lds_pos<>(e & (Sh::N - 1))]);
        }
    } else if (valid) {
#pragma unroll
        for (int m = 0; m < Sh::E; ++m) {
            float2 v = x[m];
            if (cs) v = cscale(cconj(v), scale);
            io.store(f * Sh::N + t + Sh::T * m, v);
        }
    }
}

// ---------------------------------------------------------------------------
// 32 elements per thread, exchanges in halves.  T = L/32 threads hold 32
// elements each (positions t + T*m) and run NB = 32/R butterflies
// b = t + T*i of every stage of the radix list (16, ..., 16, r).  Butterfly b
// of stage s writes to j*L_s*R + k + q*L_s (j = b / L_s, k = b % L_s), below
// L/2 exactly when i < NB/2 (b < T), so every exchange can run in two rounds
// through LDS holding L/2 positions: round h writes butterflies
// i in [h*NB/2, (h+1)*NB/2), then each thread reads its elements
// m in [16h, 16h + 16).  The last stage's outputs are the thread's own
// positions t + T*m.  Used by the first pass of 1D multi-pass plans
// (fft_tile.hpp, G columns per workgroup) and by the single-pass 8192- to
// 32768-point transforms (fft_row_halves_body below): half the LDS of the
// 16-element layout, so twice the workgroups per CU (32768 points: the one
// layout that fits a CU at all).
template <int LOGL>
struct HalvesShape {
    static constexpr int N = 1 << LOGL, E = 32, T = N / E, HALF = N / 2;
    static constexpr int NFULL = LOGL / 4, REM = LOGL % 4;
    static constexpr int NSTAGES = NFULL + (REM ? 1 : 0);
    static_assert(LOGL >= 7 && LOGL <= 15, "half exchanges: 128 .. 4096-point tile columns, 8192 .. 32768-point rows");
};

template <int LOGL, int S>
struct HalvesStage {
    static constexpr int LOGR = (S < HalvesShape<LOGL>::NFULL) ? 4 : HalvesShape<LOGL>::REM;
    static constexpr int R = 1 << LOGR;
    static constexpr int NB = HalvesShape<LOGL>::E / R;  // butterflies per thread
    static constexpr int L = 1 << (4 * S);              // product of the earlier radices
};

// Stage S: y[i + NB*q] = output q of butterfly i (inputs x[i + NB*p]).  The
// twiddles come from the table of the radix list (16, ..., 16, r), the one
// the 16-element geometry uses.
template <int LOGL, int S>
__device__ __forceinline__ void halves_stage(const float2* x, float2* y, int t, const float2* __restrict__ tw) {
    using H = HalvesShape<LOGL>;
    using St = HalvesStage<LOGL, S>;
#pragma unroll
    for (int i = 0; i < St::NB; ++i) {
        float2 u[St::R];
#pragma unroll
        for (int p = 0; p < St::R; ++p) u[p] = x[i + St::NB * p];
        if constexpr (St::L > 1) {
            const int k = (t + H::T * i) & (St::L - 1);
            apply_stage_twiddles_at<St::R, St::L>(u, tw + stockham_tw_offset<LOGL, 4>(S), k);
        }
        Dft<St::R>::run(u);
#pragma unroll
        for (int q = 0; q < St::R; ++q) y[i + St::NB * q] = u[q];
    }
}

// Exchange after stage S of one contiguous transform: x[m] = the element at
// position t + T*m.  The LDS holds L/2 positions, one pad slot per 16
// (lds_pos): lds_pos(d + q*L_s) = lds_pos(d) + q*(L_s + L_s/16) for L_s a
// multiple of 16, and at stage 0 (L_s = 1) butterfly b writes 16b + q, slot
// 17b + q.
template <int LOGN, int S>
__device__ __forceinline__ void row_halves_exchange(const float2* y, float2* x, int t, float2* __restrict__ lds) {
    using H = HalvesShape<LOGN>;
    using St = HalvesStage<LOGN, S>;
    static_assert(St::R == 16 && H::T % 16 == 0, "exchanges follow radix-16 stages");
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (S > 0 || h > 0) __syncthreads();  // the previous round's readers are done
#pragma unroll
        for (int ii = 0; ii < St::NB / 2; ++ii) {
            const int i = h * (St::NB / 2) + ii;
            const int b = t + H::T * i;
            float2* base;
            if constexpr (St::L == 1) {
                base = lds + 17 * (b - (H::HALF / 16) * h);
#pragma unroll
                for (int q = 0; q < 16; ++q) base[q] = y[i + St::NB * q];
            } else {
                const int d0 = (b >> (4 * S)) * St::L * 16 + (b & (St::L - 1)) - H::HALF * h;
                base = lds + lds_pos<>(d0);
#pragma unroll
                for (int q = 0; q < 16; ++q) base[q * (St::L + St::L / 16)] = y[i + St::NB * q];
            }
        }
        __syncthreads();
        const float2* rbase = lds + lds_pos<>(t);
#pragma unroll
        for (int m = 0; m < H::E / 2; ++m) x[(H::E / 2) * h + m] = rbase[m * (H::T + H::T / 16)];
    }
}

template <int LOGN, int S>
struct RowHalvesStages {
    __device__ __forceinline__ static void run(float2* x, float2* y, int t, const float2* __restrict__ tw,
                                               float2* __restrict__ lds) {
        halves_stage<LOGN, S>(x, y, t, tw);
        if constexpr (S + 1 < HalvesShape<LOGN>::NSTAGES) {
            row_halves_exchange<LOGN, S>(y, x, t, lds);
            RowHalvesStages<LOGN, S + 1>::run(x, y, t, tw, lds);
        }
    }
};

// One transform of N = 2^LOGN (8192, 16384 or 32768) points per workgroup of
// N/32 threads, 32 elements per thread, LDS of N/2 + N/32 positions (68 KB at
// 16384: two workgroups per CU where the 16-element layout's 136 KB allows
// one; 136 KB and 1024 threads at 32768).  IO and flags as
// fft_stockham_body; the stage table is the radix list (16, 16, 16, r) of
// the 16-element layout.
template <int LOGN, class IO>
__device__ __forceinline__ void fft_row_halves_body(const IO io, const float2* __restrict__ tw, uint64_t batch,
                                                    float scale, uint32_t flags) {
    using H = HalvesShape<LOGN>;
    __shared__ float2 lds[H::HALF + H::HALF / 16];
    const int t = threadIdx.x;
    const uint64_t f = blockIdx.x;
    if (f >= batch) return;  // uniform over the workgroup (the host launches batch of them)
    stagger_lockstep_start<(H::HALF + H::HALF / 16) * 8, H::T>();  // 16384 / 32768 points
    float2 x[H::E], y[H::E];
#pragma unroll
    for (int m = 0; m < H::E; ++m) x[m] = io.load_row(f * H::N + H::T * m, t);
    if (flags & FG_PASS_CONJ_IN) {
#pragma unroll
        for (int m = 0; m < H::E; ++m) x[m] = cconj(x[m]);
    }
    RowHalvesStages<LOGN, 0>::run(x, y, t, tw, lds);
    const bool cs = (flags & FG_PASS_CONJ_SCALE_OUT) != 0;
#pragma unroll
    for (int m = 0; m < H::E; ++m) {
        float2 v = y[m];
        if (cs) v = cscale(cconj(v), scale);
        io.store_row(f * H::N + H::T * m, t, v);
    }
}

// ---------------------------------------------------------------------------
// N = 1024, two transforms per 128-thread workgroup, radix list 8 * 16 * 8.
// Thread t (0..127) loads element t + 128 m of the workgroup's 2048 (m < 16:
// transform m / 8, position t + 128 (m % 8)), so each pair of load
// instructions of the two waves covers 1 KB of contiguous memory -- a copy
// probe of this shape moved 512 MiB in 168.6 us against 174.1 us for one
// 8 KB transform per wave.  The layout fits the Stockham recurrence
// (gather b + p N/R, twiddle W_{L R}^{p k}, scatter j L R + k + q L):
//   stage 0, R = 8, L = 1: butterfly b = t of each transform, positions
//            t + 128 p, no twiddles; outputs to 8 t + q;
//   stage 1, R = 16, L = 8: thread t takes butterfly t % 64 of transform
//            t / 64 (positions b + 64 p), twiddles W_128^{p (b % 8)};
//   stage 2, R = 8, L = 128: butterfly b = t of each transform (positions
//            t + 128 p), twiddles W_1024^{p t}; outputs to t + 128 q, so the
//            stores are the same 1 KB rows.
// Stage table (fft1024_x2_twiddles on the host): stage 1 rows k < 8 of
// W_128^{p k}, p in {1, 2, 3, 4, 8, 12}; stage 2 rows k < 128 of
// W_1024^{p k}, p in {1, 2, 3, 4} from entry 48 (apply_stage_twiddles forms
// the other exponents).  The exchanges cross the two waves (__syncthreads).
template <class IO>
__device__ __forceinline__ void fft1024_x2_body(const IO io, const float2* __restrict__ tw, uint64_t batch,
                                                float scale, uint32_t flags) {
    __shared__ float2 lds[2][1024 + 64];
    const int t = threadIdx.x;
    const uint64_t f0 = (uint64_t)blockIdx.x * 2;
    const bool has1 = f0 + 1 < batch;  // the last workgroup may hold one transform
    float2 x[16];
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int p = 0; p < 8; ++p)
            x[8 * f + p] = (f == 0 || has1) ? io.load((f0 + f) * 1024 + t + 128 * p) : make_float2(0.f, 0.f);
    if (flags & FG_PASS_CONJ_IN) {
#pragma unroll
        for (int m = 0; m < 16; ++m) x[m] = cconj(x[m]);
    }
#pragma unroll
    for (int f = 0; f < 2; ++f) {
        Dft<8>::run(x + 8 * f);
#pragma unroll
        for (int q = 0; q < 8; ++q) lds[f][lds_pos<>(8 * t + q)] = x[8 * f + q];
    }
    __syncthreads();
    {
        const int g = t >> 6, b = t & 63, k = b & 7;
        // lds_pos(b + 64 m) = lds_pos(b) + 68 m
        const float2* src = &lds[g][0] + lds_pos<>(b);
#pragma unroll
        for (int m = 0; m < 16; ++m) x[m] = src[68 * m];
        __syncthreads();  // every stage-1 read done before the scatter below
        apply_stage_twiddles<16>(x, tw + 6 * k);
        Dft<16>::run(x);
        // d0 = (b / 8) * 128 + k with d0 % 16 = k < 8: lds_pos(d0 + 8 q) = lds_pos(d0) + 8 q + q / 2
        float2* dst = &lds[g][0] + lds_pos<>((b >> 3) * 128 + k);
#pragma unroll
        for (int q = 0; q < 16; ++q) dst[8 * q + (q >> 1)] = x[q];
    }
    __syncthreads();
    const bool cs = (flags & FG_PASS_CONJ_SCALE_OUT) != 0;
#pragma unroll
    for (int f = 0; f < 2; ++f) {
        // lds_pos(t + 128 p) = lds_pos(t) + 136 p
        const float2* src = &lds[f][0] + lds_pos<>(t);
        float2 u[8];
#pragma unroll
        for (int p = 0; p < 8; ++p) u[p] = src[136 * p];
        apply_stage_twiddles<8>(u, tw + 48 + 4 * t);
        Dft<8>::run(u);
        if (f == 0 || has1) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                float2 v = u[q];
                if (cs) v = cscale(cconj(v), scale);
                io.store((f0 + f) * 1024 + t + 128 * q, v);
            }
        }
    }
}

}  // namespace fg

// fft_2d_halves.hpp -- the whole 2D FFT of one image of R x C = 2^LR x 2^LC =
// 2048 to 16384 points per workgroup, in registers, with the exchanges in
// halves.
//
// Holding such an image in LDS (fft_2d_small.hpp) takes up to 141 KB (one
// workgroup per CU at 16384 points, two at 8192, four at 4096), and the
// workgroups' load, transform and store phases then barely overlap.  Here
// T = N/32 threads (64 .. 512) hold 32 elements each at positions t + T*m of
// the row-major image (coalesced loads), and the exchanges run in two rounds
// through N/2 + N/32 LDS slots (8.5 .. 68 KB), as in the single-pass 1D
// kernels of 8192 points and up (fft_row_halves_body).  Below 2048 points
// (T < 64: part of a wave per image) the LDS-resident kernel measured as fast
// or faster.
//
// The 2D DFT is one Stockham pass over all N positions whose radix list is
// R's list (16, .., 16, r) followed by C's:
//   * the first block takes the DFT over the row index (a position's top LR
//     bits), with the 1D stage twiddles W_{L R_s}^{p k} of length R;
//   * the second block takes the DFT over the column index with no twiddle
//     between the blocks: stage twiddles W_{Ld R_s}^{p (k >> LR)} of length C
//     (Ld: the product of the block's earlier radices), since k = k_r + R k'
//     there and k_r only indexes the transformed rows;
//   * the autosort leaves output (k_r, k_c) at position k_r + R k_c, and a
//     last exchange moves it to k_r C + k_c, so the stores are the loads'
//     coalesced rows.
// Butterfly b of a stage before the last writes to j L R_s + k + q L, inside
// [j L R_s, (j + 1) L R_s) with L R_s <= N/2, so butterflies i < NB/2 of every
// thread (b = t + T i) write the lower half and each exchange is two rounds:
// round h writes half h, then every thread reads its elements m in
// [16h, 16h + 16).  In the last exchange output m of thread t goes to round
// (k_r >= R/2) with k_r = (t + T m) mod R.  tests/test_fft2d_halves_model.py
// replays this bookkeeping against the oracle.
#pragma once
#include "fft_stockham.hpp"

namespace fg {

template <int LR, int LC>
struct Halves2D {
    static constexpr int N = 1 << (LR + LC), E = 32, T = N / E, HALF = N / 2;
    static constexpr int NR = 1 << LR, NC = 1 << LC;
    static constexpr int SR = LR / 4 + (LR % 4 ? 1 : 0);  // stages over the row index
    static constexpr int SC = LC / 4 + (LC % 4 ? 1 : 0);  // stages over the column index
    static constexpr int NSTAGES = SR + SC;
    static_assert(LR + LC >= 11 && LR + LC <= 14 && LR >= 4 && LC >= 4,
                  "2048- to 16384-point images, at least 16 per side");
    static_assert(T % 16 == 0, "reads at lds_pos(t) + m (T + T/16)");
};

template <int LR, int LC, int S>
struct Halves2DStage {
    using H = Halves2D<LR, LC>;
    static constexpr bool ROWIDX = S < H::SR;              // DFT over the row index
    static constexpr int BITS = ROWIDX ? LR : LC;
    static constexpr int SD = ROWIDX ? S : S - H::SR;      // stage within its block
    static constexpr int LOGR = SD < BITS / 4 ? 4 : BITS % 4;
    static constexpr int R = 1 << LOGR;
    static constexpr int NB = H::E / R;                   // butterflies per thread
    static constexpr int LOGLD = 4 * SD;
    static constexpr int LD = 1 << LOGLD;                 // the block's earlier radices
    static constexpr int LOGL = ROWIDX ? LOGLD : LR + LOGLD;
    static constexpr int L = 1 << LOGL;                   // every earlier radix
    static_assert(L == 1 || L % 16 == 0, "scatter offsets q (L + L/16)");
};

// Stage S: y[i + NB q] = output q of butterfly i (inputs x[i + NB p]).
// tw_r / tw_c: the stage tables of the radix lists for lengths R and C.
template <int LR, int LC, int S>
__device__ __forceinline__ void halves2d_stage(const float2* x, float2* y, int t, const float2* __restrict__ tw_r,
                                               const float2* __restrict__ tw_c) {
    using H = Halves2D<LR, LC>;
    using St = Halves2DStage<LR, LC, S>;
#pragma unroll
    for (int i = 0; i < St::NB; ++i) {
        float2 u[St::R];
#pragma unroll
        for (int p = 0; p < St::R; ++p) u[p] = x[i + St::NB * p];
        if constexpr (St::LD > 1) {
            const int k = (t + H::T * i) & (St::L - 1);
            if constexpr (St::ROWIDX)
                apply_stage_twiddles_at<St::R, St::LD>(u, tw_r + stockham_tw_offset<LR, 4>(St::SD), k);
            else
                apply_stage_twiddles_at<St::R, St::LD>(u, tw_c + stockham_tw_offset<LC, 4>(St::SD), k >> LR);
        }
        Dft<St::R>::run(u);
#pragma unroll
        for (int q = 0; q < St::R; ++q) y[i + St::NB * q] = u[q];
    }
}

// Exchange after stage S (not the last): x[m] = the element at position t + T m.
template <int LR, int LC, int S>
__device__ __forceinline__ void halves2d_exchange(const float2* y, float2* x, int t, float2* __restrict__ lds) {
    using H = Halves2D<LR, LC>;
    using St = Halves2DStage<LR, LC, S>;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (S > 0 || h > 0) __syncthreads();  // the previous round's readers are done
#pragma unroll
        for (int ii = 0; ii < St::NB / 2; ++ii) {
            const int i = h * (St::NB / 2) + ii;
            const int b = t + H::T * i;
            const int d0 = (b >> St::LOGL) * St::L * St::R + (b & (St::L - 1)) - H::HALF * h;
            float2* base = lds + lds_pos<>(d0);
            if constexpr (St::L == 1) {
                // d0 = R b - HALF h with R <= 16 dividing 16: lds_pos(d0 + q) = lds_pos(d0) + q
#pragma unroll
                for (int q = 0; q < St::R; ++q) base[q] = y[i + St::NB * q];
            } else {
#pragma unroll
                for (int q = 0; q < St::R; ++q) base[q * (St::L + St::L / 16)] = y[i + St::NB * q];
            }
        }
        __syncthreads();
        const float2* rbase = lds + lds_pos<>(t);
#pragma unroll
        for (int m = 0; m < H::E / 2; ++m) x[(H::E / 2) * h + m] = rbase[m * (H::T + H::T / 16)];
    }
}

// The last exchange: output m of thread t (position P = t + T m holds
// (k_r, k_c) = (P mod R, P / R)) moves to Q = k_r C + k_c; x[m] = the element
// at t + T m of the row-major output.  Its LDS slots take one pad per output
// row, tpos(Q) = Q + Q / C: the writes of a wave run down a column (lanes
// k_r, k_r + 1, ..: stride C + 1, odd, so no two lanes of a 16-lane group
// share a bank), where the 1-in-16 padding of the other exchanges would put
// every lane on one of four banks.  C + 1 slots per row of C: at most
// N/2 + N/32 for C >= 16.
template <int LR, int LC>
__device__ __forceinline__ void halves2d_transpose(const float2* y, float2* x, int t, float2* __restrict__ lds) {
    using H = Halves2D<LR, LC>;
    static_assert(H::HALF + H::HALF / H::NC <= H::HALF + H::HALF / 16, "the transpose's slots fit the exchange buffer");
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        __syncthreads();  // the previous exchange's (round's) readers are done
        if constexpr (H::NR <= H::T) {
            // k_r = t mod R for all 32 outputs (T is a multiple of R), so the
            // thread writes in one round: k_c = t / R + (T / R) m, and
            // (t / R) + (T / R) m < C keeps the pad term at q0 / C
            const int kr = t & (H::NR - 1);
            if ((kr >= H::NR / 2) == (h == 1)) {
                const int q0 = kr * H::NC + (t >> LR) - H::HALF * h;
                float2* base = lds + q0 + q0 / H::NC;
#pragma unroll
                for (int m = 0; m < H::E; ++m) base[(H::T / H::NR) * m] = y[m];
            }
        } else {
            // R = 2T: k_r = t + T (m mod 2), k_c = m / 2; round h takes the m
            // with m mod 2 = h, at slots 17 t + m / 2 (C = 16)
            static_assert(H::NR == 2 * H::T, "R <= T or R = 2T");
            float2* base = lds + t * (H::NC + 1);
#pragma unroll
            for (int m = h; m < H::E; m += 2) base[m >> 1] = y[m];
        }
        __syncthreads();
        // reads of t + T m - HALF h, m in [0, 16): tpos = t + t / C + m (T + T / C)
        // for C <= T; otherwise C = 2T (R = 16): t + T m + m / 2
#pragma unroll
        for (int m = 0; m < H::E / 2; ++m) {
            int slot;
            if constexpr (H::NC <= H::T)
                slot = t + t / H::NC + m * (H::T + H::T / H::NC);
            else
                slot = t + H::T * m + m / 2;
            x[(H::E / 2) * h + m] = lds[slot];
        }
    }
}

template <int LR, int LC, int S>
struct Halves2DStages {
    __device__ __forceinline__ static void run(float2* x, float2* y, int t, const float2* __restrict__ tw_r,
                                               const float2* __restrict__ tw_c, float2* __restrict__ lds) {
        halves2d_stage<LR, LC, S>(x, y, t, tw_r, tw_c);
        if constexpr (S + 1 < Halves2D<LR, LC>::NSTAGES) {
            halves2d_exchange<LR, LC, S>(y, x, t, lds);
            Halves2DStages<LR, LC, S + 1>::run(x, y, t, tw_r, tw_c, lds);
        }
    }
};

// One 2^LR x 2^LC image per workgroup of N/32 threads.  tw_rows / tw_cols are
// the stage tables for lengths C and R (the host's small-2D tables); IO and
// flags as fft_stockham_body.
template <int LR, int LC, class IO>
__device__ __forceinline__ void fft2d_halves_body(const IO io, const float2* __restrict__ tw_rows,
                                                  const float2* __restrict__ tw_cols, uint64_t batch, float scale,
                                                  uint32_t flags) {
    using H = Halves2D<LR, LC>;
    __shared__ float2 lds[H::HALF + H::HALF / 16];
    const int t = threadIdx.x;
    const uint64_t f = blockIdx.x;
    // f is uniform over the workgroup (the host launches batch of them, N/32
    // threads each); threads beyond N/32 in a larger block would only idle
    if (f >= batch || t >= H::T) return;
    stagger_lockstep_start<(H::HALF + H::HALF / 16) * 8, H::T>();  // 16384-point images
    float2 x[H::E], y[H::E];
#pragma unroll
    for (int m = 0; m < H::E; ++m) x[m] = io.load_row(f * H::N + H::T * m, t);
    if (flags & FG_PASS_CONJ_IN) {
#pragma unroll
        for (int m = 0; m < H::E; ++m) x[m] = cconj(x[m]);
    }
    Halves2DStages<LR, LC, 0>::run(x, y, t, tw_cols, tw_rows, lds);
    halves2d_transpose<LR, LC>(y, x, t, lds);
    const bool cs = (flags & FG_PASS_CONJ_SCALE_OUT) != 0;
#pragma unroll
    for (int m = 0; m < H::E; ++m) {
        float2 v = x[m];
        if (cs) v = cscale(cconj(v), scale);
        io.store_row(f * H::N + H::T * m, t, v);
    }
}

}  // namespace fg

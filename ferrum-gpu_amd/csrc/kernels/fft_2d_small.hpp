// fft_2d_small.hpp -- the whole 2D FFT of images of R x C <= 1024 points in
// one pass through HBM: a row pass and a column pass would each move every
// byte once; here a workgroup loads FPI whole images into LDS, transforms
// their rows and then their columns there, and stores them.  E = 8 elements
// per thread (the template also takes 16).  Images of 2048 points and more
// run fft_2d_halves.hpp: held in LDS they left few workgroups per CU.
//
// Per image the LDS holds R rows of pitch P (the shape's Small2DLayout):
//   1. coalesced load of the workgroup's images (64 lanes x 8 contiguous bytes
//      per instruction), element (r, c) at r*P + c;
//   2. rows: thread (r, t), t < C/E, takes positions t + (C/E)*m of row r and
//      runs the Stockham stages of length C (fft_stockham.hpp), exchanging in
//      its own row's P slots (padded positions, C + C/2^shr <= P); its outputs
//      go back to r*P + k;
//   3. columns: thread (c, t), t < R/E, takes rows t + (R/E)*m of column c;
//      once every column is read, the image's memory holds the column
//      exchanges (column c at c*CP, C*CP <= R*P) for the Stockham stages of
//      length R; the outputs go back to k*P + c;
//   4. coalesced store.
// A row's (a column's) threads lie in one wave, so their
// exchanges need only wave-scope ordering; the phases are separated by
// workgroup barriers.  Stage twiddles: the tables of the radix lists
// (E, ..., E, r) for lengths C and R.  Inverse: conjugate on load, conjugate
// and scale on store.
#pragma once
#include "fft_stockham.hpp"

namespace fg {

// LDS layout of one shape: row pitch P = C + C/2^shr + dp, column-exchange
// stride CP = R + R/2^shc + dc, the row (column) exchanges padded one slot per
// 2^shr (2^shc) positions, and which lanes of a wave take a row's (column's)
// threads: consecutive lanes (line-major) or every (64/T)-th lane
// (thread-major).  Chosen per shape so that the 16 lanes that share an LDS
// cycle of a 64-bit access hit distinct banks in every phase (a CPU model of
// 32 four-byte banks, which reproduces the conflict rates rocprof measured on
// the first layout, the default below; tests/test_fft2d_small_banks.py).
struct Small2DLayout {
    int dp, dc, shr, shc;
    bool row_tm, col_tm;
};

__host__ __device__ constexpr Small2DLayout small2d_layout(int lr, int lc) {
    switch (lr * 16 + lc) {
        // modelled conflict cycles per access cycle: first layout -> this one
        case 4 * 16 + 4: return {0, 0, 4, 4, true, true};  // 0.40 -> 0.00
        case 4 * 16 + 5: return {1, 0, 4, 4, true, true};  // 0.70 -> 0.00
        case 4 * 16 + 6: return {2, 0, 4, 4, true, true};  // 0.70 -> 0.10
        case 4 * 16 + 7: return {0, 0, 4, 4, false, true};  // 0.33 -> 0.08
        case 4 * 16 + 8: return {8, 0, 3, 3, true, false};  // 0.33 -> 0.00
        case 4 * 16 + 9: return {0, 0, 4, 4, false, true};  // 0.33 -> 0.08
        case 5 * 16 + 4: return {0, 1, 3, 4, false, true};  // 0.40 -> 0.00
        case 5 * 16 + 5: return {1, 1, 4, 4, true, true};  // 0.70 -> 0.00
        case 5 * 16 + 6: return {2, 1, 4, 4, true, true};  // 0.70 -> 0.10
        case 5 * 16 + 7: return {4, 0, 3, 3, true, false};  // 0.33 -> 0.00
        case 5 * 16 + 8: return {8, 1, 3, 3, true, true};  // 0.67 -> 0.00
        case 5 * 16 + 9: return {8, 0, 4, 4, false, false};  // 0.17 -> 0.00
        case 6 * 16 + 4: return {0, 0, 3, 3, false, false};  // 0.20 -> 0.00
        case 6 * 16 + 5: return {1, 0, 4, 4, true, false};  // 0.70 -> 0.30
        case 6 * 16 + 6: return {2, 0, 3, 3, true, false};  // 0.70 -> 0.00
        case 6 * 16 + 7: return {10, 0, 4, 3, false, false};  // 0.33 -> 0.08
        case 6 * 16 + 8: return {4, 0, 4, 4, false, false};  // 0.60 -> 0.00
        case 7 * 16 + 4: return {0, 0, 4, 4, true, false};  // 0.33 -> 0.08
        case 7 * 16 + 5: return {1, 0, 4, 4, true, false};  // 0.42 -> 0.08
        case 7 * 16 + 6: return {2, 4, 3, 3, true, true};  // 0.42 -> 0.17
        case 7 * 16 + 7: return {2, 0, 4, 4, true, false};  // 0.60 -> 0.00
        case 8 * 16 + 4: return {0, 0, 4, 4, true, false};  // 0.33 -> 0.08
        case 8 * 16 + 5: return {1, 0, 4, 4, true, false};  // 0.42 -> 0.08
        case 8 * 16 + 6: return {1, 0, 4, 4, true, false};  // 0.40 -> 0.00
        case 9 * 16 + 4: return {0, 0, 4, 4, true, false};  // 0.33 -> 0.08
        case 9 * 16 + 5: return {1, 0, 4, 4, true, false};  // 0.33 -> 0.00
        case 10 * 16 + 4: return {0, 0, 4, 4, false, false};  // 0.40 -> 0.00
        default: return {1, 0, 4, 4, false, false};
    }
}

template <int LR, int LC, int LOGE, int FPI>
struct Small2D {
    static constexpr Small2DLayout LAY = small2d_layout(LR, LC);
    static constexpr int R = 1 << LR, C = 1 << LC, N = R * C, E = 1 << LOGE;
    static constexpr int TC = C / E;                 // threads per row
    static constexpr int TR = R / E;                 // threads per column
    static constexpr int TIMG = N / E;               // threads per image
    static constexpr int BLOCK = FPI * TIMG;
    static constexpr int SHR = LAY.shr, SHC = LAY.shc;
    static constexpr int P = C + (C >> SHR) + LAY.dp;   // LDS row pitch
    static constexpr int CP = R + (R >> SHC) + LAY.dc;  // column exchange stride
    static constexpr int IMG = R * P;                   // LDS elements per image
    static constexpr int K = TIMG < 64 ? TIMG : 64;     // threads of one wave's part of an image
    static_assert(LOGE <= LR && LOGE <= LC, "at least E points per row and column");
    static_assert(LAY.dp >= 0 && LAY.dc >= 0, "the exchange regions hold the padded lines");
    static_assert(C * CP <= IMG, "the column exchange regions fit the image's LDS");
    static_assert(TC <= 64 && TR <= 64 && 64 % TC == 0 && 64 % TR == 0, "a row's / column's threads lie in one wave");
    static_assert(BLOCK <= 1024 && BLOCK % 64 == 0, "whole waves, at most 1024 threads");
    static_assert(LOGE == FG_SMALL2D_LOGE(LR, LC) && BLOCK == FG_SMALL2D_BLOCK(LR, LC), "the host's launch geometry");
    static_assert(FPI * IMG * 8 <= 160 * 1024, "the workgroup's images fit the LDS");
};

template <int LR, int LC, int LOGE, int FPI, class IO>
__device__ __forceinline__ void fft2d_small_body(const IO io, const float2* __restrict__ tw_rows,
                                                 const float2* __restrict__ tw_cols, uint64_t batch, float scale,
                                                 uint32_t flags) {
    using S = Small2D<LR, LC, LOGE, FPI>;
    __shared__ float2 lds[FPI * S::IMG];
    const int tid = threadIdx.x;
    const int slot = tid / S::TIMG;
    const int local = tid - slot * S::TIMG;
    const uint64_t i0 = (uint64_t)blockIdx.x * FPI;
    float2* img = lds + slot * S::IMG;
    const bool cin = (flags & FG_PASS_CONJ_IN) != 0;
    const bool cs = (flags & FG_PASS_CONJ_SCALE_OUT) != 0;

    // 1. Load: element e of the block's FPI*N -> image e / N, (row, col) of e % N.
#pragma unroll
    for (int j = 0; j < S::E; ++j) {
        const int e = tid + S::BLOCK * j;
        const int is = e >> (LR + LC);
        const int n = e & (S::N - 1);
        float2 v = make_float2(0.f, 0.f);
        if (i0 + is < batch) v = io.load(i0 * S::N + e);
        if (cin) v = cconj(v);
        lds[is * S::IMG + (n >> LC) * S::P + (n & (S::C - 1))] = v;
    }
    __syncthreads();

    // 2. Rows.  Both lane orders keep a row's threads inside one wave.
    {
        const int part = local / S::K, l = local - part * S::K;
        constexpr int PER = S::K / S::TC;   // rows per wave part
        const int r = part * PER + (S::LAY.row_tm ? l % PER : l / S::TC);
        const int t = S::LAY.row_tm ? l / PER : l % S::TC;
        float2* row = img + r * S::P;
        float2 x[S::E];
#pragma unroll
        for (int m = 0; m < S::E; ++m) x[m] = row[t + S::TC * m];
        StockhamStages<LC, LOGE, 0, S::SHR>::template run<true>(x, t, tw_rows, row);
        wave_sync();  // the row's last exchange reads are done before the row is rewritten
#pragma unroll
        for (int m = 0; m < S::E; ++m) row[t + S::TC * m] = x[m];
    }
    __syncthreads();

    // 3. Columns.
    {
        const int part = local / S::K, l = local - part * S::K;
        constexpr int PER = S::K / S::TR;   // columns per wave part
        const int c = part * PER + (S::LAY.col_tm ? l % PER : l / S::TR);
        const int t = S::LAY.col_tm ? l / PER : l % S::TR;
        float2 x[S::E];
#pragma unroll
        for (int m = 0; m < S::E; ++m) x[m] = img[(t + S::TR * m) * S::P + c];
        __syncthreads();  // every column read before the image's memory holds exchanges
        StockhamStages<LR, LOGE, 0, S::SHC>::template run<true>(x, t, tw_cols, img + c * S::CP);
        __syncthreads();  // every exchange done before the plain layout is rewritten
#pragma unroll
        for (int m = 0; m < S::E; ++m) img[(t + S::TR * m) * S::P + c] = x[m];
    }
    __syncthreads();

    // 4. Store.
#pragma unroll
    for (int j = 0; j < S::E; ++j) {
        const int e = tid + S::BLOCK * j;
        const int is = e >> (LR + LC);
        const int n = e & (S::N - 1);
        if (i0 + is < batch) {
            float2 v = lds[is * S::IMG + (n >> LC) * S::P + (n & (S::C - 1))];
            if (cs) v = cscale(cconj(v), scale);
            io.store(i0 * S::N + e, v);
        }
    }
}

}  // namespace fg

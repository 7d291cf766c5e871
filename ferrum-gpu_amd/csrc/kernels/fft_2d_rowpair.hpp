// fft_2d_rowpair.hpp -- the row pass of a 2D FFT whose column DFT over R rows
// is split radix-2 over the row index (decimation in frequency):
//   X[2k]     = sum_{r < R/2} W_{R/2}^{r k} (A_r + B_r)
//   X[2k + 1] = sum_{r < R/2} W_{R/2}^{r k} (A_r - B_r) W_R^r
// with A_r, B_r the DFTs of rows r and r + R/2 (per column).  One workgroup
// takes that pair of rows, one row per half of its threads (a Stockham layout
// of fft_stockham.hpp, each half in its own LDS region), and stores A + B to
// output row 2r and (A - B) W_R^r to output row 2r + 1.  The
// column pass then takes R/2-point DFTs over the rows of each parity in place
// (element stride 2C), which leaves X[2k + h] at row 2k + h: an R/2-point
// column tile holds twice the columns of an R-point one in the same LDS, so
// the column pass of 4096-row images runs 2048-row tiles of 8 columns (two
// workgroups per CU where a 4096-row tile takes the CU's LDS) and those of
// 2048- / 1024-row images (1024 rows: of 2048 / 4096 columns) 1024- /
// 512-row tiles of 16 columns (whole 128-byte lines; four workgroups per CU
// at 512 rows).  Rows
// 2r, 2r + 1 are not the rows r, r + R/2 read, so the pass is out of place
// only.
#pragma once
#include "fft_stockham.hpp"

namespace fg {

// Half S of the workgroup holds row S of the pair, positions T m + t (E
// elements per thread, T threads per row).  It hands the positions the other
// half combines (m in [(1 - S) E/2, (2 - S) E/2)) to it through LDS region S.
template <int E, int T, int S>
__device__ __forceinline__ void rowpair_send(const float2* x, int t, float2* region) {
#pragma unroll
    for (int m = 0; m < E / 2; ++m) region[T * m + t] = x[(E / 2) * (1 - S) + m];
}

// ... and combines positions T m + t, m in [S E/2, (S + 1) E/2), with the
// other row's values from LDS region 1 - S.
template <int E, int T, int S, class IO>
__device__ __forceinline__ void rowpair_combine(const float2* x, int t, const float2* region, const IO& io,
                                                uint64_t row_out, uint64_t n, float2 w) {
#pragma unroll
    for (int m = 0; m < E / 2; ++m) {
        const float2 o = region[T * m + t];
        const float2 a = S == 0 ? x[m] : o;
        const float2 b = S == 0 ? o : x[E / 2 + m];
        const uint64_t pos = (uint64_t)T * ((E / 2) * S + m);
        io.store_row(row_out * n + pos, t, make_float2(a.x + b.x, a.y + b.y));
        io.store_row((row_out + 1) * n + pos, t, cmul(make_float2(a.x - b.x, a.y - b.y), w));
    }
}

// The row pair a workgroup takes: pair index p = image * R/2 + r.  For
// 4096-row images the launch's images run in reverse order (workgroup b
// takes image images - 1 - b / (R/2)), rows in order within each: the
// column pass starts with the launch's first image, so that image's rows are
// the last ones stored and are still in the Infinity Cache when a chunk is
// larger than the cache, and its 8-column tiles (half lines) gain from it.
// Measured on gfx950 (alternating runs on four boxes, us): config 5 (two
// 4096 x 4096 images) per step -1.5, -4.4, +0.8, -1.2 (the column pass 1.7
// .. 4.1 faster on every box, the row pass up to 0.7 slower); at 512 MiB per
// execution 4096 x 4096 381 -> 379, 4096 x 2048 376 -> 370, 4096 x 1024 368
// -> 361.  The 2048-row plans (16-column tiles, whole lines) lost 0.3 .. 1.2
// % and keep the natural order.
__device__ __forceinline__ uint64_t rowpair_index(uint64_t b, uint64_t pairs, uint32_t log_rows) {
    const uint32_t lh = log_rows - 1;
    // the plans launch R/2 pairs per image; any other count keeps the natural order
    if (log_rows != 12 || (pairs & ((1ull << lh) - 1)) != 0) return b;
    const uint64_t images = pairs >> lh;
    return ((images - 1 - (b >> lh)) << lh) | (b & ((1ull << lh) - 1));
}

// Pair p (rowpair_index): image p / (R/2), row r = p mod (R/2), R = 2^log_rows <=
// 4096; 2T threads.  big[j] = W_4096^j (the multi-pass plans' two-level root
// table), so W_R^r = big[r * 4096 / R].  flags as fft_stockham_body: the
// inverse conjugates on load here and conjugates and scales at the column
// pass.
template <int LOGN>
__device__ __forceinline__ void fft2d_rowpair_body(const float2* __restrict__ in, float2* __restrict__ out,
                                                   const float2* __restrict__ tw, const float2* __restrict__ big,
                                                   uint64_t pairs, uint32_t log_rows, uint32_t flags) {
    using Sh = StockhamShape<LOGN, 4>;
    static_assert(Sh::T % 64 == 0 && Sh::E == 16, "whole waves per row, 16 elements per thread");
    __shared__ float2 lds[2][Sh::LDS_ELEMS];
    const int s = threadIdx.x / Sh::T;  // the same for a whole wave
    const int t = threadIdx.x - s * Sh::T;
    if (blockIdx.x >= pairs) return;  // uniform over the workgroup
    const uint64_t p = rowpair_index(blockIdx.x, pairs, log_rows);
    const uint64_t half = 1ull << (log_rows - 1);
    const uint64_t r = p & (half - 1);
    const uint64_t first = (p >> (log_rows - 1)) << log_rows;  // the image's first row
    const InterleavedIOT<false, true> io{in, out};              // rows streamed in, outputs kept cached
    const uint64_t row_in = first + r + (s ? half : 0);
    float2 x[Sh::E];
#pragma unroll
    for (int m = 0; m < Sh::E; ++m) x[m] = io.load_row(row_in * Sh::N + Sh::T * m, t);
    if (flags & FG_PASS_CONJ_IN) {
#pragma unroll
        for (int m = 0; m < Sh::E; ++m) x[m] = cconj(x[m]);
    }
    StockhamStages<LOGN, 4, 0>::template run<false>(x, t, tw, lds[s]);
    __syncthreads();  // every read of the last exchange is done
    if (s == 0) rowpair_send<Sh::E, Sh::T, 0>(x, t, lds[0]);
    else rowpair_send<Sh::E, Sh::T, 1>(x, t, lds[1]);
    __syncthreads();
    const float2 w = big[r << (12 - log_rows)];
    const uint64_t row_out = first + 2 * r;
    if (s == 0) rowpair_combine<Sh::E, Sh::T, 0>(x, t, lds[1], io, row_out, Sh::N, w);
    else rowpair_combine<Sh::E, Sh::T, 1>(x, t, lds[0], io, row_out, Sh::N, w);
}

// Stages S0 .. SL of one row with the exchanges between them (the exchange
// after SL is the caller's): y holds stage SL's outputs on return.
template <int LOGN, int S0, int SL>
struct RowHalvesPrefix {
    __device__ __forceinline__ static void run(float2* x, float2* y, int t, const float2* __restrict__ tw,
                                               float2* __restrict__ lds) {
        halves_stage<LOGN, S0>(x, y, t, tw);
        if constexpr (S0 < SL) {
            row_halves_exchange<LOGN, S0>(y, x, t, lds);
            RowHalvesPrefix<LOGN, S0 + 1, SL>::run(x, y, t, tw, lds);
        }
    }
};

// The row-pair pass with 32 elements per thread (N/16 threads: two rows of
// T = N/32) and the pair combined in registers.  Half s of the
// workgroup runs row s's stages up to the one before the last (each row in
// its own LDS region, exchanges in halves); the exchange before the last
// stage then crosses the rows: each row scatters into its own region as
// usual, and thread t of half s gathers, from both regions, the inputs of
// last-stage butterfly b = T s + t of both rows (positions b + (N/16) p), so
// it holds outputs b + (N/16) q of both rows after the last stage and stores
// A + B and (A - B) W_R^r directly.  Every element goes through the same
// arithmetic as when each half runs its own row's last stage and the pair
// is exchanged through LDS afterwards (the same butterflies and twiddles,
// only run by other threads), without that exchange; the two rows' last
// butterflies share their twiddle reads.
// Measured on gfx950 against the same pass with each row's last exchange
// in its own region and the pair exchanged after it (same bits): config 5
// row pass 88.1 -> 86.4 us per 512 MiB launch, step 186.8 -> 185.1 us.
template <int LOGN>
__device__ __forceinline__ void fft2d_rowpair_fused_body(const float2* __restrict__ in, float2* __restrict__ out,
                                                         const float2* __restrict__ tw,
                                                         const float2* __restrict__ big, uint64_t pairs,
                                                         uint32_t log_rows, uint32_t flags) {
    using H = HalvesShape<LOGN>;
    static_assert(H::T % 64 == 0, "whole waves per row");
    static_assert(H::REM == 0 && H::NSTAGES >= 2, "radix-16 stages only: two last-stage butterflies per thread");
    constexpr int SP = H::NSTAGES - 2;   // the stage before the last
    constexpr int LL = H::N / 16;        // the last stage's L: butterflies per row
    constexpr int LLP = LL + LL / 16;    // lds_pos(x + LL) - lds_pos(x)
    using St = HalvesStage<LOGN, SP>;
    __shared__ float2 lds[2][H::HALF + H::HALF / 16];
    const int s = threadIdx.x / H::T;  // the same for a whole wave
    const int t = threadIdx.x - s * H::T;
    if (blockIdx.x >= pairs) return;  // uniform over the workgroup
    const uint64_t p = rowpair_index(blockIdx.x, pairs, log_rows);
    const uint64_t half = 1ull << (log_rows - 1);
    const uint64_t r = p & (half - 1);
    const uint64_t first = (p >> (log_rows - 1)) << log_rows;
    const InterleavedIOT<false, true> io{in, out};
    const uint64_t row_in = first + r + (s ? half : 0);
    float2 x[H::E], y[H::E];
#pragma unroll
    for (int m = 0; m < H::E; ++m) x[m] = io.load_row(row_in * H::N + H::T * m, t);
    if (flags & FG_PASS_CONJ_IN) {
#pragma unroll
        for (int m = 0; m < H::E; ++m) x[m] = cconj(x[m]);
    }
    RowHalvesPrefix<LOGN, 0, SP>::run(x, y, t, tw, lds[s]);
    // The cross exchange: round h, own region's writes as row_halves_exchange
    // (positions below / above N/2), then both regions' reads of inputs
    // p in [8h, 8h + 8) of butterfly b (x[p]: row 0, x[16 + p]: row 1).
    const int b = H::T * s + t;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        __syncthreads();  // the previous round's (or exchange's) readers are done
#pragma unroll
        for (int ii = 0; ii < St::NB / 2; ++ii) {
            const int i = h * (St::NB / 2) + ii;
            const int bb = t + H::T * i;
            const int d0 = (bb >> (4 * SP)) * St::L * 16 + (bb & (St::L - 1)) - H::HALF * h;
            float2* base = &lds[s][0] + lds_pos<>(d0);
#pragma unroll
            for (int q = 0; q < 16; ++q) base[q * (St::L + St::L / 16)] = y[i + St::NB * q];
        }
        __syncthreads();
        const float2* r0 = &lds[0][0] + lds_pos<>(b);
        const float2* r1 = &lds[1][0] + lds_pos<>(b);
#pragma unroll
        for (int pp = 0; pp < 8; ++pp) {
            x[8 * h + pp] = r0[pp * LLP];
            x[16 + 8 * h + pp] = r1[pp * LLP];
        }
    }
    // The last stage for both rows: butterfly b, k = b (j = 0), outputs q at b + LL q.
    const float2* twl = tw + stockham_tw_offset<LOGN, 4>(H::NSTAGES - 1);
#pragma unroll
    for (int row = 0; row < 2; ++row) {
        apply_stage_twiddles_at<16, LL>(x + 16 * row, twl, b);
        Dft<16>::run(x + 16 * row);
    }
    const float2 w = big[r << (12 - log_rows)];
    const uint64_t row_out = first + 2 * r;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const float2 a = x[q], c = x[16 + q];
        const uint64_t pos = (uint64_t)LL * q + H::T * s;
        io.store_row(row_out * H::N + pos, t, make_float2(a.x + c.x, a.y + c.y));
        io.store_row((row_out + 1) * H::N + pos, t, cmul(make_float2(a.x - c.x, a.y - c.y), w));
    }
}

}  // namespace fg

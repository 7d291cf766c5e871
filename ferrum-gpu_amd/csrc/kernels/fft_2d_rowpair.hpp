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
// workgroups per CU where a 4096-row tile takes the CU's LDS) and that of
// 2048-row images 1024-row tiles of 16 columns (whole 128-byte lines).  Rows
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

// Pair p of a launch: image p / (R/2), row r = p mod (R/2), R = 2^log_rows <=
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
    const uint64_t p = blockIdx.x;
    if (p >= pairs) return;  // uniform over the workgroup
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

// The same pass with 32 elements per thread and each row's exchanges in
// halves (fft_stockham.hpp, RowHalvesStages): 2T = N/16 threads and N/2 +
// N/32 LDS positions per row, half the LDS of the 16-element layout.
template <int LOGN>
__device__ __forceinline__ void fft2d_rowpair_halves_body(const float2* __restrict__ in, float2* __restrict__ out,
                                                          const float2* __restrict__ tw,
                                                          const float2* __restrict__ big, uint64_t pairs,
                                                          uint32_t log_rows, uint32_t flags) {
    using H = HalvesShape<LOGN>;
    static_assert(H::T % 64 == 0, "whole waves per row");
    __shared__ float2 lds[2][H::HALF + H::HALF / 16];
    const int s = threadIdx.x / H::T;  // the same for a whole wave
    const int t = threadIdx.x - s * H::T;
    const uint64_t p = blockIdx.x;
    if (p >= pairs) return;  // uniform over the workgroup
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
    RowHalvesStages<LOGN, 0>::run(x, y, t, tw, lds[s]);
    __syncthreads();  // every read of the last exchange is done
    if (s == 0) rowpair_send<H::E, H::T, 0>(y, t, lds[0]);
    else rowpair_send<H::E, H::T, 1>(y, t, lds[1]);
    __syncthreads();
    const float2 w = big[r << (12 - log_rows)];
    const uint64_t row_out = first + 2 * r;
    if (s == 0) rowpair_combine<H::E, H::T, 0>(y, t, lds[1], io, row_out, H::N, w);
    else rowpair_combine<H::E, H::T, 1>(y, t, lds[0], io, row_out, H::N, w);
}

}  // namespace fg

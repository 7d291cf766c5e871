// shape_copy.hpp -- yardstick copies: out = in with exactly the global access
// shape, workgroup size, LDS footprint and launch order of an FFT kernel, and
// no arithmetic.  The time of such a copy is the floor of that kernel's
// access shape: how fast HBM (or the Infinity Cache) serves those loads and
// stores at that occupancy.  The bench times them beside the FFT kernels
// (bench.py --workload shape_*), like fg_copy_f4 beside every workload.
//
// Each copy keeps its kernel's LDS allocation (one write and read of the
// thread's own slot around a barrier, so the compiler keeps the array and
// with it the workgroups-per-CU limit) and returns every element unchanged.
#pragma once
#include "fft_tile.hpp"
#include "fft_2d_rowpair.hpp"

namespace fg {

// The LDS footprint of a kernel: the thread's own slot written, a barrier,
// read back (the value is unchanged).
__device__ __forceinline__ float2 touch_lds(float2* lds, float2 v) {
    lds[threadIdx.x] = v;
    __syncthreads();
    return lds[threadIdx.x];
}

// fg_fft_n13 .. n15 (fft_row_halves_body): one 2^LOGN-point row per
// workgroup of N/32 threads, 32 elements per thread at t + T m, nontemporal
// both ways, N/2 + N/32 LDS slots, the same start stagger.
template <int LOGN>
__device__ __forceinline__ void copy_shape_rows_halves(const float2* __restrict__ in, float2* __restrict__ out,
                                                       uint64_t batch) {
    using H = HalvesShape<LOGN>;
    __shared__ float2 lds[H::HALF + H::HALF / 16];
    const int t = threadIdx.x;
    const uint64_t f = blockIdx.x;
    if (f >= batch) return;
    stagger_lockstep_start<(H::HALF + H::HALF / 16) * 8, H::T>();
    const InterleavedIO io{in, out};
    float2 x[H::E];
#pragma unroll
    for (int m = 0; m < H::E; ++m) x[m] = io.load_row(f * H::N + H::T * m, t);
    x[0] = touch_lds(lds, x[0]);
#pragma unroll
    for (int m = 0; m < H::E; ++m) io.store_row(f * H::N + H::T * m, t, x[m]);
}

// fg_fft_n10 (fft1024_x2_body): two 1024-point transforms per 128-thread
// workgroup, thread t at t + 128 p of each, nontemporal both ways, 2 x (1024
// + 64) LDS slots.
__device__ __forceinline__ void copy_shape_x2_1024(const float2* __restrict__ in, float2* __restrict__ out,
                                                   uint64_t batch) {
    __shared__ float2 lds[2][1024 + 64];
    const int t = threadIdx.x;
    const uint64_t f0 = (uint64_t)blockIdx.x * 2;
    const bool has1 = f0 + 1 < batch;
    const InterleavedIO io{in, out};
    float2 x[16];
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int p = 0; p < 8; ++p)
            x[8 * f + p] = (f == 0 || has1) ? io.load((f0 + f) * 1024 + t + 128 * p) : make_float2(0.f, 0.f);
    x[0] = touch_lds(&lds[0][0], x[0]);
#pragma unroll
    for (int f = 0; f < 2; ++f)
        if (f == 0 || has1) {
#pragma unroll
            for (int p = 0; p < 8; ++p) io.store((f0 + f) * 1024 + t + 128 * p, x[8 * f + p]);
        }
}

// fg_tile_l<LOGL>_g<G>_h<policy> (fft_tile_halves_body): G columns of 2^LOGL
// points per workgroup at the tile geometry's strides and tile order, 32
// elements per thread, the pass's cache policy, TileLayout<LOGL - 1, G> of
// LDS.  With the FFT pass's own geometry (in == out for an in-place pass)
// every element goes back where it was read.
template <int LOGL, int G, bool LOAD_CACHED, bool STORE_CACHED>
__device__ __forceinline__ void copy_shape_tile_halves(const float2* __restrict__ in, float2* __restrict__ out,
                                                       const TileGeom& g) {
    using H = HalvesShape<LOGL>;
    __shared__ float2 lds[TileLayout<LOGL - 1, G>::ELEMS];
    const int tid = threadIdx.x;
    const int c = tid % G;
    const int t = tid / G;
    const TileCoords tc = tile_coords<G>(g);
    const char* in_tile = reinterpret_cast<const char*>(in + tc.ib);
    char* out_tile = reinterpret_cast<char*>(out + tc.ob);
    float2 x[H::E];
    {
        const uint32_t lane_off = (uint32_t)((c + (uint64_t)t * g.ies) * sizeof(float2));
        const uint64_t row_step = (uint64_t)H::T * g.ies * sizeof(float2);
#pragma unroll
        for (int m = 0; m < H::E; ++m)
            x[m] = gload<LOAD_CACHED>(reinterpret_cast<const float2*>(in_tile + m * row_step + lane_off));
    }
    x[0] = touch_lds(lds, x[0]);
    const uint32_t lane_off = (uint32_t)((c + (uint64_t)t * g.oes) * sizeof(float2));
    const uint64_t row_step = (uint64_t)H::T * g.oes * sizeof(float2);
#pragma unroll
    for (int m = 0; m < H::E; ++m)
        gstore<STORE_CACHED>(reinterpret_cast<float2*>(out_tile + m * row_step + lane_off), x[m]);
}

// fg_fft2d_rowpair_n<LOGN> with 32 elements per thread
// (fft2d_rowpair_fused_body): rows r and r + R/2 of an image per workgroup,
// images in the kernel's order (rowpair_index)
// of 2T threads, streamed in, stored cached to rows 2r and 2r + 1 (each
// row's values to its own output row: a permutation of the rows), two
// N/2 + N/32-slot LDS regions.
template <int LOGN>
__device__ __forceinline__ void copy_shape_rowpair_halves(const float2* __restrict__ in, float2* __restrict__ out,
                                                          uint64_t pairs, uint32_t log_rows) {
    using H = HalvesShape<LOGN>;
    __shared__ float2 lds[2][H::HALF + H::HALF / 16];
    const int s = threadIdx.x / H::T;
    const int t = threadIdx.x - s * H::T;
    if (blockIdx.x >= pairs) return;
    const uint64_t p = rowpair_index(blockIdx.x, pairs, log_rows);
    const uint64_t half = 1ull << (log_rows - 1);
    const uint64_t r = p & (half - 1);
    const uint64_t first = (p >> (log_rows - 1)) << log_rows;
    const InterleavedIOT<false, true> io{in, out};
    const uint64_t row_in = first + r + (s ? half : 0);
    float2 x[H::E];
#pragma unroll
    for (int m = 0; m < H::E; ++m) x[m] = io.load_row(row_in * H::N + H::T * m, t);
    x[0] = touch_lds(&lds[0][0], x[0]);
    const uint64_t row_out = first + 2 * r + s;
#pragma unroll
    for (int m = 0; m < H::E; ++m) io.store_row(row_out * H::N + H::T * m, t, x[m]);
}

}  // namespace fg

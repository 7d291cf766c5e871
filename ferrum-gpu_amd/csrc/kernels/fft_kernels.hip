// fft_kernels.hip -- the gfx950 code object loaded by the HIP backend.
//
// Every kernel has an unmangled extern "C" name so the host looks it up with
// hipModuleGetFunction, the way the reference's host runner looks up the
// kernels of its embedded module (crates/ferrum-gpu-py/src/lib.rs:54-79).
//
// Built by ferrum-gpu_amd/csrc/Makefile with
//   hipcc --genco --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops
#include "fft_stockham.hpp"

using namespace fg;

// Launch geometry is fixed per kernel and mirrored on the host in
// fft_plan.cpp (kStockhamTable): LOGE = min(4, LOGN); FPB transforms per
// workgroup of FPB * (N / E) threads.  fg_fft_n<L> reads and writes
// interleaved complex64; fg_fft_n<L>_split the split layout (re and im arrays,
// the reference's *_split kernels K4/K8/K11), with the same arithmetic.
#define FG_STOCKHAM(LOGN, LOGE, FPB)                                                          \
    extern "C" __global__ __launch_bounds__(FPB * ((1 << LOGN) >> LOGE)) void                  \
        fg_fft_n##LOGN(const float2* __restrict__ in, float2* __restrict__ out,                \
                       const float2* __restrict__ tw, uint64_t batch, float scale,            \
                       uint32_t flags) {                                                      \
        fft_stockham_body<LOGN, LOGE, FPB>(InterleavedIO{in, out}, tw, batch, scale, flags);  \
    }                                                                                         \
    extern "C" __global__ __launch_bounds__(FPB * ((1 << LOGN) >> LOGE)) void                  \
        fg_fft_n##LOGN##_split(const float* __restrict__ in_re, const float* __restrict__ in_im, \
                               float* __restrict__ out_re, float* __restrict__ out_im,          \
                               const float2* __restrict__ tw, uint64_t batch, float scale,    \
                               uint32_t flags) {                                              \
        fft_stockham_body<LOGN, LOGE, FPB>(SplitIO{in_re, in_im, out_re, out_im}, tw, batch,  \
                                           scale, flags);                                     \
    }

// fg_fft_n<L>_sc: the same transform with the input streamed and the output
// stored cached -- the first launch of a 2D plan's chunk, whose output the
// column passes read next (fft_common.hpp, gload/gstore).
#define FG_STOCKHAM_SC(LOGN, LOGE, FPB)                                                        \
    extern "C" __global__ __launch_bounds__(FPB * ((1 << LOGN) >> LOGE)) void                  \
        fg_fft_n##LOGN##_sc(const float2* __restrict__ in, float2* __restrict__ out,           \
                            const float2* __restrict__ tw, uint64_t batch, float scale,       \
                            uint32_t flags) {                                                 \
        fft_stockham_body<LOGN, LOGE, FPB>(InterleavedIOT<false, true>{in, out}, tw, batch,   \
                                           scale, flags);                                     \
    }

FG_STOCKHAM(2, 2, 64)    // N=4:    1 thread  / transform, 64 per wave
FG_STOCKHAM(3, 3, 64)    // N=8:    1 thread  / transform
FG_STOCKHAM(4, 3, 32)    // N=16:   2 threads / transform
FG_STOCKHAM(5, 3, 16)    // N=32:   4 threads / transform
FG_STOCKHAM(6, 2, 4)     // N=64:   16 threads (4 elements each)
FG_STOCKHAM(7, 3, 4)     // N=128:  16 threads (8 elements each)
FG_STOCKHAM(8, 4, 4)     // N=256:  16 threads
FG_STOCKHAM(9, 4, 2)     // N=512:  32 threads
// N=1024: two transforms per 128-thread workgroup, radix list 8 * 16 * 8
// (fft1024_x2_body): fg_fft_n10, its split twin and the cached-store variant
// fg_fft_n10_sc share the body, so they give the same bits.
#define FG_STOCKHAM_X2_1024()                                                                        \
    extern "C" __global__ __launch_bounds__(128) void fg_fft_n10(                                   \
        const float2* __restrict__ in, float2* __restrict__ out, const float2* __restrict__ tw,      \
        uint64_t batch, float scale, uint32_t flags) {                                              \
        fft1024_x2_body(InterleavedIO{in, out}, tw, batch, scale, flags);                           \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(128) void fg_fft_n10_split(                             \
        const float* __restrict__ in_re, const float* __restrict__ in_im, float* __restrict__ out_re, \
        float* __restrict__ out_im, const float2* __restrict__ tw, uint64_t batch, float scale,     \
        uint32_t flags) {                                                                           \
        fft1024_x2_body(SplitIO{in_re, in_im, out_re, out_im}, tw, batch, scale, flags);            \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(128) void fg_fft_n10_sc(                                \
        const float2* __restrict__ in, float2* __restrict__ out, const float2* __restrict__ tw,      \
        uint64_t batch, float scale, uint32_t flags) {                                              \
        fft1024_x2_body(InterleavedIOT<false, true>{in, out}, tw, batch, scale, flags);             \
    }
FG_STOCKHAM_X2_1024()
FG_STOCKHAM(11, 4, 1)    // N=2048: 128 threads
FG_STOCKHAM(12, 4, 1)    // N=4096: 256 threads
// N = 8192 / 16384: one transform per workgroup of N/32 threads with 32
// elements each and the exchanges in halves (fft_row_halves_body), at most
// 128 VGPRs (four waves per SIMD): 34 / 68 KB of LDS, four / two workgroups
// per CU.  The stage table is the 16-element layout's (kStockham holds
// log_e = 5 for the geometry; the host builds the table with log_e = 4).
#define FG_STOCKHAM_HALVES(LOGN)                                                               \
    extern "C" __global__ __launch_bounds__(HalvesShape<LOGN>::T) __attribute__((amdgpu_waves_per_eu(4))) \
    void fg_fft_n##LOGN(const float2* __restrict__ in, float2* __restrict__ out,               \
                        const float2* __restrict__ tw, uint64_t batch, float scale, uint32_t flags) { \
        fft_row_halves_body<LOGN>(InterleavedIO{in, out}, tw, batch, scale, flags);            \
    }                                                                                          \
    extern "C" __global__ __launch_bounds__(HalvesShape<LOGN>::T) __attribute__((amdgpu_waves_per_eu(4))) \
    void fg_fft_n##LOGN##_split(const float* __restrict__ in_re, const float* __restrict__ in_im, \
                                float* __restrict__ out_re, float* __restrict__ out_im,        \
                                const float2* __restrict__ tw, uint64_t batch, float scale,     \
                                uint32_t flags) {                                               \
        fft_row_halves_body<LOGN>(SplitIO{in_re, in_im, out_re, out_im}, tw, batch, scale, flags); \
    }
FG_STOCKHAM_HALVES(13)   // N=8192:  256 threads
FG_STOCKHAM_HALVES(14)   // N=16384: 512 threads
FG_STOCKHAM_HALVES(15)   // N=32768: 1024 threads, 136 KB of LDS
// fg_fft_n<L>_lat[_split]: one transform per workgroup with fewer elements per
// thread (kStockhamLatency in fft_plan.cpp), for batches too small to fill the
// GPU; the split twin keeps split and interleaved results bit-identical.
#define FG_STOCKHAM_LAT(LOGN, LOGE)                                                            \
    extern "C" __global__ __launch_bounds__((1 << LOGN) >> LOGE) void                           \
        fg_fft_n##LOGN##_lat(const float2* __restrict__ in, float2* __restrict__ out,           \
                             const float2* __restrict__ tw, uint64_t batch, float scale,       \
                             uint32_t flags) {                                                 \
        fft_stockham_body<LOGN, LOGE, 1>(InterleavedIO{in, out}, tw, batch, scale, flags);     \
    }                                                                                          \
    extern "C" __global__ __launch_bounds__((1 << LOGN) >> LOGE) void                           \
        fg_fft_n##LOGN##_lat_split(const float* __restrict__ in_re, const float* __restrict__ in_im, \
                                   float* __restrict__ out_re, float* __restrict__ out_im,      \
                                   const float2* __restrict__ tw, uint64_t batch, float scale,  \
                                   uint32_t flags) {                                           \
        fft_stockham_body<LOGN, LOGE, 1>(SplitIO{in_re, in_im, out_re, out_im}, tw, batch,     \
                                         scale, flags);                                        \
    }
FG_STOCKHAM_LAT(8, 2)    // N=256:  64 threads (4 elements each)
FG_STOCKHAM_LAT(10, 3)   // N=1024: 128 threads (8 elements each)
FG_STOCKHAM_LAT(12, 3)   // N=4096: 512 threads (8 elements each)

FG_STOCKHAM_SC(4, 3, 32)
FG_STOCKHAM_SC(5, 3, 16)
FG_STOCKHAM_SC(6, 2, 4)
FG_STOCKHAM_SC(7, 3, 4)
FG_STOCKHAM_SC(8, 4, 4)
FG_STOCKHAM_SC(9, 4, 2)
FG_STOCKHAM_SC(11, 4, 1)
FG_STOCKHAM_SC(12, 4, 1)

// ---------------------------------------------------------------- utilities

// Streaming copy, 16 bytes per lane with nontemporal hints, one element per
// thread in 64-thread workgroups (the fastest plain-copy shape measured on
// gfx950): the HBM yardstick the bench reports beside the FFT, and the
// known-size kernel used to scale rocprof's FETCH_SIZE / WRITE_SIZE counters.
extern "C" __global__ __launch_bounds__(64) void fg_copy_f4(const float4* __restrict__ in,
                                                            float4* __restrict__ out,
                                                            uint64_t n4) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    const v4f* src = reinterpret_cast<const v4f*>(in);
    v4f* dst = reinterpret_cast<v4f*>(out);
    uint64_t i = (uint64_t)blockIdx.x * 64 + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * 64;
    for (; i < n4; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// out[b][c][r] = in[b][r][c] for `batch` rows x cols complex64 matrices: the
// tiled transpose of the reference's 2D path (transpose_complex_pow2,
// crates/ferrum-gpu-fft-kernels/src/kernels_body.rs:763-805), here as a
// standalone operation on any shape.  64 x 64 tiles through LDS (pitch 65:
// the transposed reads of a wave hit distinct banks); both the global reads
// and writes are 64 lanes x 8 contiguous bytes.  tiles_c = ceil(cols / 64),
// tiles_r = ceil(rows / 64); grid = tiles_c * tiles_r * batch.
extern "C" __global__ __launch_bounds__(256) void fg_transpose_c64(const float2* __restrict__ in,
                                                                   float2* __restrict__ out, uint32_t rows,
                                                                   uint32_t cols, uint32_t tiles_c,
                                                                   uint32_t tiles_r) {
    __shared__ float2 tile[64][65];
    uint32_t bx = blockIdx.x;
    const uint32_t tc = bx % tiles_c;
    bx /= tiles_c;
    const uint32_t tr = bx % tiles_r;
    const uint64_t img = (uint64_t)(bx / tiles_r) * rows * cols;
    const uint32_t tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const uint32_t c = tc * 64 + tx;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t r = tr * 64 + ty + 4 * i;
        if (r < rows && c < cols) tile[ty + 4 * i][tx] = load_stream(in + img + (uint64_t)r * cols + c);
    }
    __syncthreads();
    const uint32_t orow_col = tr * 64 + tx;  // output column = input row
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t orow = tc * 64 + ty + 4 * i;  // output row = input column
        if (orow < cols && orow_col < rows) store_stream(out + img + (uint64_t)orow * rows + orow_col, tile[tx][ty + 4 * i]);
    }
}

// The same transpose for matrices of at least 128 x 128: 128 x 128 tiles
// (1024 threads, 132 KB of LDS, pitch 129), each global read and write a
// 1 KB row piece, and the tiles walked in super-tiles of sc x sr tiles
// (8 x 8, fewer along a dimension with fewer tiles), tile column fastest
// inside a super-tile and super-tiles row-major, so the workgroups in flight
// cover a square region of both the input and the output.  On an 8192 x 8192
// matrix this moved 6.1 TB/s against 4.4 TB/s for the 64 x 64 tiles in row
// order (copy probes and the kernel itself).  Grid = image blocks * batch,
// image blocks = ceil(tiles_c / sc) sc * ceil(tiles_r / sr) sr; blocks past
// the last tile of a row or column of tiles exit at once.
extern "C" __global__ __launch_bounds__(1024) void fg_transpose_c64_t128(
    const float2* __restrict__ in, float2* __restrict__ out, uint32_t rows, uint32_t cols, uint32_t tiles_c,
    uint32_t tiles_r, uint32_t sc, uint32_t sr, uint32_t supers_c, uint32_t image_blocks) {
    __shared__ float2 tile[128][129];
    const uint32_t b = blockIdx.x % image_blocks;
    const uint64_t img = (uint64_t)(blockIdx.x / image_blocks) * rows * cols;
    const uint32_t per = sc * sr, sb = b / per, k = b % per;
    const uint32_t tc = (sb % supers_c) * sc + k % sc, tr = (sb / supers_c) * sr + k / sc;
    if (tc >= tiles_c || tr >= tiles_r) return;  // whole workgroup, before any barrier
    const uint32_t tx = threadIdx.x & 127, ty = threadIdx.x >> 7;
    const uint32_t c = tc * 128 + tx;
    // Interior tiles (every tile of a matrix whose sides are multiples of 128)
    // issue all sixteen loads, then all sixteen stores, with no per-element
    // test; edge tiles test each element.
    const bool full = (tr + 1) * 128 <= rows && (tc + 1) * 128 <= cols;
    if (full) {
        float2 v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = load_stream(in + img + (uint64_t)(tr * 128 + ty + 8 * i) * cols + c);
#pragma unroll
        for (int i = 0; i < 16; ++i) tile[ty + 8 * i][tx] = v[i];
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t r = tr * 128 + ty + 8 * i;
            if (r < rows && c < cols) tile[ty + 8 * i][tx] = load_stream(in + img + (uint64_t)r * cols + c);
        }
    }
    __syncthreads();
    const uint32_t ocol = tr * 128 + tx;  // output column = input row
    if (full) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            store_stream(out + img + (uint64_t)(tc * 128 + ty + 8 * i) * rows + ocol, tile[tx][ty + 8 * i]);
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t orow = tc * 128 + ty + 8 * i;  // output row = input column
            if (orow < cols && ocol < rows)
                store_stream(out + img + (uint64_t)orow * rows + ocol, tile[tx][ty + 8 * i]);
        }
    }
}

// c = a + b over n floats: the substrate smoke kernel (the reference's
// hand-written vector_add, examples/vector-add/src/main.rs:17-60).
extern "C" __global__ __launch_bounds__(256) void fg_vector_add(const float* __restrict__ a,
                                                                const float* __restrict__ b,
                                                                float* __restrict__ c,
                                                                uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) c[i] = a[i] + b[i];
}

// ------------------------------------------------------------ small 2D
//
// fg_fft2d_l<LR>_<LC>[_split]: the whole 2D FFT of 2^LR x 2^LC images (<= 16384 points)
// in one pass, FG_SMALL2D_FPI images per workgroup (fft_2d_small.hpp).
#include "fft_2d_small.hpp"
#include "fft_2d_halves.hpp"

#define FG_FFT2D(LR, LC)                                                                            \
    extern "C" __global__ __launch_bounds__(FG_SMALL2D_BLOCK(LR, LC)) void                           \
        fg_fft2d_l##LR##_##LC(const float2* __restrict__ in, float2* __restrict__ out,              \
                              const float2* __restrict__ tw_rows, const float2* __restrict__ tw_cols, \
                              uint64_t batch, float scale, uint32_t flags) {                         \
        fft2d_small_body<LR, LC, FG_SMALL2D_LOGE(LR, LC), FG_SMALL2D_FPI(LR, LC)>(InterleavedIO{in, out}, tw_rows, \
                                                                          tw_cols, batch, scale, flags); \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(FG_SMALL2D_BLOCK(LR, LC)) void                           \
        fg_fft2d_l##LR##_##LC##_split(const float* __restrict__ in_re, const float* __restrict__ in_im, \
                                      float* __restrict__ out_re, float* __restrict__ out_im,        \
                                      const float2* __restrict__ tw_rows,                             \
                                      const float2* __restrict__ tw_cols, uint64_t batch, float scale, \
                                      uint32_t flags) {                                               \
        fft2d_small_body<LR, LC, FG_SMALL2D_LOGE(LR, LC), FG_SMALL2D_FPI(LR, LC)>(                    \
            SplitIO{in_re, in_im, out_re, out_im}, tw_rows, tw_cols, batch, scale, flags);            \
    }
// 2048- to 16384-point images: one per workgroup of N/32 threads, in
// registers, the exchanges in halves (fft2d_halves_body).
#define FG_FFT2D_HALVES(LR, LC)                                                                     \
    extern "C" __global__ __launch_bounds__(FG_SMALL2D_BLOCK(LR, LC)) __attribute__((amdgpu_waves_per_eu(4))) void \
        fg_fft2d_l##LR##_##LC(const float2* __restrict__ in, float2* __restrict__ out,              \
                              const float2* __restrict__ tw_rows, const float2* __restrict__ tw_cols, \
                              uint64_t batch, float scale, uint32_t flags) {                         \
        fft2d_halves_body<LR, LC>(InterleavedIO{in, out}, tw_rows, tw_cols, batch, scale, flags);    \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(FG_SMALL2D_BLOCK(LR, LC)) __attribute__((amdgpu_waves_per_eu(4))) void \
        fg_fft2d_l##LR##_##LC##_split(const float* __restrict__ in_re, const float* __restrict__ in_im, \
                                      float* __restrict__ out_re, float* __restrict__ out_im,        \
                                      const float2* __restrict__ tw_rows,                             \
                                      const float2* __restrict__ tw_cols, uint64_t batch, float scale, \
                                      uint32_t flags) {                                               \
        fft2d_halves_body<LR, LC>(SplitIO{in_re, in_im, out_re, out_im}, tw_rows, tw_cols, batch, scale, \
                                  flags);                                                             \
    }
FG_FFT2D(4, 4)
FG_FFT2D(4, 5)
FG_FFT2D(4, 6)
FG_FFT2D_HALVES(4, 7)
FG_FFT2D_HALVES(4, 8)
FG_FFT2D_HALVES(4, 9)
FG_FFT2D_HALVES(4, 10)
FG_FFT2D(5, 4)
FG_FFT2D(5, 5)
FG_FFT2D_HALVES(5, 6)
FG_FFT2D_HALVES(5, 7)
FG_FFT2D_HALVES(5, 8)
FG_FFT2D_HALVES(5, 9)
FG_FFT2D(6, 4)
FG_FFT2D_HALVES(6, 5)
FG_FFT2D_HALVES(6, 6)
FG_FFT2D_HALVES(6, 7)
FG_FFT2D_HALVES(6, 8)
FG_FFT2D_HALVES(7, 4)
FG_FFT2D_HALVES(7, 5)
FG_FFT2D_HALVES(7, 6)
FG_FFT2D_HALVES(7, 7)
FG_FFT2D_HALVES(8, 4)
FG_FFT2D_HALVES(8, 5)
FG_FFT2D_HALVES(8, 6)
FG_FFT2D_HALVES(9, 4)
FG_FFT2D_HALVES(9, 5)
FG_FFT2D_HALVES(10, 4)

// Row pass of 2D plans of 2048 / 4096 rows of 1024 .. 4096 points: rows r
// and r + R/2 per workgroup, combined radix-2 over the row index
// (fft_2d_rowpair.hpp), so the column pass runs R/2-row tiles.  1024 / 2048
// points: the 16-element layout (64 / 128 threads and 8.5 / 17 KB of LDS per
// row, 128 / 256 threads per workgroup); 4096 points:
// 32 elements per thread with the exchanges in halves (128 threads and 17 KB
// per row, four workgroups per CU; the last exchange crosses the pair so the
// pair combines in registers, fft2d_rowpair_fused_body), measured on gfx950
// per 4096 x 4096 image against the 16-element layout (512 threads, 68 KB,
// two per CU): whole plan 101.4 -> 99.1 us, same bits.
#include "fft_2d_rowpair.hpp"
extern "C" __global__ __launch_bounds__(128) void fg_fft2d_rowpair_n10(
    const float2* __restrict__ in, float2* __restrict__ out, const float2* __restrict__ tw,
    const float2* __restrict__ big, uint64_t pairs, uint32_t log_rows, uint32_t flags) {
    fft2d_rowpair_body<10>(in, out, tw, big, pairs, log_rows, flags);
}
extern "C" __global__ __launch_bounds__(256) void fg_fft2d_rowpair_n11(
    const float2* __restrict__ in, float2* __restrict__ out, const float2* __restrict__ tw,
    const float2* __restrict__ big, uint64_t pairs, uint32_t log_rows, uint32_t flags) {
    fft2d_rowpair_body<11>(in, out, tw, big, pairs, log_rows, flags);
}
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void fg_fft2d_rowpair_n12(
    const float2* __restrict__ in, float2* __restrict__ out, const float2* __restrict__ tw,
    const float2* __restrict__ big, uint64_t pairs, uint32_t log_rows, uint32_t flags) {
    fft2d_rowpair_fused_body<12>(in, out, tw, big, pairs, log_rows, flags);
}

// ------------------------------------------------------- multi-pass tiles
//
// fg_tile_l<LOGL>_g<G>_<c|r|h>[_<policy>]: one pass over G columns of length
// 2^LOGL per workgroup (G * 2^LOGL / 16 threads; 'h': / 32).  'c': columns
// contiguous in memory (column passes); 'r': rows contiguous (the last 1D
// pass, which transposes through LDS); 'h': a column pass with 32 elements
// per thread and the exchanges in halves (the first 1D pass).  Policy (fft_common.hpp, gload/gstore): none =
// stream in and out; _sc = stream in, cached out (a chunk's first pass); _cc
// (middle passes); _cs = cached in, stream out (last pass).  The host picks
// the names in fft_plan.cpp (tile_name).
#include "fft_tile.hpp"

#define FG_TILE_P(LOGL, G, RW, TAG, LC, SC)                                                          \
    extern "C" __global__ __launch_bounds__(G * ((1 << LOGL) >> (LOGL < 4 ? LOGL : 4))) void        \
        fg_tile_l##LOGL##_g##G##_##TAG(const float2* __restrict__ in, float2* __restrict__ out,     \
                                       const float2* __restrict__ tw, const float2* __restrict__ big, \
                                       TileGeom g) {                                                  \
        fft_tile_pass<LOGL, (LOGL < 4 ? LOGL : 4), G, RW, true, LC, SC>(in, out, tw, big, g);        \
    }
#define FG_TILE(LOGL, G, RW, TAG)                  \
    FG_TILE_P(LOGL, G, RW, TAG, false, false)      \
    FG_TILE_P(LOGL, G, RW, TAG##_cs, true, false)  \
    FG_TILE_P(LOGL, G, RW, TAG##_sc, false, true)  \
    FG_TILE_P(LOGL, G, RW, TAG##_cc, true, true)
// Narrow tiles (G < 16: 32- or 64-byte pieces of each line) only ever load
// and store through the caches, in XCD-aware order: the _cc policy alone.
#define FG_TILE_NARROW(LOGL, G, RW, TAG) FG_TILE_P(LOGL, G, RW, TAG##_cc, true, true)

// Column passes of 2D images of 16 .. 64 rows (at least 512 columns, so 64
// per tile).  From 128 points up the wide column passes run the halves
// tiles below.
FG_TILE(4, 64, false, c)
FG_TILE(5, 64, false, c)
FG_TILE(6, 64, false, c)
// Column passes over cache-resident data of 1D middle digits of 128 points:
// 8 columns per tile (256 points: the 16-column halves tile below).
FG_TILE_NARROW(7, 8, false, c)
// Column passes at the HBM width from 128 points up (the first 1D pass, 1D
// middle passes of unchunked plans, 2D column passes of 128 .. 1024 rows):
// the column DFTs and four-step twiddle with 32 elements per thread and the
// exchanges in halves (fft_tile_halves_body), half the LDS of the 16-element
// tile, so twice the workgroups per CU; at most 128 VGPRs (four waves per
// SIMD).  Policies: none (unchunked) and _sc (a chunk's first pass).
#define FG_TILE_HALVES_P(LOGL, G, TAG, LC, SC)                                                             \
    extern "C" __global__ __launch_bounds__(G * HalvesShape<LOGL>::T) __attribute__((amdgpu_waves_per_eu(4))) \
    void fg_tile_l##LOGL##_g##G##_h##TAG(const float2* __restrict__ in, float2* __restrict__ out,              \
                                         const float2* __restrict__ tw, const float2* __restrict__ big,       \
                                         TileGeom g) {                                                        \
        fft_tile_halves_pass<LOGL, G, LC, SC>(in, out, tw, big, g);                                           \
    }
#define FG_TILE_HALVES(LOGL, G)                  \
    FG_TILE_HALVES_P(LOGL, G, , false, false)    \
    FG_TILE_HALVES_P(LOGL, G, _sc, false, true)
FG_TILE_HALVES(7, 64)
FG_TILE_HALVES(8, 32)
FG_TILE_HALVES(9, 16)
FG_TILE_HALVES(10, 16)
// 2D column passes of 2048 / 4096 rows (cached in and out, like every narrow
// tile): 8 columns per tile, 512 / 1024 threads, 68 / 136 KB of LDS.
#define FG_TILE_HALVES_NARROW(LOGL, G) FG_TILE_HALVES_P(LOGL, G, _cc, true, true)
FG_TILE_HALVES_NARROW(11, 8)
FG_TILE_HALVES_NARROW(12, 8)
// The 1D middle pass of 256 points over cache-resident data: 16 columns
// (whole 128-byte lines), 128 threads, 17 KB of LDS, cached in and out.
FG_TILE_HALVES_P(8, 16, _cc, true, true)
// 2D column passes of chunked plans at the HBM width: 128 .. 1024 rows,
// cached in, streamed out.
FG_TILE_HALVES_P(7, 64, _cs, true, false)
FG_TILE_HALVES_P(8, 32, _cs, true, false)
FG_TILE_HALVES_P(9, 16, _cs, true, false)
FG_TILE_HALVES_P(10, 16, _cs, true, false)
// 1D last passes of 256 points in 32-row tiles and of 512 / 1024 points in
// 16-row tiles: rows in (all loads issued at once, each half transposed
// through LDS), exchanges in halves, columns out (256- / 128-byte pieces),
// streamed out or unchunked.
#define FG_TILE_ROW_HALVES(LOGL, G, TAG, LC, SC)                                                           \
    extern "C" __global__ __launch_bounds__(G * HalvesShape<LOGL>::T) __attribute__((amdgpu_waves_per_eu(4))) \
    void fg_tile_l##LOGL##_g##G##_rh##TAG(const float2* __restrict__ in, float2* __restrict__ out,             \
                                          const float2* __restrict__ tw, const float2* __restrict__ big,      \
                                          TileGeom g) {                                                       \
        fft_tile_halves_pass<LOGL, G, LC, SC, true>(in, out, tw, big, g);                                     \
    }
FG_TILE_ROW_HALVES(8, 32, , false, false)
FG_TILE_ROW_HALVES(8, 32, _cs, true, false)
FG_TILE_ROW_HALVES(9, 16, , false, false)
FG_TILE_ROW_HALVES(9, 16, _cs, true, false)
FG_TILE_ROW_HALVES(10, 16, , false, false)
FG_TILE_ROW_HALVES(10, 16, _cs, true, false)
// Row passes (last 1D digit: rows contiguous, transposed store): the widths
// for HBM-resident input, then those for cache-resident input.
FG_TILE(7, 64, true, r)
FG_TILE(7, 16, true, r)
FG_TILE_NARROW(9, 8, true, r)

// ------------------------------------------------------------- pointwise
//
// fg_<op>_vec: 16-byte accesses (every pointer 16-byte aligned; W elements
// per thread step: 2 on interleaved streams, 4 for cmul_split); fg_<op>_elem:
// one element per thread step, any alignment.  n is the number of complex
// elements.  256-thread workgroups, grid-stride.
#include "pointwise.hpp"

#define FG_POINTWISE(SUFFIX, WC, WS)                                                                  \
    extern "C" __global__ __launch_bounds__(256) void fg_cmul_c64_##SUFFIX(                          \
        const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out, uint64_t n) { \
        cmul_c64_body<WC>(a, b, out, n);                                                              \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(256) void fg_cmul_split_##SUFFIX(                        \
        const float* __restrict__ a_re, const float* __restrict__ a_im, const float* __restrict__ b_re, \
        const float* __restrict__ b_im, float* __restrict__ o_re, float* __restrict__ o_im, uint64_t n) { \
        cmul_split_body<WS>(a_re, a_im, b_re, b_im, o_re, o_im, n);                                   \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(256) void fg_deinterleave_c64_##SUFFIX(                  \
        const float* __restrict__ in, float* __restrict__ re, float* __restrict__ im, uint64_t n) {   \
        deinterleave_body<WC>(in, re, im, n);                                                         \
    }                                                                                                 \
    extern "C" __global__ __launch_bounds__(256) void fg_interleave_c64_##SUFFIX(                    \
        const float* __restrict__ re, const float* __restrict__ im, float* __restrict__ out, uint64_t n) { \
        interleave_body<WC>(re, im, out, n);                                                          \
    }

FG_POINTWISE(vec, 2, 4)
FG_POINTWISE(elem, 1, 1)

// ------------------------------------------------------------- synthetic data
//
// fg_fill_c64: n seeded complex64 values, uniform in [-1, 1) or standard normal
// (the generator is defined in fill.hpp).  256-thread workgroups, grid-stride.
#include "fill.hpp"

extern "C" __global__ __launch_bounds__(256) void fg_fill_c64(float2* __restrict__ out, uint64_t n, uint64_t seed,
                                                             uint32_t normal) {
    fill_c64_body(out, n, seed, normal);
}

// ------------------------------------------------------------ shape copies
//
// fg_copy_shape_*: out = in with the access shape, workgroup size and LDS of
// an FFT kernel and no arithmetic (shape_copy.hpp): the memory-only floor of
// that kernel, timed by the bench beside it.  n10: fg_fft_n10 (config 3);
// n14 / n15: fg_fft_n14 / fg_fft_n15; rowpair_n12 and tile_l11_g8_h_cc:
// config 5's row and column passes (the column pass launched with that
// pass's geometry, in place).
#include "shape_copy.hpp"

extern "C" __global__ __launch_bounds__(128) void fg_copy_shape_n10(const float2* __restrict__ in,
                                                                   float2* __restrict__ out, uint64_t batch) {
    copy_shape_x2_1024(in, out, batch);
}
extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void fg_copy_shape_n14(
    const float2* __restrict__ in, float2* __restrict__ out, uint64_t batch) {
    copy_shape_rows_halves<14>(in, out, batch);
}
extern "C" __global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4))) void fg_copy_shape_n15(
    const float2* __restrict__ in, float2* __restrict__ out, uint64_t batch) {
    copy_shape_rows_halves<15>(in, out, batch);
}
extern "C" __global__ __launch_bounds__(8 * HalvesShape<11>::T) __attribute__((amdgpu_waves_per_eu(4))) void
fg_copy_shape_tile_l11_g8_h_cc(const float2* __restrict__ in, float2* __restrict__ out, TileGeom g) {
    copy_shape_tile_halves<11, 8, true, true>(in, out, g);
}
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void fg_copy_shape_rowpair_n12(
    const float2* __restrict__ in, float2* __restrict__ out, uint64_t pairs, uint32_t log_rows) {
    copy_shape_rowpair_halves<12>(in, out, pairs, log_rows);
}

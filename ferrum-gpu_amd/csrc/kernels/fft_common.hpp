// fft_common.hpp -- device-side building blocks shared by every FFT kernel:
// complex helpers and in-register forward DFTs of size 2, 4, 8 and 16.
//
// Complex values are float2 (x = re, y = im), the interleaved complex64 layout
// of the reference's Complex32 (crates/ferrum-gpu-fft/src/complex.rs:10-53).
// All butterflies compute the forward transform X_k = sum_n x_n W^{nk} with
// W = exp(-2 pi i / R); the inverse is obtained by conjugating on load and on
// store, the same identity the reference applies on the host
// (crates/ferrum-gpu-fft/src/cpu.rs:106-121).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fg {

__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
    return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ float2 cconj(float2 a) { return make_float2(a.x, -a.y); }
__device__ __forceinline__ float2 cscale(float2 a, float s) { return make_float2(a.x * s, a.y * s); }
// a * (-i)
__device__ __forceinline__ float2 cmul_negi(float2 a) { return make_float2(a.y, -a.x); }

// cos/sin of multiples of pi/8 (exact mathematics, not library constants).
constexpr float kC8 = 0.92387953251128675613f;  // cos(pi/8)
constexpr float kS8 = 0.38268343236508977173f;  // sin(pi/8)
constexpr float kR2 = 0.70710678118654752440f;  // cos(pi/4) = sin(pi/4)

template <int R>
struct Dft;

template <>
struct Dft<1> {
    __device__ __forceinline__ static void run(float2*) {}
};

template <>
struct Dft<2> {
    __device__ __forceinline__ static void run(float2* v) {
        float2 a = v[0], b = v[1];
        v[0] = cadd(a, b);
        v[1] = csub(a, b);
    }
};

template <>
struct Dft<4> {
    // X0 = (x0+x2)+(x1+x3); X2 = (x0+x2)-(x1+x3);
    // X1 = (x0-x2) - i(x1-x3); X3 = (x0-x2) + i(x1-x3).
    __device__ __forceinline__ static void run(float2* v) {
        float2 a = cadd(v[0], v[2]), b = csub(v[0], v[2]);
        float2 c = cadd(v[1], v[3]), d = csub(v[1], v[3]);
        v[0] = cadd(a, c);
        v[2] = csub(a, c);
        v[1] = make_float2(b.x + d.y, b.y - d.x);
        v[3] = make_float2(b.x - d.y, b.y + d.x);
    }
};

template <>
struct Dft<8> {
    // Decimation in time: E = DFT4(even), O = DFT4(odd),
    // X_q = E_q + W8^q O_q, X_{q+4} = E_q - W8^q O_q.
    __device__ __forceinline__ static void run(float2* v) {
        float2 e[4] = {v[0], v[2], v[4], v[6]};
        float2 o[4] = {v[1], v[3], v[5], v[7]};
        Dft<4>::run(e);
        Dft<4>::run(o);
        float2 w1 = make_float2(kR2 * (o[1].x + o[1].y), kR2 * (o[1].y - o[1].x));   // W8^1 = (r,-r)
        float2 w2 = cmul_negi(o[2]);                                                  // W8^2 = -i
        float2 w3 = make_float2(kR2 * (o[3].y - o[3].x), -kR2 * (o[3].x + o[3].y));  // W8^3 = (-r,-r)
        v[0] = cadd(e[0], o[0]);
        v[4] = csub(e[0], o[0]);
        v[1] = cadd(e[1], w1);
        v[5] = csub(e[1], w1);
        v[2] = cadd(e[2], w2);
        v[6] = csub(e[2], w2);
        v[3] = cadd(e[3], w3);
        v[7] = csub(e[3], w3);
    }
};

template <>
struct Dft<16> {
    // 16 = 4 x 4: n = 4*n1 + n2, k = k1 + 4*k2.
    //   Y[n2][k1] = DFT4_{n1} x[4 n1 + n2];  Y[n2][k1] *= W16^{n2 k1};
    //   X[k1 + 4 k2] = DFT4_{n2} Y[n2][k1].
    __device__ __forceinline__ static void run(float2* v) {
        float2 y[4][4];
#pragma unroll
        for (int n2 = 0; n2 < 4; ++n2) {
            y[n2][0] = v[n2];
            y[n2][1] = v[4 + n2];
            y[n2][2] = v[8 + n2];
            y[n2][3] = v[12 + n2];
            Dft<4>::run(y[n2]);
        }
        // n2 = 1: W16^1, W16^2, W16^3
        y[1][1] = cmul(y[1][1], make_float2(kC8, -kS8));
        y[1][2] = make_float2(kR2 * (y[1][2].x + y[1][2].y), kR2 * (y[1][2].y - y[1][2].x));
        y[1][3] = cmul(y[1][3], make_float2(kS8, -kC8));
        // n2 = 2: W16^2, W16^4, W16^6
        y[2][1] = make_float2(kR2 * (y[2][1].x + y[2][1].y), kR2 * (y[2][1].y - y[2][1].x));
        y[2][2] = cmul_negi(y[2][2]);
        y[2][3] = make_float2(kR2 * (y[2][3].y - y[2][3].x), -kR2 * (y[2][3].x + y[2][3].y));
        // n2 = 3: W16^3, W16^6, W16^9
        y[3][1] = cmul(y[3][1], make_float2(kS8, -kC8));
        y[3][2] = make_float2(kR2 * (y[3][2].y - y[3][2].x), -kR2 * (y[3][2].x + y[3][2].y));
        y[3][3] = cmul(y[3][3], make_float2(-kC8, kS8));
#pragma unroll
        for (int k1 = 0; k1 < 4; ++k1) {
            float2 z[4] = {y[0][k1], y[1][k1], y[2][k1], y[3][k1]};
            Dft<4>::run(z);
            v[k1] = z[0];
            v[k1 + 4] = z[1];
            v[k1 + 8] = z[2];
            v[k1 + 12] = z[3];
        }
    }
};

// Streaming global access.  Transform data is touched exactly once per pass,
// so loads and stores carry the nontemporal hint: it keeps the stream from
// displacing the twiddle tables in L2 and measurably raises HBM throughput on
// gfx950 (the FFT access shape moves ~6.1 TB/s with it, ~5.5 TB/s without).
typedef float fg_v2f __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float2 load_stream(const float2* p) {
    fg_v2f v = __builtin_nontemporal_load(reinterpret_cast<const fg_v2f*>(p));
    return make_float2(v.x, v.y);
}
__device__ __forceinline__ void store_stream(float2* p, float2 a) {
    fg_v2f v = {a.x, a.y};
    __builtin_nontemporal_store(v, reinterpret_cast<fg_v2f*>(p));
}
__device__ __forceinline__ float load_stream(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void store_stream(float* p, float a) { __builtin_nontemporal_store(a, p); }

// Pass-level cache policy.  A single-pass transform streams (nontemporal) both
// ways.  A multi-pass plan runs chunk by chunk, each chunk small enough for
// the 256 MB Infinity Cache, and keeps its intermediate arrays cached: its
// first pass streams the input in and stores cached, the middle passes load
// and store cached, the last loads cached and streams the output out.  On
// gfx950 a copy whose working set fits the Infinity Cache moved 8.4 TB/s with
// ordinary accesses and 6.3 TB/s with nontemporal ones (which bypass it).
template <bool CACHED>
__device__ __forceinline__ float2 gload(const float2* p) {
    if constexpr (CACHED) return *p;
    else return load_stream(p);
}
template <bool CACHED>
__device__ __forceinline__ void gstore(float2* p, float2 v) {
    if constexpr (CACHED) *p = v;
    else store_stream(p, v);
}

// Global layouts of transform data.  Element i of the flat batch (transform f,
// position p: i = f * N + p) is in[i] in the interleaved complex64 layout (the
// reference's Complex32 arrays), or (re[i], im[i]) in the split layout: two f32
// arrays, the reference's SoA kernels (kernels_body.rs:509-626).
template <bool LOAD_CACHED, bool STORE_CACHED>
struct InterleavedIOT {
    const float2* in;
    float2* out;
    __device__ __forceinline__ float2 load(uint64_t i) const { return gload<LOAD_CACHED>(in + i); }
    __device__ __forceinline__ void store(uint64_t i, float2 v) const { gstore<STORE_CACHED>(out + i, v); }
    // Element row + lane with `row` the same for the whole wave: a scalar base
    // plus a 32-bit lane offset, no 64-bit vector address per access.
    __device__ __forceinline__ float2 load_row(uint64_t row, uint32_t lane) const {
        return gload<LOAD_CACHED>(reinterpret_cast<const float2*>(reinterpret_cast<const char*>(in + row) + lane * 8u));
    }
    __device__ __forceinline__ void store_row(uint64_t row, uint32_t lane, float2 v) const {
        gstore<STORE_CACHED>(reinterpret_cast<float2*>(reinterpret_cast<char*>(out + row) + lane * 8u), v);
    }
};
using InterleavedIO = InterleavedIOT<false, false>;
struct SplitIO {
    const float* in_re;
    const float* in_im;
    float* out_re;
    float* out_im;
    __device__ __forceinline__ float2 load(uint64_t i) const {
        return make_float2(load_stream(in_re + i), load_stream(in_im + i));
    }
    __device__ __forceinline__ void store(uint64_t i, float2 v) const {
        store_stream(out_re + i, v.x);
        store_stream(out_im + i, v.y);
    }
    __device__ __forceinline__ float2 load_row(uint64_t row, uint32_t lane) const {
        const uint32_t b = lane * 4u;
        return make_float2(load_stream(reinterpret_cast<const float*>(reinterpret_cast<const char*>(in_re + row) + b)),
                           load_stream(reinterpret_cast<const float*>(reinterpret_cast<const char*>(in_im + row) + b)));
    }
    __device__ __forceinline__ void store_row(uint64_t row, uint32_t lane, float2 v) const {
        const uint32_t b = lane * 4u;
        store_stream(reinterpret_cast<float*>(reinterpret_cast<char*>(out_re + row) + b), v.x);
        store_stream(reinterpret_cast<float*>(reinterpret_cast<char*>(out_im + row) + b), v.y);
    }
};

// Lock-step start of kernels that hold at most two workgroups per CU.
// Every CU starts its first workgroups together, so with one or two per CU
// all CUs load, transform and store in step, round after round: HBM idles
// while every CU transforms, and the CUs wait together on memory.  Delaying
// the first round's workgroups by 0, 1, ..., 15 us (by their per-XCD index:
// workgroup b runs on XCD b % 8 as its (b / 8)-th) puts the CUs out of step
// for the whole launch, since each CU's next workgroup starts when its
// previous one ends.  Measured on gfx950 at 512 MiB per launch (us): 32768-
// point transforms (one 1024-thread workgroup per CU) 265 -> 247, 16384-point
// ones (two per CU) 199 -> 193, 128 x 128 images (two per CU) 217 -> 203;
// kernels with four or more workgroups per CU lost (N = 1024: 169 -> 182,
// N = 8192: 181 -> 185), as did the multi-pass tiles, whose chained launches
// are out of step already.  Only grids of at least two full rounds wait, so a
// batch that fills the GPU once or less runs without delay.  The wait is a
// bounded poll of the 100 MHz constant clock (s_memrealtime) with s_sleep.
constexpr unsigned kGpuCus = 256;          // MI355X: 8 XCDs x 32 CUs
constexpr long long kStaggerTicks = 100;   // 1 us per phase at the 100 MHz wall clock
constexpr unsigned kStaggerPhases = 16;

template <int LDS_BYTES, int THREADS>
__device__ __forceinline__ void stagger_lockstep_start() {
    // workgroups per CU: the LDS (160 KB) and, at up to 128 VGPRs, 16 waves
    constexpr int by_lds = 163840 / LDS_BYTES, by_waves = 1024 / THREADS;
    constexpr int per_cu = by_lds < by_waves ? by_lds : by_waves;
    if constexpr (per_cu >= 1 && per_cu <= 2) {
        constexpr unsigned first = kGpuCus * per_cu;
        if (gridDim.x >= 2 * first && blockIdx.x < first) {
            const long long wait = kStaggerTicks * (long long)((blockIdx.x >> 3) % kStaggerPhases);
            const long long t0 = wall_clock64();
            while (wall_clock64() - t0 < wait) __builtin_amdgcn_s_sleep(4);
        }
    }
}

// Wave-scope ordering of LDS traffic: a wave's LDS operations execute in
// program order, so a compiler-level barrier plus wavefront-scope fences is
// enough between one wave's LDS writes and its own later reads.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace fg

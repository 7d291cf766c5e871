// pointwise.hpp -- elementwise complex kernels: the reference's cmul_interleaved,
// cmul_split, deinterleave and interleave (kernels_body.rs:1612-1672).
//
// Each is one read and one write of every byte (HBM-bound).  A thread takes W
// consecutive elements per grid-stride step.  The vector kernels use one
// 16-byte access per thread on each interleaved complex64 stream (W = 2) and
// per f32 stream of cmul_split (W = 4), so consecutive lanes touch consecutive
// 16-byte pieces and one wave instruction covers 1 KB; f32 streams of
// deinterleave / interleave take 8 bytes per lane.  The host picks them when
// every pointer is 16-byte aligned.  W = 1 goes element by element for any
// complex64 / f32 alignment.  The complex product is evaluated as written,
// re = ar*br - ai*bi, im = ar*bi + ai*br, with no fused multiply-add, so
// results equal the reference's f32 arithmetic (Rust does not contract) bit
// for bit.
#pragma once

#include "fft_common.hpp"

namespace fg {

typedef float fg_v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ fg_v4f load_stream4(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const fg_v4f*>(p));
}
__device__ __forceinline__ void store_stream4(float* p, fg_v4f v) {
    __builtin_nontemporal_store(v, reinterpret_cast<fg_v4f*>(p));
}
__device__ __forceinline__ fg_v2f load_stream2(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const fg_v2f*>(p));
}
__device__ __forceinline__ void store_stream2(float* p, fg_v2f v) {
    __builtin_nontemporal_store(v, reinterpret_cast<fg_v2f*>(p));
}

__device__ __forceinline__ float mul_re(float ar, float ai, float br, float bi) {
#pragma clang fp contract(off)
    return ar * br - ai * bi;
}
__device__ __forceinline__ float mul_im(float ar, float ai, float br, float bi) {
#pragma clang fp contract(off)
    return ar * bi + ai * br;
}

// Grid-stride loop over chunks of W elements of [0, n): full chunks go to
// vec(i0) when W > 1, everything else element by element to one(i).
template <int W, class Vec, class One>
__device__ __forceinline__ void for_chunks(uint64_t n, Vec vec, One one) {
    const uint64_t chunks = (n + W - 1) / W;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t c = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += stride) {
        const uint64_t i0 = c * W;
        if (W > 1 && i0 + W <= n) {
            vec(i0);
        } else {
#pragma unroll
            for (int j = 0; j < W; ++j)
                if (i0 + j < n) one(i0 + j);
        }
    }
}

// out[i] = a[i] * b[i], interleaved complex64 (cmul_interleaved).
template <int W>
__device__ __forceinline__ void cmul_c64_body(const float* a, const float* b, float* out, uint64_t n) {
    static_assert(W == 1 || W == 2, "the vector path below moves exactly W elements");
    for_chunks<W>(
        n,
        [&](uint64_t i0) {  // W = 2: two complex per 16-byte vector
            const fg_v4f x = load_stream4(a + 2 * i0);
            const fg_v4f y = load_stream4(b + 2 * i0);
            const fg_v4f r = {mul_re(x.x, x.y, y.x, y.y), mul_im(x.x, x.y, y.x, y.y),
                              mul_re(x.z, x.w, y.z, y.w), mul_im(x.z, x.w, y.z, y.w)};
            store_stream4(out + 2 * i0, r);
        },
        [&](uint64_t i) {
            const float ar = load_stream(a + 2 * i), ai = load_stream(a + 2 * i + 1);
            const float br = load_stream(b + 2 * i), bi = load_stream(b + 2 * i + 1);
            store_stream(out + 2 * i, mul_re(ar, ai, br, bi));
            store_stream(out + 2 * i + 1, mul_im(ar, ai, br, bi));
        });
}

// (o_re, o_im)[i] = (a_re, a_im)[i] * (b_re, b_im)[i], split layout (cmul_split).
template <int W>
__device__ __forceinline__ void cmul_split_body(const float* a_re, const float* a_im, const float* b_re,
                                                const float* b_im, float* o_re, float* o_im, uint64_t n) {
    static_assert(W == 1 || W == 4, "the vector path below moves exactly W elements");
    for_chunks<W>(
        n,
        [&](uint64_t i0) {  // W = 4: four f32 per 16-byte vector
            const fg_v4f ar = load_stream4(a_re + i0), ai = load_stream4(a_im + i0);
            const fg_v4f br = load_stream4(b_re + i0), bi = load_stream4(b_im + i0);
            fg_v4f r, m;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                r[j] = mul_re(ar[j], ai[j], br[j], bi[j]);
                m[j] = mul_im(ar[j], ai[j], br[j], bi[j]);
            }
            store_stream4(o_re + i0, r);
            store_stream4(o_im + i0, m);
        },
        [&](uint64_t i) {
            const float ar = load_stream(a_re + i), ai = load_stream(a_im + i);
            const float br = load_stream(b_re + i), bi = load_stream(b_im + i);
            store_stream(o_re + i, mul_re(ar, ai, br, bi));
            store_stream(o_im + i, mul_im(ar, ai, br, bi));
        });
}

// re[i], im[i] = in[i] (deinterleave).
template <int W>
__device__ __forceinline__ void deinterleave_body(const float* in, float* re, float* im, uint64_t n) {
    static_assert(W == 1 || W == 2, "the vector path below moves exactly W elements");
    for_chunks<W>(
        n,
        [&](uint64_t i0) {  // W = 2
            const fg_v4f x = load_stream4(in + 2 * i0);
            store_stream2(re + i0, fg_v2f{x.x, x.z});
            store_stream2(im + i0, fg_v2f{x.y, x.w});
        },
        [&](uint64_t i) {
            store_stream(re + i, load_stream(in + 2 * i));
            store_stream(im + i, load_stream(in + 2 * i + 1));
        });
}

// out[i] = (re[i], im[i]) (interleave).
template <int W>
__device__ __forceinline__ void interleave_body(const float* re, const float* im, float* out, uint64_t n) {
    static_assert(W == 1 || W == 2, "the vector path below moves exactly W elements");
    for_chunks<W>(
        n,
        [&](uint64_t i0) {  // W = 2
            const fg_v2f r = load_stream2(re + i0), m = load_stream2(im + i0);
            store_stream4(out + 2 * i0, fg_v4f{r.x, m.x, r.y, m.y});
        },
        [&](uint64_t i) {
            store_stream(out + 2 * i, load_stream(re + i));
            store_stream(out + 2 * i + 1, load_stream(im + i));
        });
}

}  // namespace fg

// fill.hpp -- seeded synthetic complex64 data, generated in place on the device.
//
// Counter-based: float j of the output (j = 2i for the real part of element i,
// 2i + 1 for the imaginary part) depends only on (seed, j), so any grid gives
// the same array, and the CPU restatement reproduces it.
//   z(j)    = splitmix64 output for state seed + (j + 1) * 0x9E3779B97F4A7C15
//             (Steele, Lea and Flood, "Fast splittable pseudorandom number
//             generators", OOPSLA 2014; the mixing constants of Vigna's
//             public-domain splitmix64.c)
//   uniform: u = z(j) >> 40 (24 bits), value = u * 2^-23 - 1, exactly
//            representable in f32, in [-1, 1)
//   normal:  Box-Muller on the pair (z(2i), z(2i+1)) in f64:
//            u1 = ((z(2i) >> 11) + 1) * 2^-53 in (0, 1], u2 = (z(2i+1) >> 11) * 2^-53,
//            r = sqrt(-2 ln u1), (re, im) = (r cos 2 pi u2, r sin 2 pi u2), rounded to f32
#pragma once

#include <stdint.h>

namespace fg {

__host__ __device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t j) {
    uint64_t z = seed + (j + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float uniform_at(uint64_t seed, uint64_t j) {
    const uint32_t u = (uint32_t)(splitmix64_at(seed, j) >> 40);
    return (float)u * 0x1p-23f - 1.0f;
}

__device__ __forceinline__ float2 normal_pair_at(uint64_t seed, uint64_t i) {
    const double u1 = (double)((splitmix64_at(seed, 2 * i) >> 11) + 1) * 0x1p-53;
    const double u2 = (double)(splitmix64_at(seed, 2 * i + 1) >> 11) * 0x1p-53;
    const double r = sqrt(-2.0 * log(u1));
    const double a = 6.283185307179586476925286766559 * u2;
    return make_float2((float)(r * cos(a)), (float)(r * sin(a)));
}

// n complex elements; normal != 0 selects the normal distribution.
__device__ __forceinline__ void fill_c64_body(float2* out, uint64_t n, uint64_t seed, uint32_t normal) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float2 v = normal ? normal_pair_at(seed, i)
                                : make_float2(uniform_at(seed, 2 * i), uniform_at(seed, 2 * i + 1));
        out[i] = v;
    }
}

}  // namespace fg

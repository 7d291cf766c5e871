// fft_tile.hpp -- one pass of a multi-pass FFT: G independent transforms of
// length L = 2^LOGL ("columns") per workgroup, read and written through
// arbitrary (column, element) strides, with the four-step twiddle fused into
// the store.
//
// Used for 1D lengths above 4096 (N = N_1 * N_2 [* N_3], every pass moves the
// whole array once) and for the column FFT of 2D images.  The column index is
// the lane index within a wave, so every global access of a wave covers G
// adjacent columns -- G*8 contiguous bytes per element row -- and every LDS
// access of a wave touches one element position of G columns (contiguous in
// the [position][column] LDS layout, so no bank conflicts).
//
// Tile addressing (TileGeom): tile b = t0 + t0n*(t1 + t1n*t2) has input base
// t0*is0 + t1*is1 + t2*is2 and output base t0*os0 + t1*os1 + t2*os2; element n of
// column c is at in_base + c*ics + n*ies, output k of column c at
// out_base + c*ocs + k*oes.  If log_m != 0 the output is multiplied by
// W_M^(r*k), M = 2^log_m, r = twc*c + tw0*t0 + tw1*t1 (the four-step twiddle of
// crates/ferrum-gpu-fft/src/warp_fft.rs:138-143, generalised to any pass).
#pragma once
#include "fft_stockham.hpp"
#include "tile_geom.h"

namespace fg {

// W_M^e for M = 2^log_m <= 2^24 from two 4096-entry tables:
// big[j] = W_4096^j and big[4096 + j] = W_{2^24}^j, so
// W_{2^24}^e' = big[e' >> 12] * big[4096 + (e' & 4095)] with e' = e * 2^(24 - log_m).
__device__ __forceinline__ float2 big_twiddle(const float2* __restrict__ big, uint64_t e, uint32_t log_m) {
    const uint32_t ep = (uint32_t)((e << (24 - log_m)) & 0xFFFFFFull);
    return cmul(big[ep >> 12], big[4096 + (ep & 4095)]);
}

// Multiplies x[m] (output position k = q + T*m) by W_M^(r*k).  TWREC = false
// looks every factor up (2 table reads + 1 multiply each); TWREC = true looks
// up W^(r*q) and W^(r*T) once and forms the rest as W^(r*q) * (W^(r*T))^m by
// repeated multiplication (error grows by about one rounding per step, ~1e-6
// relative after 16 steps).
template <int E, int T, bool TWREC>
__device__ __forceinline__ void apply_pass_twiddle(float2* x, const float2* __restrict__ big, uint64_t r, int q,
                                                   uint32_t log_m) {
    if constexpr (TWREC) {
        float2 w = big_twiddle(big, r * (uint64_t)q, log_m);
        const float2 step = big_twiddle(big, r * (uint64_t)T, log_m);
#pragma unroll
        for (int m = 0; m < E; ++m) {
            x[m] = cmul(x[m], w);
            if (m + 1 < E) w = cmul(w, step);
        }
    } else {
#pragma unroll
        for (int m = 0; m < E; ++m) x[m] = cmul(x[m], big_twiddle(big, r * (uint64_t)(q + T * m), log_m));
    }
}

// LDS layout of a tile, [position][column].  G >= 16: row pitch G + 1 (one
// pad column keeps the row-wise staging writes, lanes along positions, off a
// single bank).  G < 16 (long columns, 4 or 8 per tile): pitch G with one pad
// row per 16 positions (lds_pos), which spreads the stride-16 scatter of a
// radix-16 stage over the banks and keeps a 4 x 4096 tile at 136 KB (a pad
// column would take all 160 KB of the CU's LDS).
template <int LOGL, int G>
struct TileLayout {
    static constexpr bool PADPOS = G < 16;
    static constexpr int N = 1 << LOGL;
    static constexpr int ELEMS = PADPOS ? (N + N / 16) * G : N * (G + 1);
    __device__ __forceinline__ static int at(int pos, int c) {
        if constexpr (PADPOS) return lds_pos<>(pos) * G + c;
        else return pos * (G + 1) + c;
    }
    // at(pos + D, c) - at(pos, c) for a step D that is a multiple of 16 (any D
    // without position padding): lds_pos(p + 16u) = lds_pos(p) + 17u.
    template <int D>
    static constexpr int step() {
        static_assert(!PADPOS || D % 16 == 0, "position-padded steps must be multiples of 16");
        return PADPOS ? (D + D / 16) * G : D * (G + 1);
    }
};

// Stockham stages on a [position][column] LDS tile: thread (c, q) holds
// positions q + T*m of column c.  LDS addresses are a per-thread base plus
// compile-time offsets (ds_read / ds_write immediates) wherever the layout
// allows.
template <int LOGL, int LOGE, int G, int S>
struct TileStages {
    using Sh = StockhamShape<LOGL, LOGE>;
    using Lay = TileLayout<LOGL, G>;
    __device__ __forceinline__ static void run(float2* x, int q, int c, const float2* __restrict__ tw,
                                               float2* __restrict__ lds) {
        stockham_stage_regs<LOGL, LOGE, S>(x, q, tw);
        if constexpr (S + 1 < Sh::NSTAGES) {
            constexpr int LOGR = (S < Sh::NFULL) ? LOGE : Sh::REM;
            constexpr int NB = Sh::E >> LOGR;
            constexpr int R = 1 << LOGR;
            constexpr int L = 1 << (S * LOGE);
            __syncthreads();  // previous readers of the tile are done
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                if constexpr (Lay::PADPOS && L == 1 && R == 16) {
                    // dst = 16*b + r, r < 16: lds_pos = 17*b + r
                    float2* base = lds + Lay::at(16 * (q + Sh::T * i), c);
#pragma unroll
                    for (int r = 0; r < R; ++r) base[r * G] = x[i + NB * r];
                } else if constexpr (!Lay::PADPOS || L % 16 == 0) {
                    // dst = dst(i, 0) + r*L
                    float2* base = lds + Lay::at(stockham_dst<LOGL, LOGE, S>(q, i, 0), c);
#pragma unroll
                    for (int r = 0; r < R; ++r) base[r * Lay::template step<L>()] = x[i + NB * r];
                } else {
#pragma unroll
                    for (int r = 0; r < R; ++r) lds[Lay::at(stockham_dst<LOGL, LOGE, S>(q, i, r), c)] = x[i + NB * r];
                }
            }
            __syncthreads();
            if constexpr (!Lay::PADPOS || Sh::T % 16 == 0) {
                const float2* base = lds + Lay::at(q, c);
#pragma unroll
                for (int m = 0; m < Sh::E; ++m) x[m] = base[m * Lay::template step<Sh::T>()];
            } else {
#pragma unroll
                for (int m = 0; m < Sh::E; ++m) x[m] = lds[Lay::at(q + Sh::T * m, c)];
            }
            TileStages<LOGL, LOGE, G, S + 1>::run(x, q, c, tw, lds);
        }
    }
};

// This workgroup's tile: its (t0, t1) indices and input / output bases.
struct TileCoords {
    uint32_t t0, t1;
    uint64_t ib, ob;
};

template <int G>
__device__ __forceinline__ TileCoords tile_coords(const TileGeom& g) {
    uint32_t b = blockIdx.x;
    if (g.remap == FG_TILE_ORDER_XCD_RANGES) {
        // XCD x (blockIdx % 8) takes the contiguous tile range
        // [x * grid/8, (x + 1) * grid/8): narrow tiles (4 or 8 columns, 32 or
        // 64 bytes of a 128-byte line) then share each line fill of their
        // XCD's L2 instead of each XCD fetching it (host: grid % 8 == 0).
        b = (b & 7u) * (gridDim.x >> 3) + (b >> 3);
    } else if (g.remap == FG_TILE_ORDER_LINE_GROUPS) {
        // the S tiles of a line group on one XCD, neighbouring groups on
        // neighbouring XCDs (host: grid % (8 S) == 0)
        constexpr uint32_t S = G < 16 ? 16 / G : 1;
        const uint32_t j = b >> 3;
        b = ((j / S) * 8u + (b & 7u)) * S + j % S;
    }
    TileCoords tc;
    tc.t0 = b % g.t0n;
    b /= g.t0n;
    tc.t1 = b % g.t1n;
    const uint32_t t2 = b / g.t1n;
    tc.ib = tc.t0 * g.is0 + tc.t1 * g.is1 + (uint64_t)t2 * g.is2;
    tc.ob = tc.t0 * g.os0 + tc.t1 * g.os1 + (uint64_t)t2 * g.os2;
    return tc;
}

// ROWWISE: input elements of a column are contiguous (ies == 1, rows of a
// matrix), so loads run along elements and the tile is transposed into LDS
// first; otherwise columns are contiguous (ics == 1) and each thread loads its
// own Stockham positions straight into VGPRs.  Output always has ocs == 1.
// LOAD_CACHED / STORE_CACHED select the pass's cache policy (gload/gstore).
// CONJ: the body reads the inverse's conjugation flags; forward passes
// (flags == 0) run the CONJ = false body, which has no per-element selects.
// Global addresses are a wave-uniform row base (scalar registers) plus a
// 32-bit per-lane byte offset, so each access costs no 64-bit vector
// arithmetic; a tile's offsets stay below 2^32 bytes (one transform or image
// spans at most 128 MiB).
template <int LOGL, int LOGE, int G, bool ROWWISE, bool TWREC, bool LOAD_CACHED, bool STORE_CACHED, bool CONJ>
__device__ __forceinline__ void fft_tile_body(const float2* __restrict__ in, float2* __restrict__ out,
                                              const float2* __restrict__ tw, const float2* __restrict__ big,
                                              const TileGeom& g, float2* __restrict__ lds) {
    using Sh = StockhamShape<LOGL, LOGE>;
    using Lay = TileLayout<LOGL, G>;
    constexpr int THREADS = G * Sh::T;

    const int tid = threadIdx.x;
    const int c = tid % G;
    const int q = tid / G;
    const TileCoords tc = tile_coords<G>(g);
    const uint32_t t0 = tc.t0, t1 = tc.t1;
    const char* in_tile = reinterpret_cast<const char*>(in + tc.ib);
    char* out_tile = reinterpret_cast<char*>(out + tc.ob);

    float2 x[Sh::E];
    if constexpr (ROWWISE) {
        // Coalesced along each row: linear element li -> (column li / L, position li % L).
#pragma unroll
        for (int m = 0; m < Sh::E; ++m) {
            const int li = tid + THREADS * m;
            const int cc = li >> LOGL;
            const int n = li & (Sh::N - 1);
            const uint32_t off = (uint32_t)((cc * g.ics + n) * sizeof(float2));
            lds[Lay::at(n, cc)] = gload<LOAD_CACHED>(reinterpret_cast<const float2*>(in_tile + off));
        }
        __syncthreads();
        if constexpr (!Lay::PADPOS || Sh::T % 16 == 0) {
            const float2* base = lds + Lay::at(q, c);
#pragma unroll
            for (int m = 0; m < Sh::E; ++m) x[m] = base[m * Lay::template step<Sh::T>()];
        } else {
#pragma unroll
            for (int m = 0; m < Sh::E; ++m) x[m] = lds[Lay::at(q + Sh::T * m, c)];
        }
    } else {
        const uint32_t lane_off = (uint32_t)((c + (uint64_t)q * g.ies) * sizeof(float2));
        const uint64_t row_step = (uint64_t)Sh::T * g.ies * sizeof(float2);
#pragma unroll
        for (int m = 0; m < Sh::E; ++m)
            x[m] = gload<LOAD_CACHED>(reinterpret_cast<const float2*>(in_tile + m * row_step + lane_off));
    }
    if constexpr (CONJ) {
        if (g.flags & FG_PASS_CONJ_IN) {
#pragma unroll
            for (int m = 0; m < Sh::E; ++m) x[m] = cconj(x[m]);
        }
    }
    TileStages<LOGL, LOGE, G, 0>::run(x, q, c, tw, lds);

    if (g.log_m != 0) {
        const uint64_t r = (uint64_t)g.twc * c + (uint64_t)g.tw0 * t0 + (uint64_t)g.tw1 * t1;
        apply_pass_twiddle<Sh::E, Sh::T, TWREC>(x, big, r, q, g.log_m);
    }
    const uint32_t lane_off = (uint32_t)((c + (uint64_t)q * g.oes) * sizeof(float2));
    const uint64_t row_step = (uint64_t)Sh::T * g.oes * sizeof(float2);
    const bool cs = CONJ && (g.flags & FG_PASS_CONJ_SCALE_OUT) != 0;
#pragma unroll
    for (int m = 0; m < Sh::E; ++m) {
        float2 v = x[m];
        if constexpr (CONJ) {
            if (cs) v = cscale(cconj(v), g.scale);
        }
        gstore<STORE_CACHED>(reinterpret_cast<float2*>(out_tile + m * row_step + lane_off), v);
    }
}

// ---------------------------------------------------------------------------
// Column pass with the Stockham exchanges in halves: the 32-element stages of
// fft_stockham.hpp (HalvesShape, halves_stage) on every column of the tile,
// each exchange in two rounds through an LDS tile of L/2 positions.
//  * The first pass of a 1D multi-pass plan (which reads the caller's input
//    from HBM), wide tiles: half the LDS of the 16-element tile, four 33 KB
//    workgroups per CU instead of two for 128 / 256 points (64 / 32
//    columns), two 68 KB ones instead of one for 1024 (16 columns), so more
//    of a CU's tiles are loading while others compute.
//  * The cache-resident 1D middle pass of 256 points: 16 columns (whole
//    128-byte lines) in 17 KB.
//  * 1D last passes (ROWWISE: rows in, transposed store) of 256 points in
//    32-row tiles and of 512 / 1024 points in 16-row tiles: every row load
//    is issued at once and each half of the positions is transposed through
//    the same L/2-position LDS tile, so 33 / 34 / 68 KB instead of the
//    16-element tile's 66 / 68 / 136 KB.
//  * 2D column passes of 1024 .. 4096 points, narrow tiles (8 columns, the
//    position-padded layout): twice the columns of the 16-element tile in the
//    same LDS (136 KB at 4096 points), so 64-byte row pieces instead of 32.

// at(d + q*L, c) - at(d, c) for the outputs q of a halves butterfly.  L = 1
// (stage 0, radix 16) on a position-padded layout: d = 16 b - HALF h is a
// multiple of 16, so lds_pos(d + q) = lds_pos(d) + q for q < 16.
template <class Lay, int L, int G>
constexpr int halves_scatter_step() {
    if constexpr (Lay::PADPOS && L == 1) return G;
    else return Lay::template step<L>();
}

// Exchange after stage S: x[m] = the element at position t + T*m.
template <int LOGL, int S, int G>
__device__ __forceinline__ void halves_exchange(const float2* y, float2* x, int t, int c, float2* __restrict__ lds) {
    using H = HalvesShape<LOGL>;
    using St = HalvesStage<LOGL, S>;
    using Lay = TileLayout<LOGL - 1, G>;
    static_assert(!Lay::PADPOS || St::L > 1 || St::R == 16, "position-padded scatter of stage 0 needs radix 16");
    static_assert(H::T % 16 == 0 || !Lay::PADPOS, "position-padded reads step by T, a multiple of 16");
    constexpr int QSTEP = halves_scatter_step<Lay, St::L, G>();
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (S > 0 || h > 0) __syncthreads();  // the previous round's readers are done
#pragma unroll
        for (int ii = 0; ii < St::NB / 2; ++ii) {
            const int i = h * (St::NB / 2) + ii;
            const int b = t + H::T * i;
            const int d0 = (b >> (4 * S)) * St::L * St::R + (b & (St::L - 1)) - H::HALF * h;
            float2* wbase = lds + Lay::at(d0, c);
#pragma unroll
            for (int q = 0; q < St::R; ++q) wbase[q * QSTEP] = y[i + St::NB * q];
        }
        __syncthreads();
        const float2* rbase = lds + Lay::at(t, c);
#pragma unroll
        for (int m = 0; m < H::E / 2; ++m) x[(H::E / 2) * h + m] = rbase[m * Lay::template step<H::T>()];
    }
}

template <int LOGL, int S, int G>
struct HalvesStages {
    __device__ __forceinline__ static void run(float2* x, float2* y, int t, int c, const float2* __restrict__ tw,
                                               float2* __restrict__ lds) {
        halves_stage<LOGL, S>(x, y, t, tw);
        if constexpr (S + 1 < HalvesShape<LOGL>::NSTAGES) {
            halves_exchange<LOGL, S, G>(y, x, t, c, lds);
            HalvesStages<LOGL, S + 1, G>::run(x, y, t, c, tw, lds);
        }
    }
};

template <int LOGL, int G, bool LOAD_CACHED, bool STORE_CACHED, bool CONJ, bool ROWWISE>
__device__ __forceinline__ void fft_tile_halves_body(const float2* __restrict__ in, float2* __restrict__ out,
                                                     const float2* __restrict__ tw, const float2* __restrict__ big,
                                                     const TileGeom& g, float2* __restrict__ lds) {
    using H = HalvesShape<LOGL>;
    const int tid = threadIdx.x;
    const int c = tid % G;
    const int t = tid / G;
    const TileCoords tc = tile_coords<G>(g);
    const char* in_tile = reinterpret_cast<const char*>(in + tc.ib);
    char* out_tile = reinterpret_cast<char*>(out + tc.ob);

    float2 x[H::E], y[H::E];
    if constexpr (ROWWISE) {
        // Rows contiguous (ies == 1): every load of the tile is issued at
        // once, coalesced along the rows (y[m]: half m / (E/2) of the
        // positions, linear element li -> row li / HALF, position li % HALF),
        // then each half is transposed through the LDS tile into the
        // Stockham positions t + T m of column c.
        using Lay = TileLayout<LOGL - 1, G>;
        constexpr int THREADS = G * H::T;
        static_assert(G * H::HALF == THREADS * (H::E / 2), "one half of the tile per E/2 loads");
#pragma unroll
        for (int m = 0; m < H::E; ++m) {
            const int h = m / (H::E / 2);
            const int li = tid + THREADS * (m % (H::E / 2));
            const int cc = li >> (LOGL - 1);
            const int n = li & (H::HALF - 1);
            const uint32_t off = (uint32_t)((cc * g.ics + H::HALF * h + n) * sizeof(float2));
            y[m] = gload<LOAD_CACHED>(reinterpret_cast<const float2*>(in_tile + off));
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (h > 0) __syncthreads();  // the previous half's readers are done
#pragma unroll
            for (int m = 0; m < H::E / 2; ++m) {
                const int li = tid + THREADS * m;
                lds[Lay::at(li & (H::HALF - 1), li >> (LOGL - 1))] = y[(H::E / 2) * h + m];
            }
            __syncthreads();
            const float2* rbase = lds + Lay::at(t, c);
#pragma unroll
            for (int m = 0; m < H::E / 2; ++m) x[(H::E / 2) * h + m] = rbase[m * Lay::template step<H::T>()];
        }
        __syncthreads();  // the first exchange writes the LDS tile again
    } else {
        const uint32_t lane_off = (uint32_t)((c + (uint64_t)t * g.ies) * sizeof(float2));
        const uint64_t row_step = (uint64_t)H::T * g.ies * sizeof(float2);
#pragma unroll
        for (int m = 0; m < H::E; ++m)
            x[m] = gload<LOAD_CACHED>(reinterpret_cast<const float2*>(in_tile + m * row_step + lane_off));
    }
    if constexpr (CONJ) {
        if (g.flags & FG_PASS_CONJ_IN) {
#pragma unroll
            for (int m = 0; m < H::E; ++m) x[m] = cconj(x[m]);
        }
    }
    HalvesStages<LOGL, 0, G>::run(x, y, t, c, tw, lds);
    if (g.log_m != 0) {
        // Four-step twiddle W^(r*(t + T*m)) by one 32-step recurrence (about
        // 2e-6 relative at its end, 1e-4 is the gate); restarting it at m = 16,
        // from two more table reads or from four squarings of the step,
        // measured 1.7-2.4 us slower per 128 MiB pass.
        const uint64_t r = (uint64_t)g.twc * c + (uint64_t)g.tw0 * tc.t0 + (uint64_t)g.tw1 * tc.t1;
        apply_pass_twiddle<H::E, H::T, true>(y, big, r, t, g.log_m);
    }
    const uint32_t lane_off = (uint32_t)((c + (uint64_t)t * g.oes) * sizeof(float2));
    const uint64_t row_step = (uint64_t)H::T * g.oes * sizeof(float2);
    const bool cs = CONJ && (g.flags & FG_PASS_CONJ_SCALE_OUT) != 0;
#pragma unroll
    for (int m = 0; m < H::E; ++m) {
        float2 v = y[m];
        if constexpr (CONJ) {
            if (cs) v = cscale(cconj(v), g.scale);
        }
        gstore<STORE_CACHED>(reinterpret_cast<float2*>(out_tile + m * row_step + lane_off), v);
    }
}

template <int LOGL, int G, bool LOAD_CACHED, bool STORE_CACHED, bool ROWWISE = false>
__device__ __forceinline__ void fft_tile_halves_pass(const float2* __restrict__ in, float2* __restrict__ out,
                                                     const float2* __restrict__ tw, const float2* __restrict__ big,
                                                     const TileGeom& g) {
    __shared__ float2 lds[TileLayout<LOGL - 1, G>::ELEMS];
    if (g.flags)
        fft_tile_halves_body<LOGL, G, LOAD_CACHED, STORE_CACHED, true, ROWWISE>(in, out, tw, big, g, lds);
    else
        fft_tile_halves_body<LOGL, G, LOAD_CACHED, STORE_CACHED, false, ROWWISE>(in, out, tw, big, g, lds);
}

// One pass: a forward body and one that applies the inverse's conjugations.
template <int LOGL, int LOGE, int G, bool ROWWISE, bool TWREC, bool LOAD_CACHED, bool STORE_CACHED>
__device__ __forceinline__ void fft_tile_pass(const float2* __restrict__ in, float2* __restrict__ out,
                                              const float2* __restrict__ tw, const float2* __restrict__ big,
                                              const TileGeom& g) {
    __shared__ float2 lds[TileLayout<LOGL, G>::ELEMS];
    if (g.flags)
        fft_tile_body<LOGL, LOGE, G, ROWWISE, TWREC, LOAD_CACHED, STORE_CACHED, true>(in, out, tw, big, g, lds);
    else
        fft_tile_body<LOGL, LOGE, G, ROWWISE, TWREC, LOAD_CACHED, STORE_CACHED, false>(in, out, tw, big, g, lds);
}

}  // namespace fg

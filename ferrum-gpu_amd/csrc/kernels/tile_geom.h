/* tile_geom.h -- kernel-argument structs shared by the host runtime (g++) and
 * the gfx950 kernels (hipcc).  Plain C types only, so both compilers lay them
 * out identically. */
#ifndef FG_TILE_GEOM_H
#define FG_TILE_GEOM_H

#include <stdint.h>

#ifdef __cplusplus
namespace fg {
#endif

/* Per-pass flags (Stockham and tile kernels alike). */
#define FG_PASS_CONJ_IN 1u        /* conjugate every element on load */
#define FG_PASS_CONJ_SCALE_OUT 2u /* conjugate, then multiply by `scale`, on store */

/* Tile orders of narrow tiles (G < 16 columns: 128 / (8 G) tiles share each
 * 128-byte line).  Workgroups are dealt round-robin over the 8 XCDs, so
 * workgroup b runs on XCD b % 8 as that XCD's (b / 8)-th.
 *   XCD_RANGES: XCD x takes the contiguous tile range [x grid/8, (x+1) grid/8)
 *     (grid a multiple of 8);
 *   LINE_GROUPS: the groups of s = 16 / G tiles that share lines are dealt
 *     round-robin over the XCDs: XCD x's j-th workgroup takes tile
 *     s (8 (j / s) + x) + j mod s (grid a multiple of 8 s), so the XCDs work
 *     on neighbouring line groups at the same time. */
#define FG_TILE_ORDER_XCD_RANGES 1u
#define FG_TILE_ORDER_LINE_GROUPS 2u

/* Addressing of one multi-pass tile pass (see fft_tile.hpp). */
typedef struct TileGeom {
    uint64_t is0, is1, is2; /* input base = t0*is0 + t1*is1 + t2*is2 */
    uint64_t os0, os1, os2; /* output base = t0*os0 + t1*os1 + t2*os2 */
    uint64_t ics, ies;      /* input column / element stride (complex elements) */
    uint64_t ocs, oes;      /* output column / element stride */
    uint32_t t0n, t1n;      /* tile counts along t0 and t1 (t2 takes the rest) */
    uint32_t twc, tw0, tw1; /* four-step twiddle digit r = twc*c + tw0*t0 + tw1*t1 */
    uint32_t log_m;         /* twiddle W_M^(r*k), M = 2^log_m; 0 = none */
    uint32_t flags;         /* FG_PASS_* */
    float scale;
    uint32_t remap;         /* tile order (fft_tile.hpp, tile_coords): 0 natural, FG_TILE_ORDER_* */
} TileGeom;

/* One-pass 2D FFT of images of 2^lr x 2^lc <= 16384 points: up to 1024
 * points (fft_2d_small.hpp) 2^FG_SMALL2D_LOGE(lr, lc) = 8 elements per thread
 * and FG_SMALL2D_FPI(lr, lc) images per workgroup (256 threads, or one image
 * when it needs more); 2048 to 16384 points (fft_2d_halves.hpp) one image
 * per workgroup of N/32 threads with 32 elements each.  FG_SMALL2D_LOGE also
 * names the stage tables' radix list: (8, ..., r) up to 1024 points,
 * (16, ..., r) above. */
#define FG_SMALL2D_MAX_LOG 14
#define FG_SMALL2D_HALVES_LOG 11
#define FG_SMALL2D_LOGE(lr, lc) (((lr) + (lc)) >= FG_SMALL2D_HALVES_LOG ? 4 : 3)
#define FG_SMALL2D_TPI(lr, lc) \
    (((lr) + (lc)) >= FG_SMALL2D_HALVES_LOG ? (1 << ((lr) + (lc))) / 32 : (1 << ((lr) + (lc))) >> FG_SMALL2D_LOGE(lr, lc))
#define FG_SMALL2D_FPI(lr, lc) \
    (((lr) + (lc)) >= FG_SMALL2D_HALVES_LOG || FG_SMALL2D_TPI(lr, lc) >= 256 ? 1 : 256 / FG_SMALL2D_TPI(lr, lc))
#define FG_SMALL2D_BLOCK(lr, lc) (FG_SMALL2D_FPI(lr, lc) * FG_SMALL2D_TPI(lr, lc))

#ifdef __cplusplus
}  // namespace fg
#endif
#endif

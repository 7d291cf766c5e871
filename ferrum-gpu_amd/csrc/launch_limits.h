/* launch_limits.h -- how much one kernel launch can cover, in plain C so the
 * host runtime (g++) and the CPU tests (gcc) share one definition.
 *
 * HIP's module launch takes the grid as 32-bit workgroup counts, and the AQL
 * dispatch packet it becomes holds the grid size in work-items as a 32-bit
 * number per dimension.  So one launch of `threads`-wide workgroups along x
 * covers at most FG_MAX_LAUNCH_BLOCKS workgroups and FG_MAX_LAUNCH_ITEMS
 * work-items.  A plan whose batch needs more runs it in several launches
 * (FftPlan::fit_launches); a launch beyond the limit is refused, never
 * truncated.  (The reference passes `batch as u32` as its grid and so wraps
 * silently, crates/ferrum-gpu-py/src/lib.rs:147.) */
#ifndef FG_LAUNCH_LIMITS_H
#define FG_LAUNCH_LIMITS_H

#include <stdint.h>

#define FG_MAX_LAUNCH_ITEMS 0xffffffffull
#define FG_MAX_LAUNCH_BLOCKS 0x7fffffffull
#define FG_MAX_BLOCK_THREADS 1024ull

/* Whether `blocks` workgroups of `threads` work-items fit one launch. */
static inline int fg_launch_fits(uint64_t blocks, uint64_t threads) {
    return blocks >= 1 && threads >= 1 && threads <= FG_MAX_BLOCK_THREADS && blocks <= FG_MAX_LAUNCH_BLOCKS &&
           blocks <= FG_MAX_LAUNCH_ITEMS / threads;
}

/* The most units (transforms, images) one launch covers when u units take
 * ceil(u * blocks_per_unit / units_per_block) workgroups of `threads`
 * work-items: a Stockham kernel holds units_per_block transforms per
 * workgroup (blocks_per_unit 1), a tile or row-pair pass takes
 * blocks_per_unit workgroups per unit (units_per_block 1).  A multiple of
 * units_per_block when blocks_per_unit is 1; 0 when one unit alone does not
 * fit. */
static inline uint64_t fg_max_units_per_launch(uint64_t blocks_per_unit, uint64_t units_per_block,
                                               uint64_t threads) {
    uint64_t blocks;
    if (blocks_per_unit == 0 || units_per_block == 0 || threads == 0 || threads > FG_MAX_BLOCK_THREADS) return 0;
    blocks = FG_MAX_LAUNCH_ITEMS / threads;
    if (blocks > FG_MAX_LAUNCH_BLOCKS) blocks = FG_MAX_LAUNCH_BLOCKS;
    /* u * blocks_per_unit <= blocks * units_per_block; neither product
     * overflows: blocks < 2^31 and units_per_block <= 2^10 here */
    return blocks * units_per_block / blocks_per_unit;
}

#endif

// fft_plan.cpp -- plan construction and stream-ordered execution.
#include "fft_plan.hpp"

#include "launch_limits.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <fstream>
#include <iterator>

extern "C" {
// Embedded by embed.S (.incbin of the gfx950 code object).
extern const unsigned char fg_fft_code_object_start[];
extern const unsigned char fg_fft_code_object_end[];
}

namespace fg {

namespace {

// Launch geometry of the single-pass Stockham kernels, mirroring the
// FG_STOCKHAM(LOGN, LOGE, FPB) instantiations in kernels/fft_kernels.hip.
struct StockhamGeom {
    uint32_t log_e;  // log2 of elements per thread
    uint32_t fpb;    // transforms per workgroup
};
// N = 16 .. 128 hold 4 or 8 elements per thread: 16 (the larger sizes' choice)
// measured 217 / 232 / 234 / 211 us per 512 MiB batch against 182 / 183 / 171
// / 173 us for the entries below (N = 256 .. 4096 measured best at 16).
// N = 8192 / 16384 / 32768 ({5, 1}): 32 elements per thread with the
// exchanges in halves (fg_fft_n13 / n14 / n15, kernels/fft_stockham.hpp);
// 32768 points run one 1024-thread, 136 KB workgroup per CU and measured
// 270 us per 512 MiB against 352 us for the two tile passes they replace.
constexpr StockhamGeom kStockham[kMaxLogNSingle + 1] = {
    {0, 0}, {0, 0},          // log_n 0, 1: unsupported
    {2, 64}, {3, 64}, {3, 32}, {3, 16}, {2, 4}, {3, 4}, {4, 4}, {4, 2}, {4, 2}, {4, 1}, {4, 1}, {5, 1}, {5, 1}, {5, 1},
};
// Latency geometry (fg_fft_n<L>_lat, one transform per workgroup, fewer
// elements per thread: more threads per transform, shorter serial chains),
// for single-pass plans too small to fill the GPU.  {0, 0}: none.  Measured
// with graph replay at batch 256: N = 256 5.75 -> 4.58 us per launch pair,
// N = 1024 3.94 -> 3.65 us, N = 4096 10.94 -> 10.69 us.
constexpr StockhamGeom kStockhamLatency[kMaxLogNSingle + 1] = {
    {0, 0}, {0, 0}, {0, 0}, {0, 0}, {0, 0}, {0, 0}, {0, 0}, {0, 0},
    {2, 1}, {0, 0}, {3, 1}, {0, 0}, {3, 1}, {0, 0}, {0, 0}, {0, 0},
};

// The code object named by FERRUM_GPU_CODE_OBJECT, read once per process (a
// function-local static: thread-safe when several threads open devices);
// empty if the file cannot be read.
const std::string& file_image(const char* path) {
    static const std::string image = [path] {
        std::ifstream f(path, std::ios::binary);
        if (!f) return std::string();
        return std::string(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
    }();
    return image;
}

}  // namespace

KernelArtifact fft_code_object() {
    KernelArtifact a;
    a.backend = BackendId::Hip;
    a.name = "ferrum-gpu-fft-kernels";
    a.target = "gfx950";
    if (const char* path = getenv("FERRUM_GPU_CODE_OBJECT")) {
        const std::string& image = file_image(path);
        if (image.empty()) invalid(std::string("FERRUM_GPU_CODE_OBJECT: cannot read ") + path);
        a.image = image.data();
        a.size = image.size();
    } else {
        a.image = fg_fft_code_object_start;
        a.size = (size_t)(fg_fft_code_object_end - fg_fft_code_object_start);
    }
    return a;
}

std::vector<Cf32> stockham_twiddles(uint32_t log_n, uint32_t log_e) {
    const uint32_t nfull = log_n / log_e, rem = log_n % log_e;
    const uint32_t nstages = nfull + (rem ? 1 : 0);
    std::vector<Cf32> t;
    for (uint32_t s = 1; s < nstages; ++s) {
        const uint32_t logl = s * log_e;
        const uint32_t logr = (s < nfull) ? log_e : rem;
        const uint64_t L = 1ull << logl, R = 1ull << logr, M = L * R;
        // Row exponents (kernels/fft_stockham.hpp, tw_row_len): factored rows
        // for radix 16 and 8, full rows below.
        if (L >= 1024) {
            // Two-level block (kernels/fft_stockham.hpp, tw_two_level):
            // W_M^{64 h} for h < L/64 (radix 8: h < M/64, tw_two_level_high),
            // then W_M^l for l < 64.
            for (uint64_t h = 0; h < (R == 8 ? M : L) / 64; ++h) {
                const double ang = 2.0 * M_PI * (double)((64 * h) % M) / (double)M;
                t.push_back(Cf32{(float)cos(ang), (float)-sin(ang)});
            }
            for (uint64_t l = 0; l < 64; ++l) {
                const double ang = 2.0 * M_PI * (double)l / (double)M;
                t.push_back(Cf32{(float)cos(ang), (float)-sin(ang)});
            }
            continue;
        }
        std::vector<uint64_t> ps;
        if (R == 16) ps = {1, 2, 3, 4, 8, 12};
        else if (R == 8) ps = {1, 2, 3, 4};
        else for (uint64_t p = 0; p < R; ++p) ps.push_back(p);
        for (uint64_t k = 0; k < L; ++k)
            for (uint64_t p : ps) {
                const uint64_t e = (p * k) % M;
                const double ang = 2.0 * M_PI * (double)e / (double)M;
                t.push_back(Cf32{(float)cos(ang), (float)-sin(ang)});
            }
    }
    if (t.empty()) t.push_back(Cf32{1.f, 0.f});  // single-stage sizes read no table
    return t;
}

std::vector<Cf32> fft1024_x2_twiddles() {
    auto w = [](uint64_t M, uint64_t e) {
        const double a = 2.0 * M_PI * (double)(e % M) / (double)M;
        return Cf32{(float)cos(a), (float)-sin(a)};
    };
    std::vector<Cf32> t;
    for (uint64_t k = 0; k < 8; ++k)
        for (uint64_t p : {1, 2, 3, 4, 8, 12}) t.push_back(w(128, p * k));
    for (uint64_t k = 0; k < 128; ++k)
        for (uint64_t p : {1, 2, 3, 4}) t.push_back(w(1024, p * k));
    return t;
}

std::vector<Cf32> big_twiddles() {
    std::vector<Cf32> t(8192);
    for (int j = 0; j < 4096; ++j) {
        const double a = 2.0 * M_PI * (double)j / 4096.0;
        const double b = 2.0 * M_PI * (double)j / 16777216.0;
        t[j] = Cf32{(float)cos(a), (float)-sin(a)};
        t[4096 + j] = Cf32{(float)cos(b), (float)-sin(b)};
    }
    return t;
}

std::vector<uint32_t> split_1d(uint32_t log_n) {
    // Two passes while both digits fit wide tiles (>= 16 columns, L * G <=
    // 16384 complex of LDS), three passes beyond 2^20.  Narrow tiles (2048 /
    // 4096-point digits) are for cache-resident data only: reading the input
    // from HBM in 32-byte pieces measured 2.9x slower than 256-byte ones.
    // Two digits: the first (the column pass that reads HBM) of at least 256
    // points, the last (the row-wise pass that streams the output out) of
    // at most 1024.  Measured on gfx950 at 512 MiB per execution, us, with
    // the last passes exchanging in halves (three alternations): 2^17 as 256
    // * 512 330.0 .. 330.9, 512 * 256 338.4 .. 338.9, 128 * 1024 342.0 ..
    // 343.3; 2^18 as 256 * 1024 339.7 .. 341.0, 1024 * 256 351.4 .. 352.2,
    // 512 * 512 351.3 .. 352.0; 2^19 as 512 * 1024 358.1 .. 359.8, 1024 *
    // 512 360.3 .. 361.9; earlier, 2^16 as 256 * 256 326.7 / 327.9, 128 *
    // 512 345.8, 512 * 128 345.5, 64 * 1024 380.9.  (Before those last
    // passes, with one 139 KB workgroup per CU at 1024 points, the split
    // was the other way round: 2^18 as 1024 * 256 356.0, 256 * 1024 379.2.)
    if (log_n <= 20) {
        const uint32_t b = log_n >= 16 ? std::min<uint32_t>(10, log_n - 8) : log_n / 2;
        return {log_n - b, b};
    }
    const uint32_t base = log_n / 3, rest = log_n - 3 * base;
    return {base + (rest > 0 ? 1u : 0u), base + (rest > 1 ? 1u : 0u), base};
}

uint32_t tile_columns(uint32_t log_l) {
    // Passes that read HBM (a plan's first pass; every pass of an unchunked
    // plan).  Up to 1024 points: measured on gfx950 at 2^24 = 256^3, 32 columns of 256
    // points (two 66 KB workgroups per CU) beat 64 (one 133 KB workgroup);
    // fewer than 16 columns (128-byte segments) loses HBM efficiency, so the
    // floor is 16.  2048 / 4096 points (2D columns only): 8 columns with the
    // exchanges in halves (68 / 136 KB of LDS) -- narrow tiles, which are
    // read in XCD-aware order through the caches (add_tile).
    if (log_l > 10) return 8u;
    uint32_t g = 8192u >> log_l;
    if (g > 64) g = 64;
    if (g < 16) g = 16;
    return g;
}

uint32_t cached_tile_columns(uint32_t log_l, bool rowwise) {
    // Passes whose input is the previous pass's output, still cache-resident
    // (chunked plans): the pieces of each 128-byte line meet in L2 / the
    // Infinity Cache, so narrower tiles -- more resident workgroups per CU to
    // overlap one tile's loads with another's arithmetic -- beat the wide
    // ones HBM needs.  Measured on gfx950, us per 128 MiB chunk:
    //  * column-wise, 8 columns in XCD-aware order from 128 points up: 256
    //    points 47.3 -> 42.3 (32 columns), 512 rows 50.5 -> 47.8 and 1024
    //    rows 58.2 -> 56.2 (16); at 64 points 8 columns lose (47.8 vs 40.2);
    //  * row-wise (the 1D last pass, output streamed in G * 8-byte pieces):
    //    16 rows at 128 points (43.1 -> 39.4 from 64), 8 at 512 (48.4 -> 43.9
    //    from 16), 16 at 1024 (8 lose: 60.6 vs 57.6); at 64 points 16 rows
    //    gain nothing over 64.  256 points: 32 rows exchanging in halves
    //    (use_row_halves_tile), measured at 512 MiB per execution against 16
    //    rows in the 16-element tile (two alternations, us): 2^16 323.1 /
    //    324.2 -> 321.4 / 322.0, 2^17 341.3 / 341.2 -> 338.2 / 338.7, 2^18
    //    353.4 / 353.9 -> 352.9 / 352.7, 2^24 479.5 / 479.7 -> 479.5 / 480.1
    //    (16 rows in halves: 324.1, 340.2, 354.6, 482.3).
    //  * the 1D middle pass of 256 points (three-pass plans): 16 columns
    //    exchanging in halves (use_halves_tile; whole 128-byte lines),
    //    measured at 512 MiB per execution against the 8-column tile (three
    //    alternations, us): 2^23 478.8 / 479.2 / 477.8 -> 475.7 / 475.5 /
    //    475.5, 2^24 480.8 / 481.7 / 480.7 -> 480.4 / 479.5 / 479.6; at 128
    //    points (2^21, 2^22) no gain (483.1 .. 484.5 -> 484.0 .. 485.1 at
    //    2^21), so those keep 8 columns.
    if (log_l < 7) return tile_columns(log_l);
    if (rowwise) return log_l == 9 ? 8u : log_l == 8 ? 32u : 16u;
    return log_l == 8 ? 16u : 8u;
}

bool use_halves_tile(uint32_t log_l, uint32_t g, bool rowwise) {
    // Column passes at the HBM width (tile_columns), 128 .. 1024 points, and
    // the 8-column passes of 2048 / 4096 points exchange in halves.  Measured
    // on gfx950 against the 16-element tiles: the 1D first pass at 512 MiB
    // per plan, us per 128 MiB chunk, 128 points 54.3 -> 50.6, 256: 57.0 ->
    // 54.4 (config 4's pass: 52.8 -> 48.4), 512: 63.4 -> 59.4, 1024: 68.4 ->
    // 61.0, whole plans 1-5 % faster for every 1D length 2^13 .. 2^24; 2D
    // column passes (256 MiB chunks, us per plan at 512 MiB) 128 / 256 rows
    // 0.2 .. 1.1 % faster, 512 rows 0.5 .. 4.1 % from 512 columns (0.5 %
    // slower at 128 / 256), 1024 rows 1.8 .. 7.4 %.  2048 / 4096 points: twice the columns per tile in
    // the same LDS (add_tile gives the timings).  The cache-resident
    // 8-column passes of 128 .. 1024 points keep the 16-element tile: at 512
    // points halves lost (41.5 .. 46.7 -> 45.8 .. 47.3 us per 128 MiB pass).
    // The 1D middle pass of 256 points runs 16 columns in halves instead.
    if (rowwise) return false;
    if (log_l > 10) return true;
    // the cache-resident 1D middle pass of 256 points (cached_tile_columns)
    if (log_l == 8 && g == 16) return true;
    return log_l >= 7 && g == tile_columns(log_l);
}

bool use_row_halves_tile(uint32_t log_l, uint32_t g, bool rowwise) {
    // The 1D last pass of 512 / 1024 points in 16-row tiles: every row load
    // of the tile is issued at once and each half of the positions is
    // transposed through an LDS tile of L/2 positions, then the exchanges run
    // in halves -- 34 / 68 KB instead of 68 / 136 KB, so four / two
    // workgroups per CU instead of two / one.  Measured on gfx950 at 512 MiB
    // per execution (two alternations, us): 2^20 397.7 / 396.9 -> 368.4 /
    // 369.9, 2^19 365.4 / 366.3 -> 362.3 / 362.7.  At 256 points (already
    // four workgroups per CU at 16 rows) halves of 16 rows gained nothing;
    // halves of 32 rows (33 KB, 256-byte output pieces) do
    // (cached_tile_columns).
    if (!rowwise) return false;
    return (g == 16 && (log_l == 9 || log_l == 10)) || (g == 32 && log_l == 8);
}

bool split_2d_columns(uint32_t log_rows) { return log_rows > 12; }

namespace {

size_t initial_chunk_limit() {
    // The bytes of a plan's chunks in flight at once: 256 MiB, the size of
    // the Infinity Cache that keeps the intermediates between passes.  Plans
    // that run two chunks at a time (FftPlan::choose_chunk) take chunks of
    // half of it: 128 MiB each, measured on gfx950 with a copy over a working
    // set of 2 x S: 8.4 TB/s at S = 128 MiB, 6.1 TB/s at 160.  Plans on one
    // stream take chunks of all of it: measured at 512 MiB per execution, us,
    // chunks of 128 -> 256 MiB, 2D 4096 x 4096 395 -> 380, 2048 x 2048 376
    // -> 364, 4096 x 64 394 -> 386, 16 x 4096 342 -> 321, 512 x 64 343 ->
    // 322, 4096 x 16 443 -> 413 (the two-chunk plans at 256 MiB per chunk:
    // 1D 2^24 485 -> 638, 2D 256 x 256 324 -> 403).
    size_t mib = 256;
    if (const char* e = getenv("FERRUM_GPU_CHUNK_MIB")) {
        char* end = nullptr;
        const unsigned long long v = strtoull(e, &end, 10);
        if (end != e && *end == 0 && v <= (1ull << 20)) mib = (size_t)v;
    }
    return mib << 20;
}

std::atomic<size_t>& chunk_limit_ref() {
    static std::atomic<size_t> limit{initial_chunk_limit()};
    return limit;
}

}  // namespace

size_t chunk_limit_bytes() { return chunk_limit_ref().load(); }
void set_chunk_limit_bytes(size_t bytes) { chunk_limit_ref().store(bytes); }

size_t chunk_units_for(uint64_t unit_bytes, size_t batch, size_t limit, bool* cached) {
    if (limit == 0 || unit_bytes == 0 || unit_bytes > limit) {
        *cached = false;
        return batch;
    }
    *cached = true;
    return (size_t)std::min<uint64_t>(limit / unit_bytes, batch);
}

bool FftPlan::choose_chunk(bool two_in_flight) {
    const size_t limit = chunk_limit_bytes();
    const uint64_t unit = 8ull * elems();
    if (two_in_flight && unit <= limit / 2) {
        chunk_ = chunk_units_for(unit, batch_, limit / 2, &cached_);
        if (chunks() > 1) return true;
    }
    chunk_ = chunk_units_for(unit, batch_, limit, &cached_);
    return false;
}

const char* FftPlan::policy(size_t i, size_t n) const {
    if (!cached_) return "";
    if (i == 0) return "_sc";
    return i + 1 == n ? "_cs" : "_cc";
}

namespace {

uint32_t elems_per_thread_log(uint32_t log_l) { return log_l < 4 ? log_l : 4; }

std::string tile_name(uint32_t log_l, uint32_t g, const char* kind, const char* policy) {
    return "fg_tile_l" + std::to_string(log_l) + "_g" + std::to_string(g) + "_" + kind + policy;
}

}  // namespace

const void* FftPlan::stage_table(uint32_t log_l, uint32_t log_e) {
    // One table per (length, elements per thread): the radix list, and so the
    // table, depends on both.  log_e == kX2Layout: the 8 * 16 * 8 list of the
    // two-transform 1024-point kernel.
    const uint32_t key = log_l * 64 + log_e;
    for (auto& e : stage_tables_)
        if (e.first == key) return e.second.data();
    auto tw = log_e == kX2Layout ? fft1024_x2_twiddles() : stockham_twiddles(log_l, log_e);
    Buffer<Cf32, HipBackend> b = dev_->alloc<Cf32>(tw.size());
    b.copy_from_host(tw.data(), tw.size());
    stage_tables_.emplace_back(key, std::move(b));
    return stage_tables_.back().second.data();
}

const void* FftPlan::big_table() {
    if (!big_.data()) {
        auto t = big_twiddles();
        big_ = dev_->alloc<Cf32>(t.size());
        big_.copy_from_host(t.data(), t.size());
    }
    return big_.data();
}

bool use_latency_geometry(uint32_t log_n, uint64_t count, int cu_count) {
    // The throughput geometry would give fewer than two workgroups per CU.
    const StockhamGeom t = kStockham[log_n], l = kStockhamLatency[log_n];
    return l.fpb != 0 && (count + t.fpb - 1) / t.fpb < 2ull * (uint64_t)cu_count;
}

void FftPlan::add_stockham(const HipBackend::Module& mod, uint32_t log_l, uint64_t per_unit, Buf src, Buf dst,
                           const char* policy, bool latency) {
    const StockhamGeom g = latency ? kStockhamLatency[log_l] : kStockham[log_l];
    if (g.fpb == 0) fail(FG_ERR_INTERNAL, "no latency geometry for this length");
    Step s;
    s.name = "fg_fft_n" + std::to_string(log_l) + (latency ? "_lat" : "") + policy;
    s.fn = HipBackend::get_kernel(mod, s.name.c_str());
    s.block = Dim3(((1u << log_l) >> g.log_e) * g.fpb);
    s.fpb = g.fpb;
    s.src = src;
    s.dst = dst;
    // 32-element kernels (log_e 5) run the radix-16 list of the 16-element
    // layout; the 1024-point throughput kernels the 8 * 16 * 8 list.
    s.tw = (log_l == 10 && !latency) ? stage_table(10, kX2Layout) : stage_table(log_l, std::min<uint32_t>(g.log_e, 4));
    s.per_unit = per_unit;
    steps_.push_back(s);
}

void FftPlan::add_tile(const HipBackend::Module& mod, uint32_t log_l, uint32_t g, bool rowwise,
                       const TileGeom& geom, uint64_t tiles_per_unit, Buf src, Buf dst, const char* policy) {
    // The kernel reads columns at stride 1 (column-wise) or elements at stride
    // 1 (row-wise) and always writes columns at stride 1.
    if ((rowwise ? geom.ies : geom.ics) != 1 || geom.ocs != 1) fail(FG_ERR_INTERNAL, "tile geometry not unit-stride");
    if (tiles_per_unit == 0) fail(FG_ERR_INTERNAL, "tile pass with no tiles");
    // Narrow tiles (g < 16: 32- or 64-byte pieces of each 128-byte line) load
    // and store through the caches whatever the chunking, in XCD-aware tile
    // order, so the pieces of a line from neighbouring tiles meet in one
    // XCD's L2; nontemporal access to such pieces measured 5x slower.
    const bool narrow = g < 16;
    if (narrow) policy = "_cc";
    // Every tile kernel takes G adjacent columns (row-wise: G rows, stored as
    // G adjacent output columns): the geometry must step tiles by G.
    if ((rowwise ? geom.os0 : geom.is0) != g) fail(FG_ERR_INTERNAL, "tile geometry does not step by the tile width");
    // The pass that reads the caller's input (the first 1D pass) exchanges in
    // halves: twice the workgroups per CU to cover HBM latency.
    const bool halves = use_halves_tile(log_l, g, rowwise);
    Step s;
    s.tile = true;
    if (narrow) {
        // the 16-element tiles: one contiguous tile range per XCD; the halves
        // tiles (2D columns of 1024 .. 4096 points): line groups dealt over the
        // XCDs, measured on gfx950 at 128 MiB per launch, us per pass over
        // 4096 / 2048 rows of 128 .. 4096 columns: 8 columns in halves with
        // line groups 53.8 .. 57.1 / 47.7 .. 51.0, with XCD ranges 52.0 ..
        // 72.5 / 44.5 .. 56.8 (slowest at 16 MiB images), the 16-element
        // tiles (4 / 8 columns, XCD ranges) 60.8 .. 69.7 / 54.0 .. 62.5
        s.tile_order = halves ? FG_TILE_ORDER_LINE_GROUPS : FG_TILE_ORDER_XCD_RANGES;
        s.order_unit = halves ? 8 * (16 / g) : 8;
    }
    const bool row_halves = use_row_halves_tile(log_l, g, rowwise);
    s.name = tile_name(log_l, g, halves ? "h" : row_halves ? "rh" : (rowwise ? "r" : "c"), policy);
    s.fn = HipBackend::get_kernel(mod, s.name.c_str());
    s.block = Dim3(g * ((1u << log_l) >> ((halves || row_halves) ? 5 : elems_per_thread_log(log_l))));
    s.src = src;
    s.dst = dst;
    s.tw = stage_table(log_l, elems_per_thread_log(log_l));
    s.geom = geom;
    s.per_unit = tiles_per_unit;
    steps_.push_back(s);
}

FftPlan::ChunkStream::ChunkStream(const HipBackend::DeviceHandle& d) : dev(d) {
    stream = HipBackend::chunk_stream(dev);
    HipBackend::bind(dev);
    hip_check(hipEventCreateWithFlags(&fork, hipEventDisableTiming), "hipEventCreateWithFlags");
    const hipError_t e = hipEventCreateWithFlags(&join, hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipEventDestroy(fork);
        hip_check(e, "hipEventCreateWithFlags");
    }
}

FftPlan::ChunkStream::~ChunkStream() {
    (void)hipSetDevice(dev->ordinal);
    // The plan's last execution joined the chunk stream back here (an event
    // never recorded completes at once); later work of other plans on the
    // shared stream is theirs.
    (void)hipEventSynchronize(join);
    (void)hipEventDestroy(fork);
    (void)hipEventDestroy(join);
}

void FftPlan::set_streams(int n) {
    if (n != 1 && n != 2) invalid("streams must be 1 or 2, got " + std::to_string(n));
    if (n == 2 && !aux_) invalid("this plan runs on one stream (two-stream plans: multi-pass 1D of two or more chunks)");
    use_aux_ = n == 2;
}

void FftPlan::fit_launches() {
    // Each step's largest units per launch; chunk_ takes the smallest.
    uint64_t most = chunk_;
    for (const std::vector<Step>* v : {&steps_, &steps_in_place_})
        for (const Step& s : *v) {
            const uint64_t threads = s.block.product();
            // Stockham and one-pass 2D kernels: fpb units per workgroup;
            // row-pair and tile passes: per_unit workgroups per unit.
            const bool per_block = !s.tile && !s.rowpair;
            const uint64_t m = per_block ? fg_max_units_per_launch(s.per_unit, s.fpb, threads)
                                         : fg_max_units_per_launch(s.per_unit, 1, threads);
            if (m == 0) invalid("one transform of this plan exceeds a single kernel launch");
            most = std::min(most, m);
        }
    chunk_ = (size_t)most;
}

std::unique_ptr<FftPlan> FftPlan::make_1d(HipDevice& dev, const HipBackend::Module& mod, uint32_t log_n,
                                          size_t batch) {
    if (log_n < kMinLogN1D || log_n > kMaxLogN1D)
        invalid("log_n must be in [" + std::to_string(kMinLogN1D) + ", " + std::to_string(kMaxLogN1D) +
                "], got " + std::to_string(log_n));
    if (batch == 0) invalid("batch must be positive");
    if (log_n <= kMaxLogNSingle) {
        std::unique_ptr<FftPlan> p(new FftPlan(dev, Kind::Stockham1D, log_n, 0, batch));
        const bool latency = use_latency_geometry(log_n, batch, dev.handle()->cu_count);
        p->add_stockham(mod, log_n, 1, Buf::In, Buf::Out, "", latency);
        p->main_kernel_ = p->steps_[0].name;
        p->split_fn_ = HipBackend::get_kernel(mod, (p->main_kernel_ + "_split").c_str());
        p->pw_ = Pointwise(mod);
        p->fit_launches();
        return p;
    }

    // N = N_1 * ... * N_P, digit 1 slowest; S_i = stride of digit i.
    std::unique_ptr<FftPlan> p(new FftPlan(dev, Kind::MultiPass1D, log_n, 0, batch));
    const std::vector<uint32_t> logs = split_1d(log_n);
    const size_t P = logs.size();
    const uint64_t N = 1ull << log_n;
    std::vector<uint64_t> S(P + 1);
    S[0] = N;
    for (size_t i = 1; i <= P; ++i) S[i] = S[i - 1] >> logs[i - 1];
    if (N * batch > (1ull << 40)) invalid("transform too large");
    const bool two = p->choose_chunk(true);
    p->work_ = dev.alloc<Cf32>(N * p->chunk_);
    const void* big = p->big_table();
    (void)big;
    // Passes 1..P-1: DFT over digit i for every value of the faster digits
    // (columns, contiguous) and of the slower, already transformed digits;
    // four-step twiddle W_{S_{i-1}}^{r_i k_i}; in place in the workspace.
    for (size_t i = 1; i < P; ++i) {
        const uint32_t log_l = logs[i - 1];
        // Pass 1 reads the caller's input from HBM; later passes read the
        // chunk's intermediate from the caches when the plan is chunked.
        const uint32_t g = (i > 1 && p->cached_) ? cached_tile_columns(log_l, false) : tile_columns(log_l);
        if (S[i] < g) fail(FG_ERR_INTERNAL, "digit split leaves fewer columns than a tile");
        TileGeom t{};
        t.t0n = (uint32_t)(S[i] / g);
        t.t1n = (uint32_t)(N / S[i - 1]);
        t.is0 = t.os0 = g;
        t.is1 = t.os1 = S[i - 1];
        t.is2 = t.os2 = N;
        t.ics = t.ocs = 1;
        t.ies = t.oes = S[i];
        t.twc = 1;
        t.tw0 = g;
        t.tw1 = 0;
        t.log_m = (uint32_t)__builtin_ctzll(S[i - 1]);
        p->add_tile(mod, log_l, g, false, t, (uint64_t)t.t0n * t.t1n, i == 1 ? Buf::In : Buf::Work, Buf::Work,
                    p->policy(i - 1, P));
    }
    // Pass P: contiguous rows of N_P for each (k_1, k_2..k_{P-1}); G' rows of
    // consecutive k_1 per tile, stored to the digit-reversed output position
    // k_1 + N_1 k_2 + N_1 N_2 k_P (P <= 3).
    {
        const uint32_t log_l = logs[P - 1];
        const uint64_t L = 1ull << log_l, n1 = 1ull << logs[0];
        uint32_t g = p->cached_ ? cached_tile_columns(log_l, true) : tile_columns(log_l);
        // With two chunks in flight (below) the 16-row tile wins at 512
        // points too (measured with the 512-point last digits of earlier
        // splits, 2^18 = 512 * 512 and 2^19 = 1024 * 512: 397 / 406 us at 512
        // MiB with 8 rows on one stream -> 370 / 376 us with 16 rows on two);
        // 2^17 = 256 * 512 takes it now, in halves (use_row_halves_tile).
        if (two && g < 16) g = 16;
        if (n1 < g) fail(FG_ERR_INTERNAL, "digit split leaves fewer rows than a tile");
        TileGeom t{};
        t.t0n = (uint32_t)(n1 / g);
        t.t1n = (uint32_t)(N / (n1 * L));
        t.is0 = g * S[1];
        t.is1 = L;
        t.is2 = N;
        t.ics = S[1];
        t.ies = 1;
        t.os0 = g;
        t.os1 = n1;
        t.os2 = N;
        t.ocs = 1;
        t.oes = N / L;
        p->add_tile(mod, log_l, g, true, t, (uint64_t)t.t0n * t.t1n, Buf::Work, Buf::Out, p->policy(P - 1, P));
        if (two) {
            // Two chunks in flight, one per stream: their passes overlap, so
            // one chunk's transform phases fill the other's memory phases.
            // Measured on gfx950 at 512 MiB in chunks of 128 MiB (us per
            // execution, one stream -> two): 2^16 347 -> 328, 2^17 380 -> 348,
            // 2^20 446 -> 403, 2^21 .. 2^24 510 .. 519 -> 481 .. 485.  With
            // the last pass in 8-row tiles 2^18 / 2^19 lost (397 / 405 ->
            // 502 / 515), and 2D plans lose (four 4096 x 4096 images 425 ->
            // 466): narrow pieces of one line meet in an XCD's L2 only while
            // a single chunk streams through it.
            p->work2_ = dev.alloc<Cf32>(N * p->chunk_);
            p->aux_.reset(new ChunkStream(dev.handle()));
        }
    }
    p->main_kernel_ = p->steps_[0].name;
    p->pw_ = Pointwise(mod);
    p->fit_launches();
    return p;
}

std::unique_ptr<FftPlan> FftPlan::make_2d(HipDevice& dev, const HipBackend::Module& mod, uint32_t log_rows,
                                          uint32_t log_cols, size_t batch) {
    for (uint32_t l : {log_rows, log_cols})
        if (l < kMinLogN2D || l > kMaxLogN2D)
            invalid("2D requires log_n in [" + std::to_string(kMinLogN2D) + ", " + std::to_string(kMaxLogN2D) +
                    "]; got " + std::to_string(l));
    if (batch == 0) invalid("batch must be positive");
    std::unique_ptr<FftPlan> p(new FftPlan(dev, Kind::TwoD, log_cols, log_rows, batch));
    const uint64_t R = 1ull << log_rows, C = 1ull << log_cols, RC = R * C;
    if (log_rows + log_cols <= FG_SMALL2D_MAX_LOG) {
        // Images of up to 16384 points: the whole 2D FFT in one pass through
        // LDS (kernels/fft_2d_small.hpp); nothing to chunk.
        p->chunk_ = batch;
        p->cached_ = false;
        Step s;
        s.small2d = true;
        s.name = "fg_fft2d_l" + std::to_string(log_rows) + "_" + std::to_string(log_cols);
        s.fn = HipBackend::get_kernel(mod, s.name.c_str());
        s.fpb = FG_SMALL2D_FPI(log_rows, log_cols);
        s.block = Dim3(FG_SMALL2D_BLOCK(log_rows, log_cols));
        s.src = Buf::In;
        s.dst = Buf::Out;
        s.tw = p->stage_table(log_cols, FG_SMALL2D_LOGE(log_rows, log_cols));
        s.tw_cols = p->stage_table(log_rows, FG_SMALL2D_LOGE(log_rows, log_cols));
        s.per_unit = 1;
        p->steps_.push_back(s);
        p->main_kernel_ = s.name;
        p->split_fn_ = HipBackend::get_kernel(mod, (s.name + "_split").c_str());
        p->pw_ = Pointwise(mod);
        p->fit_launches();
        return p;
    }
    const bool split = split_2d_columns(log_rows);
    const size_t npass = split ? 3 : 2;
    // One chunk at a time, of up to the whole chunk limit.  Measured on
    // gfx950 at 512 MiB against two chunks of half of it in flight on two
    // streams (with the wide column tiles), us per execution, 32 .. 1024 rows
    // of 128 .. 4096 columns: 21 of 25 shapes faster by 0.6 .. 7.5 % (256 x
    // 256 324 -> 315, 1024 x 2048 378 -> 350, 32 x 1024 336 -> 314), 128 x
    // 2048 / 4096 and 512 x 4096 0.6 .. 1.3 % slower.
    p->choose_chunk(false);
    if (split) p->work_ = dev.alloc<Cf32>(RC * p->chunk_);
    // Row pass (the reference's K1 row FFT, py lib.rs:325-336): R rows of C per image.
    p->add_stockham(mod, log_cols, R, Buf::In, split ? Buf::Work : Buf::Out, p->policy(0, npass));
    if (!split) {
        // Column pass, in place: G adjacent columns of length R per tile.
        // Chunked plans of 2048 and 4096 rows take the cache-resident
        // 8-column tiles, the others the wide tiles of the HBM passes (128 /
        // 256 rows: 64 / 32 columns; 512 / 1024 rows: 16 columns in halves,
        // output streamed): measured on gfx950 at 512 MiB in chunks of 256
        // MiB, us per execution, wide against 8 columns over 128 .. 4096
        // columns: 128 rows 0.8 .. 3.8 % faster, 256 rows 0 .. 2.6 %, 1024
        // rows 1.8 .. 7.4 % (1024 x 4096 369 -> 342), 512 rows 0.5 .. 4.1 %
        // from 512 columns (512 x 4096 345 -> 331), 0.5 % slower at 128 / 256
        // (the 16-element 16-column tile: 2 .. 3 % slower there).
        const bool narrow = p->cached_ && log_rows > 10;
        const uint32_t g = (uint32_t)std::min<uint64_t>(
            narrow ? cached_tile_columns(log_rows, false) : tile_columns(log_rows), C);
        TileGeom t{};
        t.t0n = (uint32_t)(C / g);
        t.t1n = 1;
        t.is0 = t.os0 = g;
        t.is1 = t.os1 = 0;
        t.is2 = t.os2 = RC;
        t.ics = t.ocs = 1;
        t.ies = t.oes = C;
        p->add_tile(mod, log_rows, g, false, t, (uint64_t)t.t0n, Buf::Out, Buf::Out, p->policy(1, npass));
    } else {
        // Column FFT of length R = R_1 * R_2 over the slow axis, as two column
        // passes over G = min(64, C) adjacent columns.
        const uint32_t l1 = log_rows - log_rows / 2, l2 = log_rows / 2;
        const uint64_t R1 = 1ull << l1, R2 = 1ull << l2;
        const uint32_t g = (uint32_t)std::min<uint64_t>(64, C);
        TileGeom a{};
        a.t0n = (uint32_t)(C / g);
        a.t1n = (uint32_t)R2;
        a.is0 = a.os0 = g;
        a.is1 = a.os1 = C;
        a.is2 = a.os2 = RC;
        a.ics = a.ocs = 1;
        a.ies = a.oes = R2 * C;
        a.twc = 0;
        a.tw0 = 0;
        a.tw1 = 1;
        a.log_m = log_rows;
        p->big_table();
        p->add_tile(mod, l1, g, false, a, (uint64_t)a.t0n * a.t1n, Buf::Work, Buf::Work, p->policy(1, npass));
        TileGeom b{};
        b.t0n = (uint32_t)(C / g);
        b.t1n = (uint32_t)R1;
        b.is0 = g;
        b.is1 = R2 * C;
        b.is2 = RC;
        b.ics = 1;
        b.ies = C;
        b.os0 = g;
        b.os1 = C;
        b.os2 = RC;
        b.ocs = 1;
        b.oes = R1 * C;
        p->add_tile(mod, l2, g, false, b, (uint64_t)b.t0n * b.t1n, Buf::Work, Buf::Out, p->policy(2, npass));
    }
    if ((log_rows >= 11 && log_cols >= 10) || (log_rows == 10 && log_cols >= 11)) {
        // 2048 / 4096 rows of 1024 .. 4096 points and 1024 rows of 2048 /
        // 4096 points, out of place: the column
        // DFT split radix-2 over the row index.  The row pass transforms rows
        // r and r + R/2 of an image in one workgroup and stores A + B and
        // (A - B) W_R^r to output rows 2r and 2r + 1
        // (kernels/fft_2d_rowpair.hpp); the column pass takes R/2-point DFTs
        // over the rows of each parity in place, in halves: 8 columns at 4096
        // rows (68 KB, where a 4096-row tile takes the CU's LDS), 16 at 2048
        // rows (68 KB) and at 1024 rows (34 KB), whole 128-byte lines.
        // Measured on gfx950 at 512 MiB per execution against the two passes
        // above, us: 4096 x 4096 398 -> 388, 2048 x 4096 373 -> 348, 2048 x
        // 2048 363 -> 359, 2048 x 1024 365 -> 352, 4096 x 1024 375 -> 367
        // (even in another A/B); 1024 rows (three alternations) x 2048
        // 340.0 .. 341.0 -> 333.3 .. 334.2, x 4096 340.8 .. 341.9 -> 335.8 ..
        // 336.3.  1024 x 1024 measured mixed (335.2 .. 341.1 -> 331.1 ..
        // 340.2, and 333 -> 342 in an earlier A/B), so it keeps the two
        // passes above, as every in-place execution does.
        p->steps_in_place_ = std::move(p->steps_);
        p->steps_.clear();
        Step s;
        s.rowpair = true;
        s.log_rows = log_rows;
        s.name = "fg_fft2d_rowpair_n" + std::to_string(log_cols);
        s.fn = HipBackend::get_kernel(mod, s.name.c_str());
        // two rows of 64 / 128 / 128 threads (16 / 16 / 32 elements each at
        // 1024 / 2048 / 4096 points)
        s.block = Dim3(log_cols == 10 ? 128 : 256);
        s.src = Buf::In;
        s.dst = Buf::Out;
        s.tw = p->stage_table(log_cols, 4);
        s.per_unit = R / 2;
        p->big_table();
        p->steps_.push_back(s);
        TileGeom t{};
        // 1024 / 2048 rows: 512- / 1024-row tiles of 16 columns in halves
        // (whole lines, 34 / 68 KB)
        const uint32_t gw = log_rows <= 11 ? 16u : 8u;
        t.t0n = (uint32_t)(C / gw);
        t.t1n = 2;  // row parity
        t.is0 = t.os0 = gw;
        t.is1 = t.os1 = C;
        t.is2 = t.os2 = RC;
        t.ics = t.ocs = 1;
        t.ies = t.oes = 2 * C;
        p->add_tile(mod, log_rows - 1, gw, false, t, (uint64_t)t.t0n * t.t1n, Buf::Out, Buf::Out,
                    p->policy(1, npass));
    }
    p->main_kernel_ = p->steps_.back().name;
    p->pw_ = Pointwise(mod);
    p->fit_launches();
    return p;
}

std::vector<std::string> FftPlan::kernel_names(bool in_place) const {
    const std::vector<Step>& steps = (in_place && !steps_in_place_.empty()) ? steps_in_place_ : steps_;
    std::vector<std::string> v;
    for (size_t c = 0; c < chunks(); ++c)
        for (const Step& s : steps) v.push_back(s.name);
    return v;
}

float FftPlan::scale_for(Direction dir, bool normalize) const {
    // 1/N (1D, plan.rs semantics) or 1/(rows*cols) (2D, cpu_2d.rs:55-61): powers of two, exact.
    if (dir != Direction::Inverse || !normalize) return 1.0f;
    return kind_ == Kind::TwoD ? 1.0f / ((float)(1u << log_rows_) * (float)(1u << log_n_))
                               : 1.0f / (float)(1ull << log_n_);
}

void FftPlan::exec(const void* in, void* out, Direction dir, bool normalize, hipStream_t stream,
                   hipEvent_t* events) const {
    if (!in || !out) invalid("fft exec: null buffer");
    if ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 7u)
        invalid("fft exec: buffers must be 8-byte aligned (complex64)");
    {
        // In place or disjoint: a partial overlap would let one workgroup's
        // stores reach elements another has not read yet.
        const uintptr_t x = reinterpret_cast<uintptr_t>(in), y = reinterpret_cast<uintptr_t>(out);
        const uint64_t nb = 8ull * elems() * batch_;
        if (x != y && x < y + nb && y < x + nb) invalid("fft exec: d_in and d_out overlap without being equal");
    }
    const bool inverse = dir == Direction::Inverse;
    const float scale = scale_for(dir, normalize);
    const void* big = big_.data();
    const uint64_t unit = elems();
    const hipStream_t main = stream ? stream : HipBackend::default_stream(dev_->handle());
    const std::vector<Step>& steps = (in == out && !steps_in_place_.empty()) ? steps_in_place_ : steps_;
    bool two = streams() == 2;
    if (two) {
        // Under stream capture the plan stays on the captured stream.
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        HipBackend::bind(dev_->handle());
        hip_check(hipStreamIsCapturing(main, &st), "hipStreamIsCapturing");
        two = st == hipStreamCaptureStatusNone;
    }
    if (two) {
        hip_check(hipEventRecord(aux_->fork, main), "hipEventRecord");
        hip_check(hipStreamWaitEvent(aux_->stream, aux_->fork, 0), "hipStreamWaitEvent");
    }
    size_t launch = 0;
    size_t chunk = 0;
    for (uint64_t u0 = 0; u0 < batch_; u0 += chunk_, ++chunk) {
        const uint64_t units = std::min<uint64_t>(chunk_, batch_ - u0);
        const bool odd = two && (chunk & 1);
        const hipStream_t cs = odd ? aux_->stream : main;
        // The caller's arrays are offset to the chunk; a workspace holds one chunk.
        auto bind = [&](Buf b) -> void* {
            switch (b) {
                case Buf::In: return const_cast<Cf32*>(static_cast<const Cf32*>(in)) + u0 * unit;
                case Buf::Out: return static_cast<Cf32*>(out) + u0 * unit;
                default: return odd ? work2_.data() : work_.data();
            }
        };
        for (size_t i = 0; i < steps.size(); ++i) {
            const Step& s = steps[i];
            uint32_t flags = 0;
            if (inverse && i == 0) flags |= FG_PASS_CONJ_IN;
            if (inverse && i + 1 == steps.size()) flags |= FG_PASS_CONJ_SCALE_OUT;
            void* src = bind(s.src);
            void* dst = bind(s.dst);
            const void* tw = s.tw;
            if (s.rowpair) {
                uint64_t pairs = s.per_unit * units;
                uint32_t lr = s.log_rows;
                void* args[] = {&src, &dst, (void*)&tw, (void*)&big, &pairs, &lr, &flags};
                const Dim3 grid((uint32_t)pairs);
                if (events)
                    HipBackend::launch_stamped(dev_->handle(), cs, s.fn, grid, s.block, 0, args, events[launch]);
                else
                    HipBackend::launch(dev_->handle(), cs, s.fn, grid, s.block, 0, args);
            } else if (s.small2d) {
                uint64_t count = s.per_unit * units;
                float sc = scale;
                const void* twc = s.tw_cols;
                void* args[] = {&src, &dst, (void*)&tw, (void*)&twc, &count, &sc, &flags};
                const Dim3 grid((uint32_t)((count + s.fpb - 1) / s.fpb));
                if (events)
                    HipBackend::launch_stamped(dev_->handle(), cs, s.fn, grid, s.block, 0, args, events[launch]);
                else
                    HipBackend::launch(dev_->handle(), cs, s.fn, grid, s.block, 0, args);
            } else if (!s.tile) {
                uint64_t count = s.per_unit * units;
                float sc = scale;
                void* args[] = {&src, &dst, (void*)&tw, &count, &sc, &flags};
                const Dim3 grid((uint32_t)((count + s.fpb - 1) / s.fpb));
                if (events)
                    HipBackend::launch_stamped(dev_->handle(), cs, s.fn, grid, s.block, 0, args, events[launch]);
                else
                    HipBackend::launch(dev_->handle(), cs, s.fn, grid, s.block, 0, args);
            } else {
                TileGeom g = s.geom;
                g.flags = flags;
                g.scale = scale;
                const uint64_t tiles = s.per_unit * units;
                g.remap = (s.tile_order != 0 && tiles % s.order_unit == 0) ? s.tile_order : 0u;
                void* args[] = {&src, &dst, (void*)&tw, (void*)&big, &g};
                const Dim3 grid((uint32_t)(s.per_unit * units));
                if (events)
                    HipBackend::launch_stamped(dev_->handle(), cs, s.fn, grid, s.block, 0, args, events[launch]);
                else
                    HipBackend::launch(dev_->handle(), cs, s.fn, grid, s.block, 0, args);
            }
            ++launch;
        }
    }
    if (two) {
        hip_check(hipEventRecord(aux_->join, aux_->stream), "hipEventRecord");
        hip_check(hipStreamWaitEvent(main, aux_->join, 0), "hipStreamWaitEvent");
    }
}

void FftPlan::check_split(const void* in_re, const void* in_im, const void* out_re, const void* out_im) const {
    if (!in_re || !in_im || !out_re || !out_im) invalid("fft exec_split: null buffer");
    if ((reinterpret_cast<uintptr_t>(in_re) | reinterpret_cast<uintptr_t>(in_im) | reinterpret_cast<uintptr_t>(out_re) |
         reinterpret_cast<uintptr_t>(out_im)) & 3u)
        invalid("fft exec_split: arrays must be 4-byte aligned (f32)");
    const uint64_t nb = 4ull * elems() * batch_;
    auto overlap = [nb](const void* a, const void* b) {
        const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
        return x < y + nb && y < x + nb;
    };
    // Each part is either the same array as its input counterpart or disjoint
    // from every other array.
    if (overlap(out_re, out_im) || overlap(out_re, in_im) || overlap(out_im, in_re) ||
        (out_re != in_re && overlap(out_re, in_re)) || (out_im != in_im && overlap(out_im, in_im)))
        invalid("fft exec_split: overlapping buffers (only out_re == in_re and out_im == in_im may alias)");
}

void FftPlan::split_one_launch(const void* in_re, const void* in_im, void* out_re, void* out_im, Direction dir,
                               bool normalize, hipStream_t stream) const {
    const Step& s = steps_[0];  // the split twin has the same geometry and table
    uint32_t flags = dir == Direction::Inverse ? (FG_PASS_CONJ_IN | FG_PASS_CONJ_SCALE_OUT) : 0u;
    float sc = scale_for(dir, normalize);
    const void* tw = s.tw;
    const void* twc = s.tw_cols;
    const uint64_t unit = elems();
    // One launch per chunk (one chunk unless the batch exceeds a launch).
    for (uint64_t u0 = 0; u0 < batch_; u0 += chunk_) {
        uint64_t count = s.per_unit * std::min<uint64_t>(chunk_, batch_ - u0);
        const float* ir = static_cast<const float*>(in_re) + u0 * unit;
        const float* ii = static_cast<const float*>(in_im) + u0 * unit;
        float* orr = static_cast<float*>(out_re) + u0 * unit;
        float* oi = static_cast<float*>(out_im) + u0 * unit;
        const Dim3 grid((uint32_t)((count + s.fpb - 1) / s.fpb));
        if (s.small2d) {
            void* args[] = {&ir, &ii, &orr, &oi, (void*)&tw, (void*)&twc, &count, &sc, &flags};
            HipBackend::launch(dev_->handle(), stream, split_fn_, grid, s.block, 0, args);
        } else {
            void* args[] = {&ir, &ii, &orr, &oi, (void*)&tw, &count, &sc, &flags};
            HipBackend::launch(dev_->handle(), stream, split_fn_, grid, s.block, 0, args);
        }
    }
}

void FftPlan::split_staged(const void* in_re, const void* in_im, void* out_re, void* out_im, Direction dir,
                           bool normalize, hipStream_t stream, Cf32* stage) const {
    const uint64_t n = (uint64_t)elems() * batch_;
    pw_.interleave(dev_->handle(), in_re, in_im, stage, n, stream);
    exec(stage, stage, dir, normalize, stream);
    pw_.deinterleave(dev_->handle(), stage, out_re, out_im, n, stream);
}

void FftPlan::exec_split(const void* in_re, const void* in_im, void* out_re, void* out_im, Direction dir,
                         bool normalize, hipStream_t stream) const {
    check_split(in_re, in_im, out_re, out_im);
    if (split_fn_) {
        split_one_launch(in_re, in_im, out_re, out_im, dir, normalize, stream);
        return;
    }
    {
        std::lock_guard<std::mutex> lock(stage_mu_);
        if (!stage_.data()) {
            // The allocation is hipMalloc + hipMemsetAsync + a stream sync
            // (alloc_zeros is synchronous by contract, backend.rs:30-33), none of
            // which a stream capture can record: refuse before touching HIP.
            hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
            hip_check(hipStreamIsCapturing(stream ? stream : dev_->default_stream(), &status),
                      "hipStreamIsCapturing");
            if (status != hipStreamCaptureStatusNone)
                invalid("fft exec_split: the first split-layout execution of a multi-launch plan allocates its "
                        "staging buffer, which a stream capture cannot record; run it once before capturing");
            stage_ = dev_->alloc<Cf32>((uint64_t)elems() * batch_);
        }
    }
    split_staged(in_re, in_im, out_re, out_im, dir, normalize, stream, stage_.data());
}

void FftPlan::exec_split_into(const void* in_re, const void* in_im, void* out_re, void* out_im, Direction dir,
                              bool normalize, hipStream_t stream, void* staging, size_t staging_bytes,
                              const std::string& no_staging) const {
    check_split(in_re, in_im, out_re, out_im);
    if (split_fn_) {
        split_one_launch(in_re, in_im, out_re, out_im, dir, normalize, stream);
        return;
    }
    const uint64_t need = 8ull * elems() * batch_;
    if (need > staging_bytes)
        invalid("fft exec_split_noalloc: the plan stages " + std::to_string(need) + " bytes (" +
                std::to_string(batch_) + " x " + std::to_string(elems()) + " complex64), beyond the " +
                std::to_string(staging_bytes) + "-byte device scratch area");
    if (!staging) fail(FG_ERR_INTERNAL, "fft exec_split_noalloc: " + no_staging);
    if (reinterpret_cast<uintptr_t>(staging) & 15u) fail(FG_ERR_INTERNAL, "fft exec_split_noalloc: scratch misaligned");
    split_staged(in_re, in_im, out_re, out_im, dir, normalize, stream, static_cast<Cf32*>(staging));
}

}  // namespace fg

// fft_plan.hpp -- FFT plans on a HIP device: the MI355X counterpart of the
// reference's Plan / Plan2D (crates/ferrum-gpu-fft/src/plan.rs:17-135) fused
// with the kernel dispatch of its host runner
// (crates/ferrum-gpu-py/src/lib.rs:117-233 and 273-358).
//
// A plan is built once per (shape, batch): it picks the kernels, uploads the
// twiddle tables to HBM and sizes any workspace.  exec() is stream-ordered and
// launches only kernels -- no host conjugation, no host scaling, no copies.
#pragma once

#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "device.hpp"
#include "hip_backend.hpp"
#include "kernels/tile_geom.h"
#include "pointwise_ops.hpp"

namespace fg {

using HipDevice = Device<HipBackend>;

// Interleaved complex64 on the host side (the reference's Complex32).
struct Cf32 {
    float re, im;
};

// The FFT code object compiled from kernels/fft_kernels.hip and embedded in
// this library (the reference embeds its PTX bundle in the cdylib and loads it
// with load_module_from_image, crates/ferrum-gpu-py/src/lib.rs:51-79).  The
// environment variable FERRUM_GPU_CODE_OBJECT may name a file to load instead.
KernelArtifact fft_code_object();

// Supported shapes (the reference: 1D [2, 12], plan.rs:58; 2D [4, 12],
// crates/ferrum-gpu-py/src/lib.rs:537).  1D is widened to 2^24: single-pass
// up to 2^15 (the whole transform in one workgroup: its registers and LDS),
// multi-pass beyond.
constexpr uint32_t kMinLogN1D = 2, kMaxLogN1D = 24, kMaxLogNSingle = 15;
constexpr uint32_t kMinLogN2D = 4, kMaxLogN2D = 12;

class FftPlan {
public:
    enum class Kind { Stockham1D, MultiPass1D, TwoD };

    static std::unique_ptr<FftPlan> make_1d(HipDevice& dev, const HipBackend::Module& mod, uint32_t log_n,
                                            size_t batch);
    // 2D plan for `batch` row-major images of 2^log_rows x 2^log_cols (the
    // reference's Plan2D is the square case, log_rows == log_cols).
    static std::unique_ptr<FftPlan> make_2d(HipDevice& dev, const HipBackend::Module& mod, uint32_t log_rows,
                                            uint32_t log_cols, size_t batch);

    // Forward or inverse transform of batch transforms from in to out (may alias).
    // Multi-launch plans run chunk by chunk: every pass over chunk_units()
    // transforms (images) before the next chunk, so a chunk's intermediate
    // array stays in the Infinity Cache (chunk_bytes()).  Plans with
    // streams() == 2 run the odd chunks on a second stream of their own with
    // a second workspace, forked from `stream` at the start and joined
    // back at the end (on a capturing stream: every chunk on `stream`).
    // With `events` (launches() of them), events[i] is recorded right after
    // launch i on the stream launch i runs on (chunk_stream()).
    void exec(const void* in, void* out, Direction dir, bool normalize, hipStream_t stream,
              hipEvent_t* events = nullptr) const;
    // 1, or 2 for multi-pass 1D plans of two or more chunks (unless
    // set_streams(1) turned the second stream off).
    int streams() const { return (aux_ && use_aux_) ? 2 : 1; }
    // The most streams this plan can run on (2: it has the second stream's
    // workspace and events).
    int max_streams() const { return aux_ ? 2 : 1; }
    // Runs the plan's chunks on one stream (1) or, where max_streams() is 2,
    // alternately on two (2, the default).  Same bits either way; executions
    // must not be in flight while it changes.
    void set_streams(int n);
    // The stream a chunk's launches run on: 0 the caller's, 1 the device's
    // chunk stream (HipBackend::chunk_stream).
    int chunk_stream(size_t chunk) const { return streams() == 2 ? (int)(chunk & 1) : 0; }
    // exec() on the split layout: real and imaginary parts in separate f32
    // arrays of batch * elems() each (the reference's *_split kernels,
    // kernels_body.rs:509-626).  Single-pass plans read and write the split
    // arrays in their one launch; other plans interleave into a staging buffer
    // (allocated at their first split call), run in place there and
    // deinterleave.  out_re/out_im may be in_re/in_im (in place).
    void exec_split(const void* in_re, const void* in_im, void* out_re, void* out_im, Direction dir,
                    bool normalize, hipStream_t stream) const;
    // exec_split staging through `staging` (staging_bytes long, 16-byte
    // aligned device memory the caller owns) instead of the plan's own
    // buffer: allocates nothing.  Single-pass plans use no staging; a plan
    // whose batch needs more than staging_bytes is refused, and a null
    // `staging` fails with `no_staging` as the reason.
    void exec_split_into(const void* in_re, const void* in_im, void* out_re, void* out_im, Direction dir,
                         bool normalize, hipStream_t stream, void* staging, size_t staging_bytes,
                         const std::string& no_staging) const;
    // Launches exec_split makes: one per chunk for single-pass plans (one
    // chunk unless the batch exceeds one launch, fit_launches), launches() +
    // 2 otherwise.
    int split_launches() const { return split_fn_ ? (int)chunks() : launches() + 2; }
    // Whether exec_split stages through an interleaved buffer (multi-launch
    // plans) rather than reading and writing the split arrays directly.
    bool split_staged_exec() const { return split_fn_ == nullptr; }

    Kind kind() const { return kind_; }
    // 1D: log2 of the length; 2D: log2 of the row length (columns).
    uint32_t log_n() const { return log_n_; }
    uint32_t log_rows() const { return log_rows_; }
    size_t batch() const { return batch_; }
    // Complex elements per transform (N, or N*N for 2D).
    size_t elems() const { return size_t(1) << (log_n_ + log_rows_); }
    // Kernel launches per execution: passes() per chunk, chunks() chunks.
    int launches() const { return (int)(steps_.size() * chunks()); }
    int passes() const { return (int)steps_.size(); }
    size_t chunk_units() const { return chunk_; }
    size_t chunks() const { return (batch_ + chunk_ - 1) / chunk_; }
    // Whether intermediate arrays are kept cached (chunk fits the cache limit).
    bool cache_resident() const { return cached_; }
    const std::string& main_kernel() const { return main_kernel_; }
    size_t workspace_bytes() const { return work_.bytes() + work2_.bytes(); }
    // Kernel names in launch order of an out-of-place execution, or of an
    // in-place one (in != out): the two differ for the 2D plans of 2048 /
    // 4096 rows of 1024 .. 4096 points, whose out-of-place form runs the row
    // pairs (same launch count).
    std::vector<std::string> kernel_names(bool in_place = false) const;
    // Whether in-place executions run other kernels than out-of-place ones
    // (same transform to rounding, not bit for bit).
    bool in_place_differs() const { return !steps_in_place_.empty(); }

private:
    // Buffers are named symbolically and bound at exec: the caller's input,
    // the caller's output, or the plan's workspace.
    enum class Buf { In, Out, Work };
    struct Step {
        bool tile = false;                      // tile pass (else single-pass Stockham)
        bool small2d = false;                   // one-pass 2D of small images (fg_fft2d_*)
        bool rowpair = false;                   // 2D row pass over row pairs (fg_fft2d_rowpair_*)
        uint32_t log_rows = 0;                  // rowpair: log2 of the image's rows
        const void* tw_cols = nullptr;          // small2d: the column stage table
        std::string name;
        HipBackend::KernelHandle fn = nullptr;
        Dim3 block;
        uint32_t fpb = 1;                       // Stockham: transforms per workgroup
        Buf src = Buf::In, dst = Buf::Out;
        const void* tw = nullptr;               // Stockham stage table
        // Per unit (one transform, or one 2D image): Stockham transforms, or
        // tiles of a tile pass.  A launch over u units has per_unit * u of them.
        uint64_t per_unit = 0;
        uint32_t tile_order = 0;                // tile: TileGeom::remap (FG_TILE_ORDER_*) when the grid
        uint32_t order_unit = 1;                // is a multiple of order_unit, else the natural order
        TileGeom geom{};                        // tile: addressing (flags/scale/remap set at exec)
    };

    // The second stream of a two-stream plan -- the device's one chunk stream,
    // shared by every two-stream plan on the device (HipBackend::chunk_stream)
    // -- and the plan's own fork / join events, released with the plan after
    // its last join has completed.
    struct ChunkStream {
        explicit ChunkStream(const HipBackend::DeviceHandle& dev);
        ~ChunkStream();
        ChunkStream(const ChunkStream&) = delete;
        ChunkStream& operator=(const ChunkStream&) = delete;
        HipBackend::DeviceHandle dev;
        hipStream_t stream = nullptr;  // not owned
        hipEvent_t fork = nullptr, join = nullptr;
    };

    FftPlan(HipDevice& dev, Kind kind, uint32_t log_n, uint32_t log_rows, size_t batch)
        : dev_(&dev), kind_(kind), log_n_(log_n), log_rows_(log_rows), batch_(batch), chunk_(batch) {}

    float scale_for(Direction dir, bool normalize) const;
    // The split-layout paths: argument checks, the one launch of single-pass
    // plans, and interleave -> exec in place -> deinterleave through `stage`.
    void check_split(const void* in_re, const void* in_im, const void* out_re, const void* out_im) const;
    void split_one_launch(const void* in_re, const void* in_im, void* out_re, void* out_im, Direction dir,
                          bool normalize, hipStream_t stream) const;
    void split_staged(const void* in_re, const void* in_im, void* out_re, void* out_im, Direction dir,
                      bool normalize, hipStream_t stream, Cf32* stage) const;
    // Stage table for a length-2^log_l Stockham transform with 2^log_e elements
    // per thread (uploaded once per plan).
    const void* stage_table(uint32_t log_l, uint32_t log_e);
    const void* big_table();
    void add_stockham(const HipBackend::Module& mod, uint32_t log_l, uint64_t per_unit, Buf src, Buf dst,
                      const char* policy = "", bool latency = false);
    // Narrow tiles (g < 16) override `policy` with "_cc" (fft_plan.cpp).
    void add_tile(const HipBackend::Module& mod, uint32_t log_l, uint32_t g, bool rowwise, const TileGeom& geom,
                  uint64_t tiles_per_unit, Buf src, Buf dst, const char* policy);
    // Chunking of a multi-launch plan (sets chunk_ and cached_) and the cache
    // policy suffix of pass i of n.
    // chunk_ and cached_ for the chunk limit: chunks of half of it when the
    // plan's shape runs two chunks at a time (two_in_flight) and the batch
    // makes two or more of them (returns true), else of all of it.
    bool choose_chunk(bool two_in_flight);
    const char* policy(size_t i, size_t n) const;
    // Lowers chunk_ so that every launch of steps_ and steps_in_place_ fits
    // one HIP dispatch (launch_limits.h): a batch beyond that runs in
    // several launches.  Called once the steps are built; a workspace sized
    // for the old chunk_ stays large enough.
    void fit_launches();

    HipDevice* dev_;
    Kind kind_;
    uint32_t log_n_;
    uint32_t log_rows_;  // 0 for 1D
    size_t batch_;
    size_t chunk_;         // units per chunk (batch_ when not chunked)
    bool cached_ = false;  // intermediates kept cached (else every pass streams)
    std::vector<Step> steps_;
    std::vector<Step> steps_in_place_;  // when not empty: the passes of in-place executions (in == out)
    std::vector<std::pair<uint32_t, Buffer<Cf32, HipBackend>>> stage_tables_;
    Buffer<Cf32, HipBackend> big_;
    Buffer<Cf32, HipBackend> work_;
    Buffer<Cf32, HipBackend> work2_;         // the odd chunks' workspace (two-stream 1D plans)
    std::unique_ptr<ChunkStream> aux_;       // two-stream plans: the odd chunks' stream
    bool use_aux_ = true;                    // set_streams
    std::string main_kernel_;
    HipBackend::KernelHandle split_fn_ = nullptr;  // single-pass plans: the split-layout twin
    Pointwise pw_;
    mutable std::mutex stage_mu_;                   // guards the lazy allocation of stage_
    mutable Buffer<Cf32, HipBackend> stage_;        // split layout staging of multi-launch plans
};

// ---- host-side pieces exposed for the CPU tests of the plan logic ----------

// Mixed-radix Stockham table for N = 2^log_n with 2^log_e elements per thread:
// per stage s >= 1 (L = 2^(s*log_e), R = that stage's radix) one row per k < L
// of W_{L*R}^{p*k} for p in {1,2,3,4,8,12} (R = 16), {1,2,3,4} (R = 8) or
// [0, R) (R <= 4), computed in fp64 and rounded to f32 (the kernels form the
// remaining exponents as products; kernels/fft_stockham.hpp).  A stage with
// L >= 1024 stores the two-level block W^{64 h} (h < L/64), W^l (l < 64).
std::vector<Cf32> stockham_twiddles(uint32_t log_n, uint32_t log_e);
// Stage table of the 1024-point throughput kernels (fg_fft_n10, _split, _sc;
// radix list 8 * 16 * 8, kernels/fft_stockham.hpp fft1024_x2_body): rows
// k < 8 of W_128^{p k}, p in {1,2,3,4,8,12}, then rows k < 128 of
// W_1024^{p k}, p in {1,2,3,4}.
std::vector<Cf32> fft1024_x2_twiddles();
// stage_table key for that layout (in place of elements per thread).
constexpr uint32_t kX2Layout = 63;
// Two-level root table: [j] = W_4096^j, [4096 + j] = W_{2^24}^j, j < 4096.
std::vector<Cf32> big_twiddles();
// Digit split (log2 sizes, slowest digit first) of a 1D length 2^log_n > 32768.
std::vector<uint32_t> split_1d(uint32_t log_n);
// Columns per tile for a pass of length 2^log_l that reads HBM.
uint32_t tile_columns(uint32_t log_l);
// Columns (row-wise: rows) per tile for a pass that reads cache-resident data.
uint32_t cached_tile_columns(uint32_t log_l, bool rowwise);
// Whether a tile pass runs the 32-element kernel with the exchanges in halves
// (fg_tile_l*_g*_h): column passes at the HBM width (tile_columns) of 128 ..
// 1024 points, the 16-column 1D middle pass of 256 points, and the 8-column
// passes of 2048 / 4096 points.
bool use_halves_tile(uint32_t log_l, uint32_t g, bool rowwise);
// Whether a 1D last pass (row-wise) runs the 32-element kernel with the
// exchanges in halves (fg_tile_l*_g*_rh): 32-row tiles of 256 points, 16-row
// tiles of 512 / 1024 points.
bool use_row_halves_tile(uint32_t log_l, uint32_t g, bool rowwise);
// Whether the column FFT of an image with 2^log_rows rows runs as two passes.
bool split_2d_columns(uint32_t log_rows);
// Largest chunk (bytes of one chunk's array) a multi-launch plan created from
// now on runs with its intermediates cached: FERRUM_GPU_CHUNK_MIB at load, else
// 128 MiB (half the 256 MB Infinity Cache).  0 = no chunking: one chunk of
// the whole batch, every pass streaming.
size_t chunk_limit_bytes();
void set_chunk_limit_bytes(size_t bytes);
// Units per chunk for `unit_bytes` per transform (image), and whether the
// chunk's intermediates are kept cached, under the given limit.
size_t chunk_units_for(uint64_t unit_bytes, size_t batch, size_t limit, bool* cached);
// Whether a single-pass plan of `count` transforms of 2^log_n points runs the
// latency geometry (fg_fft_n<L>_lat) on a device with `cu_count` CUs.
bool use_latency_geometry(uint32_t log_n, uint64_t count, int cu_count);

}  // namespace fg

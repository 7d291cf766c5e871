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
#include <string>
#include <vector>

#include "device.hpp"
#include "hip_backend.hpp"

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
// crates/ferrum-gpu-py/src/lib.rs:537).  1D is widened to 2^24 by the
// two-pass decomposition.
constexpr uint32_t kMinLogN1D = 2, kMaxLogN1D = 24, kMaxLogNSingle = 12;
constexpr uint32_t kMinLogN2D = 4, kMaxLogN2D = 12;

class FftPlan {
public:
    enum class Kind { Stockham1D, FourStep1D, TwoD };

    static std::unique_ptr<FftPlan> make_1d(HipDevice& dev, const HipBackend::Module& mod, uint32_t log_n,
                                            size_t batch);
    static std::unique_ptr<FftPlan> make_2d(HipDevice& dev, const HipBackend::Module& mod, uint32_t log_n,
                                            size_t batch);

    // Forward or inverse transform of batch transforms from in to out (may alias).
    void exec(const void* in, void* out, Direction dir, bool normalize, hipStream_t stream) const;

    Kind kind() const { return kind_; }
    uint32_t log_n() const { return log_n_; }
    size_t batch() const { return batch_; }
    // Complex elements per transform (N, or N*N for 2D).
    size_t elems() const { return kind_ == Kind::TwoD ? (size_t(1) << (2 * log_n_)) : (size_t(1) << log_n_); }
    int launches() const { return (int)steps_.size(); }
    const std::string& main_kernel() const { return main_kernel_; }
    size_t workspace_bytes() const { return work_.bytes(); }

private:
    // One kernel launch.  Buffers are named symbolically and bound at exec:
    // the caller's input, the caller's output, or the plan's workspace.
    enum class Buf { In, Out, Work };
    struct Step {
        HipBackend::KernelHandle fwd = nullptr;  // kernel used for the forward direction
        HipBackend::KernelHandle inv = nullptr;  // kernel used for the inverse direction
        Dim3 grid, block;
        Buf src = Buf::In, dst = Buf::Out;
        const void* tw = nullptr;  // twiddle table in HBM
        uint64_t count = 0;        // transforms (or tiles) the launch covers
        uint64_t p0 = 0, p1 = 0;   // kernel-specific scalars
        bool scales = false;       // applies the inverse's conjugate+scale on store
        bool conj_in = false;      // applies the inverse's input conjugation on load
    };

    FftPlan(HipDevice& dev, Kind kind, uint32_t log_n, size_t batch)
        : dev_(&dev), kind_(kind), log_n_(log_n), batch_(batch) {}

    HipDevice* dev_;
    Kind kind_;
    uint32_t log_n_;
    size_t batch_;
    std::vector<Step> steps_;
    std::vector<Buffer<Cf32, HipBackend>> tables_;
    Buffer<Cf32, HipBackend> work_;
    std::string main_kernel_;
};

// Host twiddle tables (exposed for the CPU-side tests of the plan logic).
// Mixed-radix Stockham table for N = 2^log_n with 2^log_e elements per thread:
// per stage s >= 1 (L = 2^(s*log_e), R = that stage's radix) the block
// [k][p] = W_{L*R}^{p*k}, k < L, p < R, computed in fp64 and rounded to f32.
std::vector<Cf32> stockham_twiddles(uint32_t log_n, uint32_t log_e);

}  // namespace fg

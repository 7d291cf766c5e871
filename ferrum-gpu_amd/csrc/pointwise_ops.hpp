// pointwise_ops.hpp -- host launchers of the elementwise complex kernels
// (kernels/pointwise.hpp): the reference's cmul_interleaved, cmul_split,
// deinterleave and interleave (kernels_body.rs:1612-1672), which it defines
// for its split-layout study and never launches from the FFT path; the
// seeded synthetic-data generator (kernels/fill.hpp); and the two
// data-movement kernels of the code object, the tiled transpose and the
// streaming copy.
//
// Every kernel handle is resolved once, from the module of the device the
// object belongs to, when the device is opened: a handle never outlives the
// module it came from.
//
// n counts complex elements.  Each launcher picks the 16-byte-access kernel
// when every pointer is 16-byte aligned and the element-wise one otherwise;
// both give identical results.  All are stream-ordered and asynchronous.
#pragma once

#include <cstdint>

#include "device.hpp"
#include "hip_backend.hpp"

namespace fg {

class Pointwise {
public:
    explicit Pointwise(const HipBackend::Module& mod);
    Pointwise() = default;

    // out[i] = a[i] * b[i]; complex64 interleaved.  out may alias a or b.
    void cmul_c64(const HipBackend::DeviceHandle& dev, const void* a, const void* b, void* out, uint64_t n,
                  hipStream_t stream) const;
    // (o_re, o_im)[i] = (a_re, a_im)[i] * (b_re, b_im)[i]; split layout.
    void cmul_split(const HipBackend::DeviceHandle& dev, const void* a_re, const void* a_im, const void* b_re,
                    const void* b_im, void* o_re, void* o_im, uint64_t n, hipStream_t stream) const;
    // re[i] = in[i].re, im[i] = in[i].im.  Outputs must not alias the input.
    void deinterleave(const HipBackend::DeviceHandle& dev, const void* in, void* re, void* im, uint64_t n,
                      hipStream_t stream) const;
    // out[i] = (re[i], im[i]).  The output must not alias the inputs.
    void interleave(const HipBackend::DeviceHandle& dev, const void* re, const void* im, void* out, uint64_t n,
                    hipStream_t stream) const;
    // n seeded complex64 values (kernels/fill.hpp): uniform in [-1, 1), or
    // standard normal when `normal`.  out must be 8-byte aligned.
    void fill_c64(const HipBackend::DeviceHandle& dev, void* out, uint64_t n, uint64_t seed, bool normal,
                  hipStream_t stream) const;
    // out[b][c][r] = in[b][r][c] for `batch` rows x cols complex64 matrices
    // (fg_transpose_c64); in and out must not alias.
    void transpose_c64(const HipBackend::DeviceHandle& dev, const void* in, void* out, uint32_t rows, uint32_t cols,
                       uint64_t batch, hipStream_t stream) const;
    // Streaming copy of `bytes` (a multiple of 16, both pointers 16-byte
    // aligned) with fg_copy_f4, the plain-copy yardstick of the benchmark.
    void stream_copy(const HipBackend::DeviceHandle& dev, const void* in, void* out, uint64_t bytes,
                     hipStream_t stream) const;

private:
    // [0]: one element per thread step, any alignment; [1]: 16-byte accesses.
    HipBackend::KernelHandle cmul_c64_[2] = {nullptr, nullptr};
    HipBackend::KernelHandle cmul_split_[2] = {nullptr, nullptr};
    HipBackend::KernelHandle deinterleave_[2] = {nullptr, nullptr};
    HipBackend::KernelHandle interleave_[2] = {nullptr, nullptr};
    HipBackend::KernelHandle fill_ = nullptr;
    HipBackend::KernelHandle transpose_ = nullptr;
    HipBackend::KernelHandle transpose128_ = nullptr;
    HipBackend::KernelHandle copy_ = nullptr;
};

}  // namespace fg

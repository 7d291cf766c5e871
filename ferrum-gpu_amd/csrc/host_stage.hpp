// host_stage.hpp -- host <-> device copies of the host-array entry points
// (fg_fft_1d_c2c_pow2_host and the 2D ones; the reference's run_fft_flat path,
// crates/ferrum-gpu-py/src/lib.rs:86-250, copies pageable Vec<f32>s).
//
// A pageable hipMemcpy measured 30 GB/s host-to-device and 18 GB/s back on the
// MI355X boxes (10.7 GB/s into a freshly allocated numpy array, whose pages
// fault on first touch), a pinned one 57 GB/s each way.  HostStager moves
// large arrays through two pinned pieces (up to kPiece bytes) per device: the host
// side of each piece is a parallel memcpy (CopyPool, which also takes the
// output's first-touch page faults on several threads), the device side an
// async copy on the device's stream, so filling one piece overlaps the DMA of
// the other.
#pragma once

#include <condition_variable>
#include <cstddef>
#include <mutex>
#include <thread>
#include <vector>

#include "hip_backend.hpp"

namespace fg {

// Process-wide parallel memcpy: the caller and up to kMaxThreads - 1 workers
// copy disjoint page-aligned parts.  One copy at a time; the workers live
// until the process ends.
class CopyPool {
public:
    static constexpr unsigned kMaxThreads = 8;
    static constexpr size_t kMinParallel = 4u << 20;  // below: one memcpy on the caller
    static CopyPool& get();
    void copy(void* dst, const void* src, size_t bytes);
    unsigned threads() const { return (unsigned)workers_.size() + 1; }

private:
    CopyPool();
    void worker();
    void run_parts(std::unique_lock<std::mutex>& lk);

    std::vector<std::thread> workers_;
    std::mutex job_mu_;  // serialises callers
    std::mutex mu_;      // guards the job below
    std::condition_variable work_cv_, done_cv_;
    char* dst_ = nullptr;
    const char* src_ = nullptr;
    size_t bytes_ = 0, part_ = 0, parts_ = 0, next_ = 0, done_ = 0;
    unsigned long long gen_ = 0;
};

// Two pinned pieces of one device (allocated on first use, kept until the
// device closes).  Not thread-safe: the caller holds the device's host-path
// lock.
class HostStager {
public:
    static constexpr size_t kPiece = 64u << 20;
    explicit HostStager(HipBackend::DeviceHandle dev) : dev_(std::move(dev)) {}
    ~HostStager();
    HostStager(const HostStager&) = delete;
    HostStager& operator=(const HostStager&) = delete;

    // Enqueues dst[0, bytes) <- src on `stream`; returns once src has been
    // read (the device copies may still be in flight, ordered on `stream`).
    void to_device(void* dst, const void* src, size_t bytes, hipStream_t stream);
    // dst[0, bytes) <- src after the work already on `stream`; returns once
    // dst holds the data.
    void to_host(void* dst, const void* src, size_t bytes, hipStream_t stream);

    // The piece size used for an array of `bytes`.
    static size_t piece_for(size_t bytes);

private:
    void ensure();
    void wait_slot(int slot);

    HipBackend::DeviceHandle dev_;
    void* pin_[2] = {nullptr, nullptr};
    hipEvent_t done_[2] = {nullptr, nullptr};  // the slot's last device copy
    bool pending_[2] = {false, false};
};

}  // namespace fg

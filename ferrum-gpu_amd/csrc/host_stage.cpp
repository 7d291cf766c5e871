// host_stage.cpp -- see host_stage.hpp.
#include "host_stage.hpp"

#include <string.h>

#include <algorithm>

namespace fg {

CopyPool& CopyPool::get() {
    // Never destroyed: the workers wait on the pool until the process ends.
    static CopyPool* pool = new CopyPool();
    return *pool;
}

CopyPool::CopyPool() {
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned n = std::min(kMaxThreads, hw);
    for (unsigned i = 1; i < n; ++i) {
        workers_.emplace_back([this] { worker(); });
        workers_.back().detach();
    }
}

// Called with mu_ held; copies parts until none is left.
void CopyPool::run_parts(std::unique_lock<std::mutex>& lk) {
    while (next_ < parts_) {
        const size_t i = next_++;
        const size_t off = i * part_;
        const size_t len = std::min(part_, bytes_ - off);
        char* dst = dst_;
        const char* src = src_;
        lk.unlock();
        memcpy(dst + off, src + off, len);
        lk.lock();
        if (++done_ == parts_) done_cv_.notify_all();
    }
}

void CopyPool::worker() {
    unsigned long long seen = 0;
    std::unique_lock<std::mutex> lk(mu_);
    for (;;) {
        work_cv_.wait(lk, [&] { return gen_ != seen; });
        seen = gen_;
        run_parts(lk);
    }
}

void CopyPool::copy(void* dst, const void* src, size_t bytes) {
    if (bytes < kMinParallel || workers_.empty()) {
        memcpy(dst, src, bytes);
        return;
    }
    std::lock_guard<std::mutex> job(job_mu_);
    std::unique_lock<std::mutex> lk(mu_);
    const size_t n = threads();
    // Page-aligned parts, a few per thread so that a slow page does not stall one.
    const size_t part = ((bytes / (4 * n) + 4095) / 4096) * 4096;
    dst_ = static_cast<char*>(dst);
    src_ = static_cast<const char*>(src);
    bytes_ = bytes;
    part_ = std::max<size_t>(part, 4096);
    parts_ = (bytes + part_ - 1) / part_;
    next_ = 0;
    done_ = 0;
    ++gen_;
    work_cv_.notify_all();
    run_parts(lk);
    done_cv_.wait(lk, [&] { return done_ == parts_; });
}

HostStager::~HostStager() {
    (void)hipSetDevice(dev_->ordinal);
    for (int s = 0; s < 2; ++s) {
        if (done_[s]) {
            (void)hipEventSynchronize(done_[s]);
            (void)hipEventDestroy(done_[s]);
        }
        if (pin_[s]) (void)hipHostFree(pin_[s]);
    }
}

void HostStager::ensure() {
    if (pin_[0]) return;
    HipBackend::bind(dev_);
    for (int s = 0; s < 2; ++s) {
        hip_check(hipHostMalloc(&pin_[s], kPiece, hipHostMallocDefault), "hipHostMalloc");
        hip_check(hipEventCreateWithFlags(&done_[s], hipEventDisableTiming), "hipEventCreateWithFlags");
    }
}

void HostStager::wait_slot(int slot) {
    if (!pending_[slot]) return;
    hip_check(hipEventSynchronize(done_[slot]), "hipEventSynchronize");
    pending_[slot] = false;
}

size_t HostStager::piece_for(size_t bytes) {
    // About four pieces per array (so that copies and DMA overlap even for a
    // few MiB), 1 MiB .. kPiece, page multiples.
    const size_t mib = 1u << 20;
    const size_t quarter = ((bytes / 4 + mib - 1) / mib) * mib;
    return std::min(kPiece, std::max(mib, quarter));
}

void HostStager::to_device(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (!bytes) return;
    ensure();
    HipBackend::bind(dev_);
    char* d = static_cast<char*>(dst);
    const char* h = static_cast<const char*>(src);
    const size_t piece = piece_for(bytes);
    for (size_t off = 0, p = 0; off < bytes; off += piece, ++p) {
        const int slot = (int)(p & 1);
        const size_t n = std::min(piece, bytes - off);
        wait_slot(slot);  // the slot's previous device copy has read it
        CopyPool::get().copy(pin_[slot], h + off, n);
        hip_check(hipMemcpyAsync(d + off, pin_[slot], n, hipMemcpyHostToDevice, stream), "hipMemcpyAsync(H2D)");
        hip_check(hipEventRecord(done_[slot], stream), "hipEventRecord");
        pending_[slot] = true;
    }
}

void HostStager::to_host(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (!bytes) return;
    ensure();
    HipBackend::bind(dev_);
    char* h = static_cast<char*>(dst);
    const char* d = static_cast<const char*>(src);
    const size_t piece = piece_for(bytes);
    const size_t pieces = (bytes + piece - 1) / piece;
    auto enqueue = [&](size_t p) {
        const int slot = (int)(p & 1);
        const size_t off = p * piece, n = std::min(piece, bytes - off);
        wait_slot(slot);
        hip_check(hipMemcpyAsync(pin_[slot], d + off, n, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(D2H)");
        hip_check(hipEventRecord(done_[slot], stream), "hipEventRecord");
        pending_[slot] = true;
    };
    enqueue(0);
    if (pieces > 1) enqueue(1);
    for (size_t p = 0; p < pieces; ++p) {
        const int slot = (int)(p & 1);
        const size_t off = p * piece, n = std::min(piece, bytes - off);
        wait_slot(slot);  // piece p has arrived
        CopyPool::get().copy(h + off, pin_[slot], n);
        if (p + 2 < pieces) enqueue(p + 2);
    }
}

}  // namespace fg

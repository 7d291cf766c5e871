// device.hpp -- the Device<B> / Buffer<T, B> facade over a backend
// (crates/ferrum-gpu/src/device.rs:12-64, crates/ferrum-gpu/src/buffer.rs:8-47).
//
// Device owns the backend device handle, its default stream and a module cache
// keyed by module name behind a mutex (device.rs:41-53).  Buffer<T, B> owns one
// zero-initialised device allocation of `len` elements and frees it on
// destruction after the default stream drains (crates/ferrum-gpu-cuda/src/buffer.rs:45-56).
#pragma once

#include <map>
#include <mutex>
#include <string>
#include <type_traits>
#include <utility>

#include "backend.hpp"

namespace fg {

template <class T, class B>
class Buffer;

template <class B>
class Device {
public:
    using Handle = typename B::DeviceHandle;

    explicit Device(Handle h) : h_(std::move(h)) {}
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;

    const Handle& handle() const { return h_; }
    typename B::Stream default_stream() const { return B::default_stream(h_); }

    // Device::sync (device.rs:36-38).
    void sync() const { B::sync_stream(h_, B::default_stream(h_)); }

    // Device::alloc (device.rs:30-33): n zeroed elements of T.
    template <class T>
    Buffer<T, B> alloc(size_t n) const {
        static_assert(std::is_trivially_copyable<T>::value, "device buffers hold plain data");
        return Buffer<T, B>(h_, n);
    }

    // Device::load_or_cache (device.rs:41-53): one load per module name.
    typename B::Module load_or_cache(const KernelArtifact& art) {
        std::lock_guard<std::mutex> g(mu_);
        auto it = modules_.find(art.name);
        if (it != modules_.end()) return it->second;
        auto m = B::load_module(h_, art);
        modules_.emplace(art.name, m);
        return m;
    }

private:
    Handle h_;
    std::mutex mu_;
    std::map<std::string, typename B::Module> modules_;
};

template <class T, class B>
class Buffer {
public:
    Buffer() = default;
    Buffer(typename B::DeviceHandle dev, size_t n)
        : dev_(std::move(dev)), len_(n), ptr_(static_cast<T*>(B::alloc_zeros(dev_, n * sizeof(T)))) {}
    Buffer(const Buffer&) = delete;
    Buffer& operator=(const Buffer&) = delete;
    Buffer(Buffer&& o) noexcept { swap(o); }
    Buffer& operator=(Buffer&& o) noexcept {
        if (this != &o) {
            reset();
            swap(o);
        }
        return *this;
    }
    ~Buffer() { reset(); }

    size_t len() const { return len_; }
    size_t bytes() const { return len_ * sizeof(T); }
    T* data() const { return ptr_; }

    // Buffer::copy_from_host (buffer.rs:14-30): src.len() <= len.
    void copy_from_host(const T* src, size_t n) {
        if (n > len_) invalid("copy_from_host: source longer than the buffer");
        B::copy_h2d(dev_, ptr_, src, n * sizeof(T));
    }
    // Buffer::copy_to_host (buffer.rs:32-46): dst.len() >= len.
    void copy_to_host(T* dst, size_t n) const {
        if (n < len_) invalid("copy_to_host: destination shorter than the buffer");
        B::copy_d2h(dev_, dst, ptr_, len_ * sizeof(T));
    }

    void reset() {
        if (ptr_) {
            try {
                B::free(dev_, ptr_);
            } catch (...) {
            }
        }
        ptr_ = nullptr;
        len_ = 0;
    }

private:
    void swap(Buffer& o) {
        std::swap(dev_, o.dev_);
        std::swap(len_, o.len_);
        std::swap(ptr_, o.ptr_);
    }
    typename B::DeviceHandle dev_{};
    size_t len_ = 0;
    T* ptr_ = nullptr;
};

}  // namespace fg

// backend.hpp -- backend-agnostic vocabulary of the substrate, restated for
// C++: BackendId, Dim3, Direction, KernelArtifact and the error type
// (crates/ferrum-gpu-core/src/{artifact,dim,error}.rs in the reference).
#pragma once

#include <stdint.h>

#include <stdexcept>
#include <string>

#include "ferrum_gpu.h"

namespace fg {

// crates/ferrum-gpu-core/src/artifact.rs:13-36, with Hip added.
enum class BackendId : uint8_t { Cuda = FG_BACKEND_CUDA, Vulkan = FG_BACKEND_VULKAN, Hip = FG_BACKEND_HIP };

// crates/ferrum-gpu-core/src/dim.rs:10-47
struct Dim3 {
    uint32_t x = 1, y = 1, z = 1;
    constexpr Dim3() = default;
    constexpr Dim3(uint32_t x_, uint32_t y_ = 1, uint32_t z_ = 1) : x(x_), y(y_), z(z_) {}
    constexpr uint64_t product() const { return (uint64_t)x * y * z; }
};

// crates/ferrum-gpu-core/src/dim.rs:52-64
enum class Direction : int8_t { Forward = FG_FORWARD, Inverse = FG_INVERSE };

// crates/ferrum-gpu-core/src/artifact.rs:96-116: a compiled module plus the
// metadata needed to refuse it on the wrong backend or target.
struct KernelArtifact {
    BackendId backend = BackendId::Hip;
    std::string name;    // module name (the reference keys its cache by crate name)
    std::string target;  // gfx target the image was built for, e.g. "gfx950"
    const void* image = nullptr;
    size_t size = 0;
};

// Typed error carrying one of the FG_ERR_* codes
// (crates/ferrum-gpu-cuda/src/error.rs:9-34, crates/ferrum-gpu-core/src/error.rs:11-37).
class Error : public std::runtime_error {
public:
    Error(int code, const std::string& msg) : std::runtime_error(msg), code_(code) {}
    int code() const { return code_; }

private:
    int code_;
};

[[noreturn]] inline void fail(int code, const std::string& msg) { throw Error(code, msg); }
[[noreturn]] inline void invalid(const std::string& msg) { throw Error(FG_ERR_INVALID_ARGUMENT, msg); }

}  // namespace fg

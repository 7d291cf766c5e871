// hip_backend.hpp -- the Backend contract implemented over libamdhip64.
//
// Mirrors the reference's `Backend` trait (crates/ferrum-gpu-core/src/backend.rs:12-77)
// as a C++ traits class: associated handle types plus static operations, so
// `Device<B>` and `Buffer<T, B>` (device.hpp) stay generic over the backend the
// way the Rust facade is.  This is the only file that talks to HIP.
#pragma once

#include <hip/hip_runtime_api.h>

#include <functional>
#include <memory>
#include <mutex>
#include <string>

#include "backend.hpp"

namespace fg {

// Owned per-device state: the ordinal, the default stream (default priority)
// and the properties read at open.
struct HipDeviceState {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    // The device's chunk stream (HipBackend::chunk_stream), created on first
    // use; default priority like every stream here.
    std::mutex chunk_mu;
    hipStream_t chunk_stream = nullptr;
    std::string arch;  // gcnArchName up to the first ':' (e.g. "gfx950")
    int cu_count = 0;
    int clock_khz = 0;
    size_t total_mem = 0;
    ~HipDeviceState();
};

struct HipModuleState {
    int ordinal = 0;
    hipModule_t module = nullptr;
    std::string name;
    ~HipModuleState();
};

// A captured launch sequence: the graph and its executable instance.
struct HipGraphState {
    int ordinal = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    size_t nodes = 0;
    ~HipGraphState();
};

struct HipBackend {
    using DeviceHandle = std::shared_ptr<HipDeviceState>;
    using Stream = hipStream_t;
    using Module = std::shared_ptr<HipModuleState>;
    using KernelHandle = hipFunction_t;
    using Graph = std::shared_ptr<HipGraphState>;

    static BackendId id() { return BackendId::Hip; }

    static int device_count();
    static DeviceHandle open(int ordinal);
    // Makes the device current on the calling thread.
    static void bind(const DeviceHandle& dev);

    // Backend::alloc_zeros (backend.rs:30-33), in bytes.
    static void* alloc_zeros(const DeviceHandle& dev, size_t bytes);
    // Drop of the buffer (crates/ferrum-gpu-cuda/src/buffer.rs:45-56).
    static void free(const DeviceHandle& dev, void* ptr);
    // Backend::copy_h2d / copy_d2h (backend.rs:35-47): synchronous.
    static void copy_h2d(const DeviceHandle& dev, void* dst, const void* src, size_t bytes);
    static void copy_d2h(const DeviceHandle& dev, void* dst, const void* src, size_t bytes);
    static void copy_async(const DeviceHandle& dev, void* dst, const void* src, size_t bytes,
                           hipMemcpyKind kind, Stream stream);

    // Backend::load_module (backend.rs:50-53): refuses artifacts of another
    // backend or gfx target.
    static Module load_module(const DeviceHandle& dev, const KernelArtifact& art);
    // Backend::get_kernel (backend.rs:56-59).
    static KernelHandle get_kernel(const Module& mod, const char* name);
    // Backend::launch (backend.rs:62-70): args[i] points at argument i's bytes.
    static void launch(const DeviceHandle& dev, Stream stream, KernelHandle k, Dim3 grid, Dim3 block,
                       uint32_t shared_bytes, void** args);

    // launch() whose completion stamps `stop` (as if it were recorded on the
    // stream right after the kernel), from the dispatch itself rather than a
    // separate marker packet between kernels: per-kernel timing that leaves
    // back-to-back launches back to back.
    static void launch_stamped(const DeviceHandle& dev, Stream stream, KernelHandle k, Dim3 grid, Dim3 block,
                               uint32_t shared_bytes, void** args, hipEvent_t stop);

    // Backend::default_stream / sync_stream (backend.rs:73-76).
    static Stream default_stream(const DeviceHandle& dev) { return dev->stream; }
    static void sync_stream(const DeviceHandle& dev, Stream stream);

    static Stream create_stream(const DeviceHandle& dev);
    static void destroy_stream(const DeviceHandle& dev, Stream s);
    // The one extra stream per device on which two-stream FFT plans run their
    // odd chunks (created at the first call, destroyed with the device), so
    // such plans add one stream to the device however many exist: with four
    // hardware queues per process (GPU_MAX_HW_QUEUES), each plan's own stream
    // would push the chunk stream onto a queue shared with the caller's.
    static Stream chunk_stream(const DeviceHandle& dev);

    // Runs `record` on a private stream under thread-local stream capture and
    // instantiates what it enqueued as one executable graph; nothing executes
    // until launch_graph.  `record` may enqueue kernel launches and event
    // records only (no memsets, no allocation).
    static Graph capture(const DeviceHandle& dev, const std::function<void(Stream)>& record);
    // The two halves of capture() for callers that record across calls:
    // begin_capture returns a new stream in thread-local capture mode;
    // end_capture ends it, destroys the stream and instantiates the graph
    // (or throws, also destroying the stream, if the capture failed).
    static Stream begin_capture(const DeviceHandle& dev);
    static Graph end_capture(const DeviceHandle& dev, Stream s);
    // Enqueues one replay of the graph on `stream` (nullptr: the default stream).
    static void launch_graph(const DeviceHandle& dev, const Graph& g, Stream stream);
};

// Throws fg::Error(FG_ERR_DRIVER or a closer code) naming the failed call.
void hip_check(hipError_t e, const char* what);

}  // namespace fg

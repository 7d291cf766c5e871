// hip_backend.cpp -- HipBackend over libamdhip64 (the replacement of the
// reference's cudarc-based `impl Backend for Cuda`,
// crates/ferrum-gpu-cuda/src/backend_impl.rs:20-184).
#include "hip_backend.hpp"

#include <string.h>

#include "launch_limits.h"

// The launch extension of libamdhip64 that stamps start / stop events from
// the kernel dispatch itself (declared in hip/hip_ext.h, whose C++ templates
// need the HIP compiler; this file is plain g++).
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY,
                                               uint32_t globalWorkSizeZ, uint32_t localWorkSizeX,
                                               uint32_t localWorkSizeY, uint32_t localWorkSizeZ,
                                               size_t sharedMemBytes, hipStream_t hStream, void** kernelParams,
                                               void** extra, hipEvent_t startEvent, hipEvent_t stopEvent,
                                               uint32_t flags);

namespace fg {

void hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    int code = FG_ERR_DRIVER;
    if (e == hipErrorOutOfMemory) code = FG_ERR_OUT_OF_MEMORY;
    else if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) code = FG_ERR_NO_DEVICE;
    else if (e == hipErrorNotFound) code = FG_ERR_KERNEL_NOT_FOUND;
    else if (e == hipErrorNoBinaryForGpu || e == hipErrorInvalidImage) code = FG_ERR_TARGET_MISMATCH;
    fail(code, std::string(what) + " failed: " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
}

HipDeviceState::~HipDeviceState() {
    for (hipStream_t s : {chunk_stream, stream}) {
        if (!s) continue;
        (void)hipSetDevice(ordinal);
        (void)hipStreamSynchronize(s);
        (void)hipStreamDestroy(s);
    }
}

HipModuleState::~HipModuleState() {
    if (module) {
        (void)hipSetDevice(ordinal);
        (void)hipModuleUnload(module);
    }
}

HipGraphState::~HipGraphState() {
    (void)hipSetDevice(ordinal);
    // A replay may still be in flight on any stream of the device.
    if (exec) (void)hipDeviceSynchronize();
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
}

int HipBackend::device_count() {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) return 0;
    hip_check(e, "hipGetDeviceCount");
    return n;
}

HipBackend::DeviceHandle HipBackend::open(int ordinal) {
    int n = device_count();
    if (n == 0) fail(FG_ERR_NO_DEVICE, "no HIP device is visible");
    if (ordinal < 0 || ordinal >= n)
        fail(FG_ERR_NO_DEVICE, "device ordinal " + std::to_string(ordinal) + " out of range (" +
                                   std::to_string(n) + " visible)");
    auto dev = std::make_shared<HipDeviceState>();
    dev->ordinal = ordinal;
    hip_check(hipSetDevice(ordinal), "hipSetDevice");
    hipDeviceProp_t p;
    hip_check(hipGetDeviceProperties(&p, ordinal), "hipGetDeviceProperties");
    std::string arch = p.gcnArchName;
    dev->arch = arch.substr(0, arch.find(':'));
    dev->cu_count = p.multiProcessorCount;
    dev->clock_khz = p.clockRate;
    dev->total_mem = p.totalGlobalMem;
    // Default priority on purpose: streams of different priorities are never mixed.
    hip_check(hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    return dev;
}

void HipBackend::bind(const DeviceHandle& dev) { hip_check(hipSetDevice(dev->ordinal), "hipSetDevice"); }

void* HipBackend::alloc_zeros(const DeviceHandle& dev, size_t bytes) {
    bind(dev);
    void* p = nullptr;
    if (bytes == 0) return nullptr;
    hip_check(hipMalloc(&p, bytes), "hipMalloc");
    hipError_t e = hipMemsetAsync(p, 0, bytes, dev->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
    if (e != hipSuccess) {
        (void)hipFree(p);
        hip_check(e, "zero-fill of a new buffer");
    }
    return p;
}

void HipBackend::free(const DeviceHandle& dev, void* ptr) {
    if (!ptr) return;
    bind(dev);
    hip_check(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
    hip_check(hipFree(ptr), "hipFree");
}

void HipBackend::copy_h2d(const DeviceHandle& dev, void* dst, const void* src, size_t bytes) {
    if (!bytes) return;
    bind(dev);
    hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, dev->stream), "hipMemcpyAsync(H2D)");
    hip_check(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
}

void HipBackend::copy_d2h(const DeviceHandle& dev, void* dst, const void* src, size_t bytes) {
    if (!bytes) return;
    bind(dev);
    hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, dev->stream), "hipMemcpyAsync(D2H)");
    hip_check(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
}

void HipBackend::copy_async(const DeviceHandle& dev, void* dst, const void* src, size_t bytes,
                            hipMemcpyKind kind, Stream stream) {
    if (!bytes) return;
    bind(dev);
    hip_check(hipMemcpyAsync(dst, src, bytes, kind, stream ? stream : dev->stream), "hipMemcpyAsync");
}

HipBackend::Module HipBackend::load_module(const DeviceHandle& dev, const KernelArtifact& art) {
    // crates/ferrum-gpu-cuda/src/backend_impl.rs:79-81: refuse foreign artifacts.
    if (art.backend != BackendId::Hip)
        fail(FG_ERR_BACKEND_MISMATCH, "backend mismatch: expected " + std::to_string((int)BackendId::Hip) +
                                          ", got " + std::to_string((int)art.backend));
    if (!art.image || art.size == 0) invalid("module image is empty");
    if (!art.target.empty() && art.target != dev->arch)
        fail(FG_ERR_TARGET_MISMATCH, "code object targets " + art.target + " but device " +
                                         std::to_string(dev->ordinal) + " is " + dev->arch);
    bind(dev);
    auto m = std::make_shared<HipModuleState>();
    m->ordinal = dev->ordinal;
    m->name = art.name;
    hip_check(hipModuleLoadData(&m->module, art.image), "hipModuleLoadData");
    return m;
}

HipBackend::KernelHandle HipBackend::get_kernel(const Module& mod, const char* name) {
    hipFunction_t f = nullptr;
    hip_check(hipSetDevice(mod->ordinal), "hipSetDevice");
    hipError_t e = hipModuleGetFunction(&f, mod->module, name);
    if (e != hipSuccess || !f) fail(FG_ERR_KERNEL_NOT_FOUND, std::string("kernel not found: ") + name);
    return f;
}

namespace {

// A launch whose work-items along some dimension exceed the dispatch packet's
// 32-bit grid size is refused here, before HIP sees it (launch_limits.h).
void check_launch(HipBackend::KernelHandle k, Dim3 grid, Dim3 block) {
    if (!k) invalid("launch of a null kernel");
    if (grid.product() == 0 || block.product() == 0) invalid("launch with an empty grid or block");
    if (block.product() > FG_MAX_BLOCK_THREADS)
        invalid("block of " + std::to_string(block.product()) + " threads exceeds 1024");
    const uint32_t g[3] = {grid.x, grid.y, grid.z}, b[3] = {block.x, block.y, block.z};
    for (int d = 0; d < 3; ++d)
        if ((uint64_t)g[d] * b[d] > FG_MAX_LAUNCH_ITEMS)
            invalid("launch of " + std::to_string(g[d]) + " x " + std::to_string(b[d]) + " work-items along one " +
                    "dimension exceeds 2^32 - 1");
}

}  // namespace

void HipBackend::launch(const DeviceHandle& dev, Stream stream, KernelHandle k, Dim3 grid, Dim3 block,
                        uint32_t shared_bytes, void** args) {
    check_launch(k, grid, block);
    bind(dev);
    hip_check(hipModuleLaunchKernel(k, grid.x, grid.y, grid.z, block.x, block.y, block.z, shared_bytes,
                                    stream ? stream : dev->stream, args, nullptr),
              "hipModuleLaunchKernel");
}

void HipBackend::launch_stamped(const DeviceHandle& dev, Stream stream, KernelHandle k, Dim3 grid, Dim3 block,
                                uint32_t shared_bytes, void** args, hipEvent_t stop) {
    check_launch(k, grid, block);
    // The extension takes the grid in work-items (32 bits each, as checked).
    const uint64_t gx = (uint64_t)grid.x * block.x, gy = (uint64_t)grid.y * block.y, gz = (uint64_t)grid.z * block.z;
    bind(dev);
    hip_check(hipExtModuleLaunchKernel(k, (uint32_t)gx, (uint32_t)gy, (uint32_t)gz, block.x, block.y, block.z,
                                       shared_bytes, stream ? stream : dev->stream, args, nullptr, nullptr, stop, 0),
              "hipExtModuleLaunchKernel");
}

void HipBackend::sync_stream(const DeviceHandle& dev, Stream stream) {
    bind(dev);
    hip_check(hipStreamSynchronize(stream ? stream : dev->stream), "hipStreamSynchronize");
}

HipBackend::Stream HipBackend::create_stream(const DeviceHandle& dev) {
    bind(dev);
    hipStream_t s = nullptr;
    hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    return s;
}

HipBackend::Stream HipBackend::chunk_stream(const DeviceHandle& dev) {
    std::lock_guard<std::mutex> lock(dev->chunk_mu);
    if (!dev->chunk_stream) dev->chunk_stream = create_stream(dev);
    return dev->chunk_stream;
}

void HipBackend::destroy_stream(const DeviceHandle& dev, Stream s) {
    if (!s) return;
    bind(dev);
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    hip_check(hipStreamDestroy(s), "hipStreamDestroy");
}

HipBackend::Stream HipBackend::begin_capture(const DeviceHandle& dev) {
    bind(dev);
    hipStream_t s = nullptr;
    hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    hipError_t began = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (began != hipSuccess) {
        (void)hipStreamDestroy(s);
        hip_check(began, "hipStreamBeginCapture");
    }
    return s;
}

HipBackend::Graph HipBackend::end_capture(const DeviceHandle& dev, Stream s) {
    if (!s) invalid("end of capture on a null stream");
    bind(dev);
    auto g = std::make_shared<HipGraphState>();
    g->ordinal = dev->ordinal;
    hipError_t ended = hipStreamEndCapture(s, &g->graph);
    (void)hipStreamDestroy(s);
    hip_check(ended, "hipStreamEndCapture");
    if (!g->graph) invalid("stream capture produced no graph");
    hip_check(hipGraphGetNodes(g->graph, nullptr, &g->nodes), "hipGraphGetNodes");
    hip_check(hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    return g;
}

HipBackend::Graph HipBackend::capture(const DeviceHandle& dev, const std::function<void(Stream)>& record) {
    hipStream_t s = begin_capture(dev);
    try {
        record(s);
    } catch (...) {
        hipGraph_t partial = nullptr;
        (void)hipStreamEndCapture(s, &partial);
        if (partial) (void)hipGraphDestroy(partial);
        (void)hipStreamDestroy(s);
        throw;
    }
    return end_capture(dev, s);
}

void HipBackend::launch_graph(const DeviceHandle& dev, const Graph& g, Stream stream) {
    if (!g || !g->exec) invalid("launch of an empty graph");
    if (g->ordinal != dev->ordinal) invalid("graph belongs to another device");
    bind(dev);
    hip_check(hipGraphLaunch(g->exec, stream ? stream : dev->stream), "hipGraphLaunch");
}

}  // namespace fg

// scratch.hip -- the device array behind fg_fft_exec_split_noalloc and the
// host code that resolves its address (scratch.hpp).
//
// Compiled by hipcc into libferrum_gpu.so (not into the FFT code object):
// the HIP runtime registers this file's code object with the library and
// loads it onto a device, with the array, the first time the array's
// address is asked for on that device.  In host code `scratch` names a
// host-side stand-in, not device memory: only the address hipGetSymbolAddress
// returns, kept per device, is ever passed to kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "scratch.hpp"

static __device__ __align__(256) float2 scratch[fg::kScratchBytes / sizeof(float2)];

namespace fg {

namespace {

std::mutex g_mu;
bool g_done[kScratchMaxDevices] = {};
void* g_ptr[kScratchMaxDevices] = {};
hipError_t g_err[kScratchMaxDevices] = {};

}  // namespace

void scratch_init(int ordinal) {
    if (ordinal < 0 || ordinal >= kScratchMaxDevices) return;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_done[ordinal]) return;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_done[ordinal] = true;
    g_err[ordinal] = e;
    g_ptr[ordinal] = (e == hipSuccess) ? p : nullptr;
}

void* scratch_device_ptr(int ordinal, std::string* why) {
    if (ordinal < 0 || ordinal >= kScratchMaxDevices) {
        if (why) *why = "device ordinal " + std::to_string(ordinal) + " beyond the scratch table";
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_done[ordinal]) {
        if (why) *why = "the scratch area of device " + std::to_string(ordinal) + " was not set up at open";
        return nullptr;
    }
    if (!g_ptr[ordinal]) {
        if (why)
            *why = std::string("hipGetSymbolAddress(scratch) failed at open: ") + hipGetErrorName(g_err[ordinal]);
        return nullptr;
    }
    return g_ptr[ordinal];
}

}  // namespace fg

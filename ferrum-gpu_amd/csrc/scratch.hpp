// scratch.hpp -- the fixed device scratch area behind the allocation-free
// entry point fg_fft_exec_split_noalloc (scratch.hip).
//
// The area is a __device__ array of the code object built from scratch.hip:
// every GPU the library opens holds its own copy, kScratchBytes large, from
// fg_device_open until the process ends.  Its device address is resolved once
// per device, at open, and kept; nothing here allocates afterwards.  Every
// user of the area on one GPU shares it and it keeps the last user's
// contents, so calls that overlap in time on one GPU race.
#pragma once

#include <stddef.h>

#include <string>

namespace fg {

// 64 MiB: 8 Mi complex64 elements (for example one 2^23-point transform, eight
// 2^20-point ones, or two 2048 x 2048 images).
constexpr size_t kScratchBytes = size_t(64) << 20;
constexpr int kScratchMaxDevices = 64;

// Resolves the area's address on device `ordinal`, which must be the calling
// thread's current device (once per device; later calls return at once).  A
// failure is recorded, not thrown: it only matters to the allocation-free
// entry point, which reports it.
void scratch_init(int ordinal);

// The area's device address on `ordinal`, or nullptr with the reason in *why.
void* scratch_device_ptr(int ordinal, std::string* why);

}  // namespace fg

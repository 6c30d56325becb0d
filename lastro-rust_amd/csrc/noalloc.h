// Fixed device scratch of the no-allocation entry point (noalloc.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

namespace moert {

// Bytes of the scratch: a 256-byte header (word 0: the cache length read by the attention kernels), then the split
// partials of up to 64 query heads x 64 splits x 66 floats.
constexpr size_t kNoallocHeader = 256;
constexpr size_t kNoallocScratchBytes = kNoallocHeader + (size_t)64 * 64 * 66 * 4;  // 1,081,600

// The scratch's device address on the current device (taken once per device with hipGetSymbolAddress); null on
// failure with the error in *err.
void* noalloc_scratch(hipError_t* err);

// *p = v by a one-thread kernel on s (a kernel, not a memset, so that the call can be captured into a graph).
hipError_t launch_set_int(hipStream_t s, int* p, int v);

}  // namespace moert

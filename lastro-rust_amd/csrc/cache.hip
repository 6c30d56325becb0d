// Host -> device copy probe for the expert cache: the PCIe read rate that bounds the cached kernels' reads of missed
// experts from the pinned host store. The reference copies experts with cuMemcpyAsync
// (ExpertCache::add_into_with, rust/moe-rt/src/cache.rs:249-354); here the cached kernels read them directly.
#include "cache.h"
#include "launch.h"

namespace moert {

constexpr int kCopyChunk = 64 * 1024;  // bytes per workgroup
constexpr int kCopyThreads = 256;

// Plain copy of `bytes` (multiple of 16) from pinned host memory into device memory by a kernel; all loads of a
// workgroup's 64 KiB are issued before its first store.
__global__ __launch_bounds__(kCopyThreads) void k_h2d_copy(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                           size_t n) {
  constexpr int PER = kCopyChunk / 16 / kCopyThreads;
  const size_t base = (size_t)blockIdx.x * (kCopyChunk / 16) + threadIdx.x;
  uint4 buf[PER];
#pragma unroll
  for (int q = 0; q < PER; q++) {
    const size_t i = base + (size_t)q * kCopyThreads;
    buf[q] = i < n ? src[i] : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int q = 0; q < PER; q++) {
    const size_t i = base + (size_t)q * kCopyThreads;
    if (i < n) dst[i] = buf[q];
  }
}

hipError_t launch_h2d_copy(hipStream_t s, const void* src, void* dst, size_t bytes) {
  const size_t n = bytes / 16;
  const int blocks = (int)((bytes + kCopyChunk - 1) / kCopyChunk);
  klaunch(k_h2d_copy, blocks, kCopyThreads, 0, s, (const uint4*)src, (uint4*)dst, n);
  return hipGetLastError();
}

}  // namespace moert

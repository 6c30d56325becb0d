// Fixed device scratch for the entry point that allocates nothing (moert_attn_decode_noalloc, for callers that
// cannot call hipMalloc: code under graph capture, tight serving loops, harnesses that forbid it). The scratch is a
// file-scope device array of fixed size that each GPU holds until the process ends. Its device address is taken once
// per device, with that device current, by hipGetSymbolAddress (in host code the array's name is only a host-side
// stand-in, never passed to a kernel or a copy), and that address is what the kernels get.
//
// Every call on a GPU uses that GPU's one array: calls that overlap on one GPU (other streams, other threads) race
// on it. Nothing in it has to start at zero: the length word is written by k_set_int on every call, and the attention
// kernels read only the partials of the splits they wrote in the same call.
#include <hip/hip_runtime.h>

#include <mutex>

#include "noalloc.h"

static __device__ __align__(256) unsigned char scratch[moert::kNoallocScratchBytes];

namespace moert {

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

__global__ void k_set_int(int* p, int v) {
  if (threadIdx.x == 0) *p = v;
}

}  // namespace

void* noalloc_scratch(hipError_t* err) {
  int dev = -1;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> l(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    g_ptr[dev] = p;
  }
  *err = hipSuccess;
  return g_ptr[dev];
}

hipError_t launch_set_int(hipStream_t s, int* p, int v) {
  hipLaunchKernelGGL(k_set_int, 1, 64, 0, s, p, v);
  return hipGetLastError();
}

}  // namespace moert

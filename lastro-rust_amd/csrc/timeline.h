// Per-workgroup phase timeline of the decode kernels: a measurement build (MOERT_TIMELINE, libmoert_tl.so) stamps
// the 100 MHz real-time clock at phase boundaries of every workgroup of every launch of a step, so that the time
// a kernel spends in each phase (activation round trip, reductions, weight stream, epilogue) and the gaps between
// kernels can be read from a graph replay of the real step. In the product build every stamp compiles to nothing
// and the Tl argument of a kernel is an unused pointer.
//
// Record of one launch: [blocks][kTlPhases] u64. Slot 0 = ~(earliest wave start), slot 1 = latest wave start,
// slot kTlPhases-1 = latest wave end (all three by atomic max over the workgroup's waves, from a zeroed record);
// slots 2.. kTlPhases-2 = phase ends as seen by wave 0 (plain stores, 0 when the kernel has no such phase).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moert {

constexpr int kTlPhases = 12;
constexpr int kTlMaxBlocks = 1024;  // workgroups per launch with a record (later ones are not stamped)

struct Tl {
  unsigned long long* p;  // this launch's record, or null
};

#ifdef MOERT_TIMELINE
__device__ __forceinline__ unsigned long long tl_now() { return __builtin_amdgcn_s_memrealtime(); }
// The workgroup's record, or null (no record, or a workgroup past kTlMaxBlocks).
__device__ __forceinline__ unsigned long long* tl_rec(const Tl& tl) {
  const unsigned wg = blockIdx.y * gridDim.x + blockIdx.x;
  return tl.p && wg < (unsigned)kTlMaxBlocks ? tl.p + (size_t)wg * kTlPhases : nullptr;
}
// Start of every wave (slot 0 keeps the earliest, slot 1 the latest).
#define TL_START(tl)                                                                                      \
  do {                                                                                                    \
    unsigned long long* r_ = tl_rec(tl);                                                                  \
    if (r_ && (threadIdx.x & 63) == 0) {                                                                  \
      const unsigned long long t_ = tl_now();                                                             \
      __hip_atomic_fetch_max(r_, ~t_, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);                        \
      __hip_atomic_fetch_max(r_ + 1, t_, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);                     \
    }                                                                                                     \
  } while (0)
// End of phase `ph` (2 .. kTlPhases - 2) as wave 0 sees it.
#define TL_PHASE(tl, ph)                                                                                  \
  do {                                                                                                    \
    unsigned long long* r_ = tl_rec(tl);                                                                  \
    if (r_ && threadIdx.x == 0) r_[ph] = tl_now();                                                        \
  } while (0)
// End of every wave (the latest is kept).
#define TL_END(tl)                                                                                        \
  do {                                                                                                    \
    unsigned long long* r_ = tl_rec(tl);                                                                  \
    if (r_ && (threadIdx.x & 63) == 0)                                                                    \
      __hip_atomic_fetch_max(r_ + kTlPhases - 1, tl_now(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   \
  } while (0)
#else
#define TL_START(tl) \
  do {               \
  } while (0)
#define TL_PHASE(tl, ph) \
  do {                   \
  } while (0)
#define TL_END(tl) \
  do {             \
  } while (0)
#endif

}  // namespace moert

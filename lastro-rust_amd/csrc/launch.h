// Kernel launch helper: plain hipLaunchKernelGGL, or hipExtLaunchKernelGGL with the event pair armed on this
// thread (arm_launch_events), whose start/stop events take the dispatch's own timestamps so that the measured
// time is the kernel's execution and not the host's enqueue of separate event markers.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

namespace moert {

// Takes (and clears) the event pair armed on this thread; false when none is armed.
bool take_armed_events(hipEvent_t* start, hipEvent_t* stop);

template <typename F, typename... Args>
static inline void klaunch(F kernel, dim3 grid, dim3 block, uint32_t shm, hipStream_t s, Args... args) {
  hipEvent_t a, z;
  if (take_armed_events(&a, &z))
    hipExtLaunchKernelGGL(kernel, grid, block, shm, s, a, z, 0u, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, shm, s, args...);
}

// Compiled row lengths and the dtype x row-length dispatch of the row-streaming launchers: BODY(KK) is expanded
// with DTC (the dtype constant) and KK (the row length) in scope.
#define MOERT_K_CASES(X) X(128) X(256) X(512) X(1024) X(1536)
#define MOERT_KDOWN_CASES(X) X(128) X(256) X(512)

#define MOERT_DISPATCH(dt, K, BODY)                                   \
  switch (dt) {                                                       \
    case DT_Q8_0: {                                                   \
      constexpr int DTC = DT_Q8_0;                                    \
      switch (K) { MOERT_K_CASES(BODY) default: return hipErrorInvalidValue; } \
    } break;                                                          \
    case DT_Q4_0: {                                                   \
      constexpr int DTC = DT_Q4_0;                                    \
      switch (K) { MOERT_K_CASES(BODY) default: return hipErrorInvalidValue; } \
    } break;                                                          \
    case DT_F32: {                                                    \
      constexpr int DTC = DT_F32;                                     \
      switch (K) { MOERT_K_CASES(BODY) default: return hipErrorInvalidValue; } \
    } break;                                                          \
    default:                                                          \
      return hipErrorInvalidValue;                                    \
  }

}  // namespace moert

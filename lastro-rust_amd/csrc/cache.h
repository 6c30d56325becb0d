// Expert cache on the device (cache.hip): an HBM pool of `slots` experts filled from a pinned host store, with
// the LRU bookkeeping done by a kernel so that a whole decode step stays one graph with no host round trip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace moert {

constexpr int kCacheMaxSlots = 4096;

// Statistics words (unsigned long long): requests that hit, copies from the host store.
enum { CS_HITS = 0, CS_COPIES = 1, CS_WORDS = 4 };

struct CacheDev {
  DMat pool_gu;           // [slots * 2I, H]: slot s holds rows [s*2I, s*2I + 2I) (gate rows, then up rows)
  DMat pool_dn;           // [slots * H, I]
  const uint8_t* host;    // pinned store, one record per key = layer * E + expert: [gu payload | gu scales |
                          // down payload | down scales], record_bytes each
  size_t record_bytes, gu_q, gu_d, dn_q;  // record size and its first three piece sizes (dn_d is the rest)
  int slots;
  int experts;
  int* slot_key;          // [slots] key held by the slot, -1 when free
  int* slot_last;         // [slots] clock of the slot's last use
  int* key_slot;          // [layers * E] slot of a resident key, -1 otherwise
  int* clock;             // [1] one tick per layer step
  unsigned long long* stats;  // [CS_WORDS]
  int* route_slot;        // [k] slots of the current layer's routed experts, top-k order
  int* miss;              // [1 + 2k]: count, then (slot, key) pairs to copy in
};

// Router of layer `layer` (rmsnorm of h, GEMV, optional bias), top-k into b.route_ids / b.route_w of the layer,
// then the LRU decision for its k keys: hits are pinned, misses take the first free slot or else the least
// recently used slot not used in this layer step.
hipError_t launch_route_lru(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                            const CacheDev& c);
// Copies the current miss list from the host store into the pool (PCIe reads by the kernel).
hipError_t launch_fill(hipStream_t s, const CacheDev& c, int k);
// Kernel copy of `bytes` (multiple of 16) from device-mapped pinned host memory to device memory.
hipError_t launch_h2d_copy(hipStream_t s, const void* src, void* dst, size_t bytes);

}  // namespace moert

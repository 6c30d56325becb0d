// Expert cache on the device: an HBM pool of `slots` experts over a pinned host store. Every workgroup of the
// cached gate/up kernel makes the LRU decision of its layer step itself, from the same slot tables, and workgroup 0
// writes the result; an expert that misses is read from the host store by the kernels that use it (gate/up, then
// down), which also write it into its slot. So a whole decode step, copies included, stays one graph of the same
// six kernels per layer as the resident model, with no host round trip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace moert {

constexpr int kCacheMaxSlots = 4096;

// Statistics words (unsigned long long): requests that hit, copies from the host store inside steps, experts copied
// ahead of their layer by the prefetch branch.
enum { CS_HITS = 0, CS_COPIES = 1, CS_PREFETCH = 2, CS_WORDS = 4 };

struct CacheDev {
  DMat pool_gu;           // [slots * 2I, H]: slot s holds rows [s*2I, s*2I + 2I) (gate rows, then up rows)
  DMat pool_dn;           // [slots * H, I]
  const uint8_t* host;    // pinned store, one record per key = layer * E + expert: [gu payload | gu scales |
                          // down payload | down scales], record_bytes each (device address of the mapping)
  size_t record_bytes, gu_q, gu_d, dn_q;  // record size and its first three piece sizes (dn_d is the rest)
  int slots;
  int experts;
  // Two copies of the slot tables and the clock: a layer step reads copy `*cur` and workgroup 0 of the gate/up
  // kernel writes the updated tables into the other copy; the down kernel then switches `*cur`. No kernel writes
  // the copy it reads, so the workgroups of one launch all decide from the same tables.
  int* slot_key;          // [2][slots] key held by the slot, -1 when free
  int* slot_last;         // [2][slots] clock of the slot's last use
  int* clock;             // [2] one tick per layer step
  int* cur;               // [1] the current copy (0 or 1)
  unsigned long long* stats;  // [CS_WORDS]
  int* route;             // [16] the current layer step: slot of each routed expert in top-k order, then its host
                          // key when it missed (read from the host store by the down kernel), -1 when it hit
  // prefetch branch (moert_cache_prefetch_mode)
  int* pf;                // [1 + 2 * 8] experts to copy ahead of the current layer: count, then (slot, key) pairs
  uint2* pfx;             // [1 + 2 * 8] the same list as epoch-tagged entries (prefetch inside the attention launch)
  int* pred_hist;         // [max_len][layers][8] predicted experts of each position and layer (-1: none)
  int* tok_hist;          // [max_len][layers][4] per position and layer: hits, copies, prefetched, 0
  const int* state;       // the step state (ST_POS: the position being decoded)
  int layers;
  // host-CPU hybrid (moert_model_create_hybrid): the token's table, key -> pool slot or -1 (the host computes that
  // expert), decided on the host; the cached kernels then read it instead of deciding, and the gate/up kernel
  // publishes the layer's normalised input for the host
  const int* table;
  float* xn;              // [H]
};

// The MoE half of a layer step of a cached model: rmsnorm + router + top-k + LRU decision + gate/up + SwiGLU of the
// routed experts (k_route_up, cached mode), then down + combine + residual (k_expert_down, cached mode).
hipError_t launch_route_up_cached(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                                  const CacheDev& c, Tl tl = {});
hipError_t launch_expert_down_cached(hipStream_t s, const Dims& d, const StepBufs& b, int layer, const CacheDev& c,
                                     Tl tl = {});
// h[i] += res * y[i] for i < n (hybrid: the host-computed experts of a layer step)
hipError_t launch_add_scaled(hipStream_t s, float* h, const float* y, float res, int n);
// A hybrid layer's doorbell: waits (bounded) for the host's flag word *flag to carry `seq` (flag = seq << 1 | any),
// then adds res * y when any; a flag that never comes sets bit 256 of *err.
hipError_t launch_hy_doorbell_add(hipStream_t s, float* h, const float* y, float res, int n, const unsigned* flag,
                                  unsigned seq, unsigned* err);

// Prefetch branch of a cached step, for layer `layer` (run on a side stream while the layer's attention runs):
// launch_prefetch_decide predicts the layer's experts from its input h (the layer's router on rmsnorm(h, ln_moe),
// top-k), records them in c.pred_hist, applies one uncounted tick of the LRU rule to the current slot tables in place
// and lists the (slot, key) pairs to copy in c.pf; launch_prefetch_copy copies those records from the host store into
// their pool slots.
hipError_t launch_prefetch_decide(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                                  const CacheDev& c);
hipError_t launch_prefetch_copy(hipStream_t s, const CacheDev& c);

// Kernel copy of `bytes` (multiple of 16) from device-mapped pinned host memory to device memory (the PCIe rate
// the cached kernels' host reads are bounded by).
hipError_t launch_h2d_copy(hipStream_t s, const void* src, void* dst, size_t bytes);

}  // namespace moert

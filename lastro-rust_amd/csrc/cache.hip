// Expert cache on the device: routing + LRU bookkeeping in one kernel per layer, and the copy of the misses from
// the pinned host store into the HBM pool by a second kernel (PCIe reads issued by the GPU). The reference does the
// bookkeeping on the host after reading the router logits back every layer and copies with cuMemcpyAsync
// (ExpertCache::add_into_with, rust/moe-rt/src/cache.rs:249-354; Slots, cache/core.rs:117-431). Here the decision
// follows the same LRU rule (the `reference_lru` of tests/model.rs:380-412, the LruSync policy) without leaving
// the device, so the whole decode step, copies included, stays one captured graph.
#include <climits>

#include "cache.h"
#include "dev_rows.h"
#include "launch.h"

namespace moert {

constexpr int kLruThreads = 512;
constexpr int kFillChunk = 64 * 1024;  // bytes of one expert record per fill workgroup
constexpr int kFillThreads = 256;

__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const unsigned lo = __shfl_xor((unsigned)(v & 0xffffffffu), m);
    const unsigned hi = __shfl_xor((unsigned)(v >> 32), m);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    v = o < v ? o : v;
  }
  return v;
}

template <int DT, int K>
__global__ __launch_bounds__(kLruThreads) void k_route_lru(DMat router, const float* __restrict__ bias,
                                                           const float* __restrict__ h, const float* __restrict__ lnw,
                                                           float eps, int k, int layer, int* __restrict__ ids_out,
                                                           float* __restrict__ w_out, CacheDev c) {
  using G = Geo<DT, K>;
  constexpr int NW = kLruThreads / 64;
  constexpr int RP = (64 + NW * G::RPW - 1) / (NW * G::RPW);
  __shared__ float xs[K];
  __shared__ __align__(16) float lg[64];
  __shared__ __align__(16) TopkLds tk;
  __shared__ int sids[8];
  __shared__ float sw[8];
  __shared__ float rs;
  __shared__ int skey[kCacheMaxSlots];
  __shared__ int slast[kCacheMaxSlots];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPR, rw = lane / G::LPR;
  const int E = router.rows, S = c.slots;
  size_t row[RP];
  bool ok[RP];
#pragma unroll
  for (int q = 0; q < RP; q++) {
    row[q] = (size_t)(q * NW + wave) * G::RPW + rw;
    ok[q] = row[q] < (size_t)E;
  }
  Rows<DT, K, RP> rr;
  rows_load<DT, K, RP>(rr, router, row, ok, sub);
  float bv[RP];
#pragma unroll
  for (int q = 0; q < RP; q++) bv[q] = (bias && ok[q]) ? bias[row[q]] : 0.0f;
  for (int i = threadIdx.x; i < S; i += kLruThreads) {
    skey[i] = c.slot_key[i];
    slast[i] = c.slot_last[i];
  }
  const int clock = *c.clock + 1;
  wg_norm<K, kLruThreads>(h, lnw, eps, xs, &rs);
  XReg<DT, K> xr;
  load_x<DT, K>(xr, xs, sub);
  float out[RP];
  rows_fma<DT, K, RP>(rr, ok, xr, sub, out);
#pragma unroll
  for (int q = 0; q < RP; q++)
    if (ok[q] && sub == 0) lg[row[q]] = bias ? out[q] + bv[q] : out[q];
  __syncthreads();
  if (wave == 0) {
    wave_topk(lg, E, k, lane, tk, sids, sw);
    wave_lds_sync();
    int key = 0, s0 = -1;
    if (lane < k) {
      key = layer * c.experts + sids[lane];
      s0 = c.key_slot[key];
      ids_out[lane] = sids[lane];
      w_out[lane] = sw[lane];
    }
    // every requested key that is resident is touched first, so no miss of this step can evict it
    if (lane < k && s0 >= 0) slast[s0] = clock;
    wave_lds_sync();
    int myslot = s0, nmiss = 0, hits = 0;
    for (int j = 0; j < k; j++) {
      const int sj = __shfl(s0, j), keyj = __shfl(key, j);
      if (sj >= 0) {
        hits++;
        continue;
      }
      // victim: the first free slot, else the least recently used slot not used in this step (lowest index)
      unsigned long long best = ~0ull;
      for (int i = lane; i < S; i += 64) {
        const bool freev = skey[i] < 0;
        if (freev || slast[i] < clock) {
          const unsigned long long cand = ((unsigned long long)(freev ? 0u : (unsigned)slast[i] + 1u) << 32) | (unsigned)i;
          best = cand < best ? cand : best;
        }
      }
      best = wave_min_u64(best);
      const int v = (int)(best & 0xffffffffu);  // S >= k guarantees a victim
      if (lane == 0) {
        const int old = skey[v];
        if (old >= 0) c.key_slot[old] = -1;
        c.key_slot[keyj] = v;
        skey[v] = keyj;
        slast[v] = clock;
        c.miss[1 + 2 * nmiss] = v;
        c.miss[2 + 2 * nmiss] = keyj;
      }
      wave_lds_sync();
      if (lane == j) myslot = v;
      nmiss++;
    }
    if (lane < k) c.route_slot[lane] = myslot;
    if (lane == 0) {
      c.miss[0] = nmiss;
      *c.clock = clock;
      c.stats[CS_HITS] += (unsigned long long)hits;
      c.stats[CS_COPIES] += (unsigned long long)nmiss;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < S; i += kLruThreads) {
    c.slot_key[i] = skey[i];
    c.slot_last[i] = slast[i];
  }
}

// Destination in the pool of byte `o` of a record copied into slot v: the record's four pieces go to the slot's rows
// of the gate_up payload and scale planes and of the down payload and scale planes.
__device__ __forceinline__ uint4* fill_dst(const CacheDev& c, size_t v, size_t o) {
  if (o < c.gu_q) return reinterpret_cast<uint4*>(const_cast<uint8_t*>(c.pool_gu.q) + v * c.gu_q + o);
  o -= c.gu_q;
  if (o < c.gu_d)
    return reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(const_cast<uint16_t*>(c.pool_gu.d)) + v * c.gu_d + o);
  o -= c.gu_d;
  if (o < c.dn_q) return reinterpret_cast<uint4*>(const_cast<uint8_t*>(c.pool_dn.q) + v * c.dn_q + o);
  o -= c.dn_q;
  const size_t dn_d = c.record_bytes - c.gu_q - c.gu_d - c.dn_q;
  return reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(const_cast<uint16_t*>(c.pool_dn.d)) + v * dn_d + o);
}

// Miss j = blockIdx.x, bytes [64 KiB * blockIdx.y, +64 KiB) of its record: host store -> the slot's four pieces.
// All loads of the chunk are issued before the first store.
__global__ __launch_bounds__(kFillThreads) void k_fill(CacheDev c) {
  constexpr int PER = kFillChunk / 16 / kFillThreads;
  const int j = blockIdx.x;
  if (j >= c.miss[0]) return;
  const size_t v = (size_t)c.miss[1 + 2 * j], key = (size_t)c.miss[2 + 2 * j];
  const size_t lo = (size_t)blockIdx.y * kFillChunk + 16 * (size_t)threadIdx.x;
  const uint4* src = reinterpret_cast<const uint4*>(c.host + key * c.record_bytes);
  uint4 buf[PER];
#pragma unroll
  for (int q = 0; q < PER; q++) {
    const size_t o = lo + (size_t)q * 16 * kFillThreads;
    buf[q] = o < c.record_bytes ? src[o / 16] : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int q = 0; q < PER; q++) {
    const size_t o = lo + (size_t)q * 16 * kFillThreads;
    if (o < c.record_bytes) *fill_dst(c, v, o) = buf[q];
  }
}

// Plain copy of `bytes` (multiple of 16) from pinned host memory into device memory by a kernel: the transfer the
// fill kernel makes, without the pool addressing (PCIe rate reference).
__global__ __launch_bounds__(kFillThreads) void k_h2d_copy(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                           size_t n) {
  constexpr int PER = kFillChunk / 16 / kFillThreads;
  const size_t base = (size_t)blockIdx.x * (kFillChunk / 16) + threadIdx.x;
  uint4 buf[PER];
#pragma unroll
  for (int q = 0; q < PER; q++) {
    const size_t i = base + (size_t)q * kFillThreads;
    buf[q] = i < n ? src[i] : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int q = 0; q < PER; q++) {
    const size_t i = base + (size_t)q * kFillThreads;
    if (i < n) dst[i] = buf[q];
  }
}

hipError_t launch_h2d_copy(hipStream_t s, const void* src, void* dst, size_t bytes) {
  const size_t n = bytes / 16;
  const int blocks = (int)((bytes + kFillChunk - 1) / kFillChunk);
  klaunch(k_h2d_copy, blocks, kFillThreads, 0, s, (const uint4*)src, (uint4*)dst, n);
  return hipGetLastError();
}

hipError_t launch_route_lru(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                            const CacheDev& c) {
  if (c.slots < d.top_k || c.slots > kCacheMaxSlots || L.router.rows > 64 || d.top_k > 8) return hipErrorInvalidValue;
#define BODY(KK)                                                                                          \
  case KK:                                                                                                \
    klaunch(k_route_lru<DTC, KK>, 1, kLruThreads, 0, s, L.router, L.router_bias, b.h, L.ln_moe, d.eps,    \
            d.top_k, layer, b.route_ids + layer * d.top_k, b.route_w + layer * d.top_k, c);               \
    break;
  MOERT_DISPATCH(L.router.dtype, L.router.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_fill(hipStream_t s, const CacheDev& c, int k) {
  if (c.record_bytes % 16 || c.gu_q % 16 || c.gu_d % 16 || c.dn_q % 16) return hipErrorInvalidValue;
  const int chunks = (int)((c.record_bytes + kFillChunk - 1) / kFillChunk);
  klaunch(k_fill, dim3(k, chunks), kFillThreads, 0, s, c);
  return hipGetLastError();
}

}  // namespace moert

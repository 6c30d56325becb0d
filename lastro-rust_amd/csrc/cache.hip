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

// ------------------------------------------------------------------------------------------------------------
// Prefetch branch. The prediction is a heuristic (its arithmetic does not enter any output): the router of layer l
// applied to the layer's input instead of to its post-attention state. Its choices are recorded per position and
// layer so that the cache counters can be replayed exactly.
#include "cache_dev.h"
#include "dev_rows.h"

namespace moert {

constexpr int kPfNW = 16;  // waves of the decide kernel

template <int DT, int K>
__global__ __launch_bounds__(kPfNW * 64) void k_prefetch_decide(DMat router, const float* __restrict__ bias,
                                                                const float* __restrict__ h,
                                                                const float* __restrict__ lnw, float eps, int k,
                                                                int layer, CacheDev c) {
  using G = Geo<DT, K>;
  constexpr int NT = kPfNW * 64;
  constexpr int RP = (64 + kPfNW * G::RPW - 1) / (kPfNW * G::RPW);
  __shared__ float xs[K];
  __shared__ float rs;
  __shared__ __align__(16) float lg[64];
  __shared__ int part[kPfNW][64];
  __shared__ int skey[kCacheMaxSlots];
  __shared__ int slast[kCacheMaxSlots];
  __shared__ int lfound[8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPR, rw = lane / G::LPR;
  const int E = router.rows, S = c.slots, cur = *c.cur;
  NormIn<K, NT> hin;
  norm_fetch<K, NT>(h, lnw, hin);
  size_t row[RP];
  bool ok[RP];
#pragma unroll
  for (int p = 0; p < RP; p++) {
    row[p] = (size_t)(p * kPfNW + wave) * G::RPW + rw;
    ok[p] = row[p] < (size_t)E;
  }
  Rows<DT, K, RP> rr;
  rows_load<DT, K, RP>(rr, router, row, ok, sub);
  float bv[RP];
#pragma unroll
  for (int p = 0; p < RP; p++) bv[p] = bias ? bias[ok[p] ? row[p] : 0] : 0.0f;
  for (int i = threadIdx.x; i < S; i += NT) {
    skey[i] = c.slot_key[cur * S + i];
    slast[i] = c.slot_last[cur * S + i];
  }
  norm_finish<K, NT>(hin, eps, xs, &rs);
  XReg<DT, K> xr;
  load_x<DT, K>(xr, xs, sub);
  float out[RP];
  rows_fma<DT, K, RP>(rr, ok, xr, sub, out);
#pragma unroll
  for (int p = 0; p < RP; p++)
    if (ok[p] && sub == 0) lg[row[p]] = bias ? out[p] + bv[p] : out[p];
  __syncthreads();
  int eid[8];
  const int rank = wg_rank<kPfNW>(lg, E, lane, wave, part);
  ids_by_rank(lane < E && rank < k, rank, k, eid);
  if (wave == 0) {
    int key = 0;
#pragma unroll
    for (int r = 0; r < 8; r++) key = lane == r ? layer * c.experts + eid[r] : key;
    const int clock = c.clock[cur] + 1;  // one tick, in place: the layer's own step takes the next one
    int slot, miss_key, hits, misses;
    lru_decide(skey, slast, lfound, S, clock, k, lane, key, slot, miss_key, hits, misses);
    // the misses in top-k order: their rank among the lanes below that missed
    const unsigned long long mb = __ballot(lane < k && miss_key >= 0);
    const int mi = __popcll(mb & ((1ull << lane) - 1ull));
    if (lane < k && miss_key >= 0) {
      c.pf[1 + 2 * mi] = slot;
      c.pf[2 + 2 * mi] = miss_key;
    }
    if (lane == 0) {
      c.pf[0] = misses;
      c.clock[cur] = clock;
      c.stats[CS_PREFETCH] += (unsigned long long)misses;
      c.tok_hist[((size_t)c.state[ST_POS] * c.layers + layer) * 4 + 2] = misses;
    }
    if (lane < 8) c.pred_hist[((size_t)c.state[ST_POS] * c.layers + layer) * 8 + lane] = lane < k ? eid[lane] : -1;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < S; i += NT) {
    c.slot_key[cur * S + i] = skey[i];
    c.slot_last[cur * S + i] = slast[i];
  }
}

// Copies the listed records: workgroup (b, j) moves part b of record j (its four pieces, each cut into gridDim.x
// parts of 16-byte words); the loads of a pass are issued before its stores. A workgroup past the list's count
// ends at once.
constexpr int kPfCopyParts = 32;

__global__ __launch_bounds__(256) void k_prefetch_copy(CacheDev c) {
  const int j = blockIdx.y;
  if (j >= c.pf[0]) return;
  const int slot = c.pf[1 + 2 * j], key = c.pf[2 + 2 * j];
  const uint8_t* rec = c.host + (size_t)key * c.record_bytes;
  const size_t dn_d = c.record_bytes - c.gu_q - c.gu_d - c.dn_q;
  const size_t off[4] = {0, c.gu_q, c.gu_q + c.gu_d, c.gu_q + c.gu_d + c.dn_q};
  const size_t len[4] = {c.gu_q, c.gu_d, c.dn_q, dn_d};
  uint8_t* dst[4] = {const_cast<uint8_t*>(c.pool_gu.q) + (size_t)slot * c.gu_q,
                     (uint8_t*)const_cast<uint16_t*>(c.pool_gu.d) + (size_t)slot * c.gu_d,
                     const_cast<uint8_t*>(c.pool_dn.q) + (size_t)slot * c.dn_q,
                     (uint8_t*)const_cast<uint16_t*>(c.pool_dn.d) + (size_t)slot * dn_d};
  for (int piece = 0; piece < 4; piece++) {
    const size_t n = len[piece] / 16, per = (n + gridDim.x - 1) / gridDim.x;
    const size_t w0 = (size_t)blockIdx.x * per, w1 = w0 + per < n ? w0 + per : n;
    const uint4* src = reinterpret_cast<const uint4*>(rec + off[piece]);
    uint4* out = reinterpret_cast<uint4*>(dst[piece]);
    for (size_t i = w0 + threadIdx.x; i < w1; i += 4 * 256) {
      uint4 v[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const size_t t = i + (size_t)q * 256;
        v[q] = t < w1 ? src[t] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const size_t t = i + (size_t)q * 256;
        if (t < w1) out[t] = v[q];
      }
    }
  }
}

hipError_t launch_prefetch_decide(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                                  const CacheDev& c) {
  if (c.slots < d.top_k || c.slots > kCacheMaxSlots || L.router.rows > 64 || d.top_k > 8) return hipErrorInvalidValue;
#define BODY(KK)                                                                                          \
  case KK:                                                                                                \
    klaunch(k_prefetch_decide<DTC, KK>, 1, kPfNW * 64, 0, s, L.router, L.router_bias, b.h, L.ln_moe, d.eps, \
            d.top_k, layer, c);                                                                           \
    break;
  MOERT_DISPATCH(L.router.dtype, L.router.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_prefetch_copy(hipStream_t s, const CacheDev& c) {
  klaunch(k_prefetch_copy, dim3(kPfCopyParts, 8), 256, 0, s, c);
  return hipGetLastError();
}

}  // namespace moert

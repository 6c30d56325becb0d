// Prefetch inside the attention launch of a cached decode step (k_attn_block_pf, attn_block.hip). After the
// launch's 8 * splits attention workgroups come one decide workgroup and kPfCopyWgs copy workgroups:
//   decide  the layer's experts predicted from its input h (its MoE norm and router applied to h before attention:
//           a heuristic whose arithmetic enters no output), top-k, one uncounted tick of the LRU rule over the
//           predicted keys in place on the current slot tables; the predicted misses go out device-wide as
//           epoch-tagged entries (count, then a (slot, key) pair each) in c.pfx;
//   copy    workgroup j takes part j of every listed record (its four pieces, each cut into kPfCopyWgs parts of
//           16-byte words) from the pinned host store into the pool slot.
// The attention workgroups wait for neither, so the copies run beside attention and the launch ends when they are
// done; the next launches (output projection, then router + gate/up, which reads the pool) come after it in the
// stream. A copy workgroup that gives up waiting for the list sets bit 16 of the attention block's error word
// (the step then reports a device error: the ticked slots would hold no record).
// This replaces the side-stream branch (k_prefetch_decide + k_prefetch_copy, cache.hip) with the same decision and
// the same records copied, so the cache counters replay the same way.
#pragma once
#include "attn_dev.h"
#include "cache_dev.h"
#include "dev_rows.h"

namespace moert {

constexpr int kPfCopyWgs = 64;
constexpr int kPfSpin = 1 << 18;

struct PfArgs {
  DMat router;
  const float* bias;
  const float* lnw;  // the layer's MoE norm weights
  float eps;
  int k;
  int layer;
  CacheDev c;
};

// The decide workgroup (NT threads). Same decision as k_prefetch_decide: logits = router(rmsnorm(h, lnw)) (+ bias)
// per row in canonical order, top-k by the total-order key (wave_topk: the same ranks as wg_rank), lru_decide with
// clock + 1 in place on the current tables.
template <int DT, int K, int NT>
__device__ __forceinline__ void pf_decide(const PfArgs& a, const float* __restrict__ h, unsigned epoch) {
  using G = Geo<DT, K>;
  constexpr int NW = NT / 64;
  constexpr int RP = (64 + NW * G::RPW - 1) / (NW * G::RPW), RB = RP < 4 ? RP : 4;
  __shared__ float xs[K];
  __shared__ float rs;
  __shared__ __align__(16) float lg[64];
  __shared__ int skey[kCacheMaxSlots];
  __shared__ int slast[kCacheMaxSlots];
  __shared__ int lfound[8];
  __shared__ __align__(16) TopkLds tk;
  __shared__ int ids_s[8];
  __shared__ float w_s[8];
  const CacheDev& c = a.c;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPR, rw = lane / G::LPR;
  const int E = a.router.rows, S = c.slots, cur = *c.cur;
  NormIn<K, NT> hin;
  norm_fetch<K, NT>(h, a.lnw, hin);
  for (int i = threadIdx.x; i < S; i += NT) {
    skey[i] = c.slot_key[cur * S + i];
    slast[i] = c.slot_last[cur * S + i];
  }
  norm_finish<K, NT>(hin, a.eps, xs, &rs);
  XReg<DT, K> xr;
  load_x<DT, K>(xr, xs, sub);
  // the router rows in batches of RB per wave (row (p * NW + wave) * RPW + rw for p < RP)
#pragma unroll 1
  for (int p0 = 0; p0 < RP; p0 += RB) {
    size_t row[RB];
    bool ok[RB];
#pragma unroll
    for (int p = 0; p < RB; p++) {
      row[p] = (size_t)((p0 + p) * NW + wave) * G::RPW + rw;
      ok[p] = p0 + p < RP && row[p] < (size_t)E;
      row[p] = ok[p] ? row[p] : 0;
    }
    Rows<DT, K, RB> rr;
    rows_load<DT, K, RB>(rr, a.router, row, ok, sub);
    float out[RB];
    rows_fma<DT, K, RB>(rr, ok, xr, sub, out);
#pragma unroll
    for (int p = 0; p < RB; p++)
      if (ok[p] && sub == 0) lg[row[p]] = a.bias ? out[p] + a.bias[row[p]] : out[p];
  }
  __syncthreads();
  if (wave == 0) {
    const int k = a.k;
    wave_topk(lg, E, k, lane, tk, ids_s, w_s);
    wave_lds_sync();
    int key = 0;
    if (lane < k) key = a.layer * c.experts + ids_s[lane];
    const int clock = c.clock[cur] + 1;  // one tick, in place: the layer's own step takes the next one
    int slot, miss_key, hits, misses;
    lru_decide(skey, slast, lfound, S, clock, k, lane, key, slot, miss_key, hits, misses);
    // the misses in top-k order: their rank among the lanes below that missed
    const unsigned long long mb = __ballot(lane < k && miss_key >= 0);
    const int mi = __popcll(mb & ((1ull << lane) - 1ull));
    if (lane < k && miss_key >= 0) {
      put_dev(&c.pfx[1 + 2 * mi], (unsigned)slot, epoch);
      put_dev(&c.pfx[2 + 2 * mi], (unsigned)miss_key, epoch);
    }
    if (lane == 0) {
      put_dev(&c.pfx[0], (unsigned)misses, epoch);
      c.clock[cur] = clock;
      c.stats[CS_PREFETCH] += (unsigned long long)misses;
      c.tok_hist[((size_t)c.state[ST_POS] * c.layers + a.layer) * 4 + 2] = misses;
    }
    if (lane < 8) c.pred_hist[((size_t)c.state[ST_POS] * c.layers + a.layer) * 8 + lane] = lane < k ? ids_s[lane] : -1;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < S; i += NT) {
    c.slot_key[cur * S + i] = skey[i];
    c.slot_last[cur * S + i] = slast[i];
  }
}

// Copy workgroup `part` (NT threads): waits (at most `spin` polls) for the list entries carrying `epoch`, then copies
// part `part` of each listed record. Returns false when the wait gave up.
template <int NT>
__device__ __forceinline__ bool pf_copy(const CacheDev& c, unsigned epoch, int part, int spin) {
  __shared__ int list_s[1 + 2 * 8];
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    // the count first, then the pairs it announces
    bool ok = false;
    unsigned n = 0;
    for (int it = 0; it < spin; it++) {
      poll_fence();
      const uint2 e = get_dev(&c.pfx[0]);
      if (e.y == epoch) {
        n = e.x < 8u ? e.x : 8u;  // at most top_k <= 8 misses
        ok = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    unsigned v = 0;
    if (ok && n > 0) {
      const bool use = lane >= 1 && lane < 1 + 2 * (int)n;
      ok = false;
      for (int it = 0; it < spin; it++) {
        poll_fence();
        const uint2 e = get_dev(&c.pfx[use ? lane : 0]);
        v = e.x;
        if (__ballot(use && e.y != epoch) == 0) {
          ok = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    if (lane == 0) list_s[0] = ok ? (int)n : -1;
    if (lane >= 1 && lane < 1 + 2 * 8) list_s[lane] = (int)v;
  }
  __syncthreads();
  const int n = list_s[0];
  if (n < 0) return false;
  const size_t dn_d = c.record_bytes - c.gu_q - c.gu_d - c.dn_q;
  const size_t off[4] = {0, c.gu_q, c.gu_q + c.gu_d, c.gu_q + c.gu_d + c.dn_q};
  const size_t len[4] = {c.gu_q, c.gu_d, c.dn_q, dn_d};
  for (int j = 0; j < n; j++) {
    const int slot = list_s[1 + 2 * j], key = list_s[2 + 2 * j];
    const uint8_t* rec = c.host + (size_t)key * c.record_bytes;
    uint8_t* dst[4] = {const_cast<uint8_t*>(c.pool_gu.q) + (size_t)slot * c.gu_q,
                       (uint8_t*)const_cast<uint16_t*>(c.pool_gu.d) + (size_t)slot * c.gu_d,
                       const_cast<uint8_t*>(c.pool_dn.q) + (size_t)slot * c.dn_q,
                       (uint8_t*)const_cast<uint16_t*>(c.pool_dn.d) + (size_t)slot * dn_d};
    for (int piece = 0; piece < 4; piece++) {
      const size_t nw = len[piece] / 16, per = (nw + kPfCopyWgs - 1) / kPfCopyWgs;
      const size_t w0 = (size_t)part * per < nw ? (size_t)part * per : nw, w1 = w0 + per < nw ? w0 + per : nw;
      const uint4* src = reinterpret_cast<const uint4*>(rec + off[piece]);
      uint4* out = reinterpret_cast<uint4*>(dst[piece]);
      for (size_t i = w0 + threadIdx.x; i < w1; i += 4 * NT) {
        uint4 v[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const size_t t = i + (size_t)q * NT;
          v[q] = t < w1 ? src[t] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const size_t t = i + (size_t)q * NT;
          if (t < w1) out[t] = v[q];
        }
      }
    }
  }
  return true;
}

}  // namespace moert

// Device side of the expert cache: the LRU decision of one layer step over slot tables held in LDS, and the row
// source of a routed expert (its pool slot, or its record in the host store when it missed).
#pragma once
#include "cache.h"
#include "dev_math.h"

namespace moert {

template <int S>
__device__ __forceinline__ unsigned long long min_stage_u64(unsigned long long v) {
  const unsigned lo = partner_u32<S>((uint32_t)(v & 0xffffffffu)), hi = partner_u32<S>((uint32_t)(v >> 32));
  const unsigned long long o = ((unsigned long long)hi << 32) | lo;
  return o < v ? o : v;
}

// Minimum over the 64 lanes, in every lane (DPP / permlane butterfly).
__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v) {
  v = min_stage_u64<1>(v);
  v = min_stage_u64<2>(v);
  v = min_stage_u64<4>(v);
  v = min_stage_u64<8>(v);
  v = min_stage_u64<16>(v);
  return min_stage_u64<32>(v);
}

// LRU decision for the k <= 8 keys of one layer step, by one wave, over the slot tables skey[S] / slast[S] in LDS
// (the LruSync rule; reference_lru, tests/model.rs:380-412): every requested key already in a slot is touched first,
// so that no miss of this step can evict it; then each miss, in top-k order, takes the first free slot, or else the
// least recently used slot not used in this step (lowest index on ties). Lane j < k holds key j on entry and
// receives its slot and, when it missed, its key in `miss_key` (-1 when it hit). The tables are updated in LDS;
// found_lds is 8 ints of LDS scratch. S >= k guarantees a victim for every miss.
__device__ __forceinline__ void lru_decide(int* skey, int* slast, int* found_lds, int S, int clock, int k, int lane,
                                           int key, int& slot, int& miss_key, int& hits, int& misses) {
  // the slot holding each requested key (keys are unique in the tables): one pass over the slots, the lane that
  // finds key j records it
  if (lane < 8) found_lds[lane] = -1;
  wave_lds_sync();
  int keys[8];
#pragma unroll
  for (int j = 0; j < 8; j++) keys[j] = __builtin_amdgcn_readlane(key, j);
  for (int i = lane; i < S; i += 64) {
    const int kk = skey[i];
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (j < k && kk == keys[j]) found_lds[j] = i;
  }
  wave_lds_sync();
  const int found = lane < k ? found_lds[lane] : -1;
  if (lane < k && found >= 0) slast[found] = clock;
  wave_lds_sync();
  int mine = found, nm = 0, nh = 0;
  for (int j = 0; j < k; j++) {
    const int sj = __builtin_amdgcn_readlane(found, j), keyj = __builtin_amdgcn_readlane(key, j);
    if (sj >= 0) {
      nh++;
      continue;
    }
    unsigned long long best = ~0ull;
    for (int i = lane; i < S; i += 64) {
      const bool freev = skey[i] < 0;
      if (freev || slast[i] < clock) {
        const unsigned long long cand = ((unsigned long long)(freev ? 0u : (unsigned)slast[i] + 1u) << 32) | (unsigned)i;
        best = cand < best ? cand : best;
      }
    }
    best = wave_min_u64(best);
    const int v = best == ~0ull ? 0 : (int)(best & 0xffffffffu);  // (no candidate cannot happen when S >= k)
    if (lane == 0) {
      skey[v] = keyj;
      slast[v] = clock;
    }
    wave_lds_sync();
    if (lane == j) mine = v;
    nm++;
  }
  slot = mine;
  miss_key = found < 0 ? key : -1;
  hits = nh;
  misses = nm;
}

// The matrix holding the rows of a routed expert: its record in the host store when it missed (rows from 0),
// else the pool (rows from slot * rows_per_expert). `piece` selects gate/up (0) or down (1).
__device__ __forceinline__ DMat expert_source(const CacheDev& c, int piece, int slot, int miss_key, size_t& row0) {
  const DMat& pool = piece == 0 ? c.pool_gu : c.pool_dn;
  const size_t rows = piece == 0 ? (size_t)c.pool_gu.rows / c.slots : (size_t)c.pool_dn.rows / c.slots;
  if (miss_key < 0) {
    row0 = (size_t)slot * rows;
    return pool;
  }
  row0 = 0;
  const uint8_t* rec = c.host + (size_t)miss_key * c.record_bytes + (piece == 0 ? 0 : c.gu_q + c.gu_d);
  const size_t q_bytes = piece == 0 ? c.gu_q : c.dn_q;
  return DMat{rec, reinterpret_cast<const uint16_t*>(rec + q_bytes), pool.dtype, (int)rows, pool.cols};
}

}  // namespace moert

// Device pieces shared by the attention kernels: the tile staging of the split-KV kernels (kernels.hip,
// attn_block.hip) and the XCD-local exchange of the attention block kernel (attn_block.hip).
#pragma once
#include "dev_math.h"

namespace moert {

// One wave's share of a V tile moved into LDS through registers, by the G waves that serve the same tile: piece e
// (e = wave, wave + G, ...) is rows 8e..8e+7, lane l carrying 16 bytes of row 8e + l/8, so each piece reads 1 KB of
// consecutive cache rows. The LDS tile is row-major [64][64] f32, converted once for the G heads, with the rows at
// and past the tile's valid length `nv` stored as +0. Plain loads (not LDS DMA) keep the wait for the tile separate
// from the waits for the kernel's other loads. A piece index past 7 (only for G = 3) loads piece 7 again and stores
// it into rows 64..71 of the tile, which are padding and never read.
template <int G>
struct VShare {
  static constexpr int N = (8 + G - 1) / G;
  uint4 a, b, c, d, e, f, g, h;  // pieces 0..N-1 of this wave (named members: no private array)
  __device__ __forceinline__ void load(const uint16_t* V, int t, int lane, int wave) {
    const uint4* src = reinterpret_cast<const uint4*>(V + ((size_t)t * 64 + (lane >> 3)) * 64 + (lane & 7) * 8);
    auto at = [&](int i) { return gload_u4(src + (size_t)min(wave + G * i, 7) * 64); };
    a = at(0);
    if (N > 1) b = at(1);
    if (N > 2) c = at(2);
    if (N > 3) d = at(3);
    if (N > 4) e = at(4);
    if (N > 5) f = at(5);
    if (N > 6) g = at(6);
    if (N > 7) h = at(7);
  }
  template <int STRIDE>
  __device__ __forceinline__ void store(float* dst, int lane, int wave, int nv) const {
    auto put = [&](int i, const uint4& v) {
      const int row = 8 * (wave + G * i) + (lane >> 3);
      const bool z = row >= nv;
      float4* o = reinterpret_cast<float4*>(dst + row * STRIDE + (lane & 7) * 8);
      o[0] = z ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
               : make_float4(h2f((uint16_t)(v.x & 0xffffu)), h2f((uint16_t)(v.x >> 16)), h2f((uint16_t)(v.y & 0xffffu)),
                             h2f((uint16_t)(v.y >> 16)));
      o[1] = z ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
               : make_float4(h2f((uint16_t)(v.z & 0xffffu)), h2f((uint16_t)(v.z >> 16)), h2f((uint16_t)(v.w & 0xffffu)),
                             h2f((uint16_t)(v.w >> 16)));
    };
    put(0, a);
    if (N > 1) put(1, b);
    if (N > 2) put(2, c);
    if (N > 3) put(3, d);
    if (N > 4) put(4, e);
    if (N > 5) put(5, f);
    if (N > 6) put(6, g);
    if (N > 7) put(7, h);
  }
  // The tile kept in fp16, row-major with rows of RS halves, as loaded (rows at and past nv stored as +0).
  template <int RS>
  __device__ __forceinline__ void store_h(uint16_t* dst, int lane, int wave, int nv) const {
    auto put = [&](int i, const uint4& v) {
      const int row = 8 * (wave + G * i) + (lane >> 3);
      *reinterpret_cast<uint4*>(dst + row * RS + (lane & 7) * 8) = row >= nv ? make_uint4(0u, 0u, 0u, 0u) : v;
    };
    put(0, a);
    if (N > 1) put(1, b);
    if (N > 2) put(2, c);
    if (N > 3) put(3, d);
    if (N > 4) put(4, e);
    if (N > 5) put(5, f);
    if (N > 6) put(6, g);
    if (N > 7) put(7, h);
  }
  // The tile kept in fp16 and transposed: element (row, dim) at dst[dim * 64 + vt_col(row, dim)] (rows 0..63; the
  // padding piece past row 63 is not stored), rows at and past nv stored as +0.
  __device__ __forceinline__ void store_ht(uint16_t* dst, int lane, int wave, int nv) const {
    auto put = [&](int i, const uint4& v) {
      const int row = 8 * (wave + G * i) + (lane >> 3);
      if (row >= 64) return;
      const bool z = row >= nv;
      const int c0 = (lane & 7) * 8;
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int dm = c0 + k;
        dst[dm * 64 + vt_col(row, dm)] = z ? (uint16_t)0 : (uint16_t)(w[k >> 1] >> (16 * (k & 1)));
      }
    };
    put(0, a);
    if (N > 1) put(1, b);
    if (N > 2) put(2, c);
    if (N > 3) put(3, d);
    if (N > 4) put(4, e);
    if (N > 5) put(5, f);
    if (N > 6) put(6, g);
    if (N > 7) put(7, h);
  }
  // Column of position `row` in dim row `dm` of the transposed tile: 8-position chunks permuted by
  // (dm ^ dm / 8) % 8, so that the 16-byte reads of one chunk by 8 consecutive dims, and the writes of one element
  // of a piece by its 64 lanes, fall in different LDS banks.
  __device__ static __forceinline__ int vt_col(int row, int dm) {
    return 8 * ((row >> 3) ^ ((dm ^ (dm >> 3)) & 7)) + (row & 7);
  }
};

// ------------------------------------------------------------------------------------------------------------
// XCD-local exchange. The chip dispatches the workgroups of a launch to its 8 XCDs in round-robin order, and each
// XCD has its own L2. Workgroups on one XCD exchange data through that L2: a store from a compute unit goes through
// its write-through L1 to the L2 (complete there once the wave's vmcnt has drained), and a load with the sc1 cache
// policy (agent scope) misses the compute unit's L1 and is served by the L2, which holds the other compute units'
// stores. A load with sc0 (workgroup scope) may still hit a stale L1 line and is not used for this.

// The XCD the calling wave runs on (hardware register XCC_ID, bits 3:0).
__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xfu;
}

// Waits until every memory operation this wave issued so far has completed (stores included: on gfx9 they are
// counted by vmcnt).
__device__ __forceinline__ void wait_mem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// A compiler-only fence for polling loops: the compiler takes a buffer load inside a loop that stores nothing as a
// read of unchanging memory and hoists it out of the loop; placed in the loop, this keeps a fresh load per pass.
__device__ __forceinline__ void poll_fence() { asm volatile("" ::: "memory"); }

// A raw buffer over `bytes` bytes at p; loads through it take an explicit cache policy, and a load past the end
// returns 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t l2_buffer(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// Loads from the XCD's L2, never from the compute unit's L1 (cache policy sc1, bit 4 of the auxiliary operand);
// byte offsets.
constexpr int kL2Policy = 16;
__device__ __forceinline__ unsigned l2_load_u32(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kL2Policy);
}
__device__ __forceinline__ float l2_load_f32(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kL2Policy));
}
__device__ __forceinline__ unsigned short l2_load_u16(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, kL2Policy);
}
__device__ __forceinline__ uint2 l2_load_u64(__amdgpu_buffer_rsrc_t r, unsigned off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kL2Policy);
  return make_uint2(v[0], v[1]);
}

// An exchange entry: a value's 32 bits and the epoch of the launch that wrote it, stored as one 8-byte word (a
// relaxed atomic store, so it is one store instruction and a reader never sees half of it).
__device__ __forceinline__ void put_entry(uint2* p, unsigned val, unsigned epoch) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), ((unsigned long long)epoch << 32) | val,
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Device-wide entries: agent-scope atomic stores and loads, coherent across the XCDs' L2s.
__device__ __forceinline__ void put_dev(uint2* p, unsigned val, unsigned epoch) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), ((unsigned long long)epoch << 32) | val,
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint2 get_dev(const uint2* p) {
  const unsigned long long v = __hip_atomic_load(reinterpret_cast<unsigned long long*>(const_cast<uint2*>(p)),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint2((unsigned)v, (unsigned)(v >> 32));
}

// Wave-level poll of up to M entries per lane (entry m of this lane at index idx[m], used when use[m]) until every
// used entry of the wave carries `epoch`; LD(i) loads entry i. Returns false when the poll gave up.
template <int M, class LD>
__device__ __forceinline__ bool poll_m(const LD& ld, const int (&idx)[M], const bool (&use)[M], unsigned epoch,
                                       int spin, unsigned (&val)[M]) {
  for (int it = 0; it < spin; it++) {
    poll_fence();
    bool stale = false;
#pragma unroll
    for (int m = 0; m < M; m++) {
      const uint2 e = ld(use[m] ? idx[m] : idx[0]);
      val[m] = e.x;
      stale |= use[m] && e.y != epoch;
    }
    if (__ballot(stale) == 0) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

}  // namespace moert

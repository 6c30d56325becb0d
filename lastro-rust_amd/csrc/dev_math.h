// Device arithmetic shared by every kernel of the decode engine (gfx950, wave64).
//
// Evaluation order is fixed so that results are reproducible bit for bit:
//   - dot products: a row is cut into chunks of 16 bytes of payload (Q8_0: 16 elements, Q4_0: 32, f32: 4);
//     chunk j is accumulated by lane j % 64 (chunks in increasing j, elements in increasing index,
//     acc = fma(w, x, acc) from +0); the 64 lane sums are combined by an xor butterfly, which leaves every lane
//     holding the balanced pairwise tree of the 64 sums;
//   - exp is dexp below (Cody-Waite reduction, degree-7 Taylor polynomial), never the hardware exp2;
//   - division and sqrt are IEEE correctly rounded (hipcc's default), nothing else is fused (-ffp-contract=off).
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moert {

constexpr int kWave = 64;

// exp(x): x = n*ln2 + r with ln2 split into a 15-bit head and a tail (Cody & Waite), e^r by the degree-7 Taylor
// polynomial in Horner form (|r| <= ln2/2, truncation < 1e-8 relative), result 2p * 2^(n-1) with both factors
// exact. x < -86.5 gives 0 (no subnormal results), x > 89 gives +inf.
__device__ __forceinline__ float dexp(float x) {
  if (x != x) return x;
  if (x > 89.0f) return __int_as_float(0x7f800000);
  if (x < -86.5f) return 0.0f;
  float n = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.42860682030941723212e-6f, r);
  float p = 1.98412698412698413e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  return (p * 2.0f) * __int_as_float((ni - 1 + 127) << 23);
}

// dexp without branches, the same value for every x: the polynomial path runs on x clamped into [-87, 89] (which
// leaves every x it serves unchanged) and the special cases are selected afterwards.
__device__ __forceinline__ float dexp_sel(float x) {
  const float xc = __builtin_fminf(__builtin_fmaxf(x, -87.0f), 89.0f);
  float n = __builtin_rintf(xc * 1.44269504088896341f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, xc);
  r = __builtin_fmaf(-n, 1.42860682030941723212e-6f, r);
  float p = 1.98412698412698413e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  float e = (p * 2.0f) * __int_as_float((ni - 1 + 127) << 23);
  e = x < -86.5f ? 0.0f : e;
  e = x > 89.0f ? __int_as_float(0x7f800000) : e;
  return x != x ? x : e;
}

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + dexp(-g))) * u; }

// Cross-lane partner of stage S of a butterfly: a lane in the other half of its aligned 2S-lane group. DPP for
// S <= 8 (quad_perm, row_half_mirror, row_mirror), permlane16/32_swap for S = 16, 32. After stage S every lane of
// an aligned 2S-group holds the same value, so v + partner(v) equals the xor butterfly bit for bit: every lane
// ends with the balanced pairwise tree of the group.
template <int S>
__device__ __forceinline__ uint32_t partner_u32(uint32_t v) {
  if (S == 1) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, true);  // quad_perm 1,0,3,2
  if (S == 2) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, true);  // quad_perm 2,3,0,1
  if (S == 4) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, true);  // row_half_mirror
  if (S == 8) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, true);  // row_mirror
  if (S == 16) {
    auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? r[0] : r[1];
  }
  auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32) ? r[0] : r[1];
}

template <int S>
__device__ __forceinline__ float partner(float v) {
  return __uint_as_float(partner_u32<S>(__float_as_uint(v)));
}
template <int S>
__device__ __forceinline__ int partner(int v) {
  return (int)partner_u32<S>((uint32_t)v);
}

// Butterfly sum over the lanes [0, W) of each aligned W-lane group (all 64 lanes must be active).
template <int W = kWave>
__device__ __forceinline__ float group_sum(float v) {
  if (W > 1) v = v + partner<1>(v);
  if (W > 2) v = v + partner<2>(v);
  if (W > 4) v = v + partner<4>(v);
  if (W > 8) v = v + partner<8>(v);
  if (W > 16) v = v + partner<16>(v);
  if (W > 32) v = v + partner<32>(v);
  return v;
}

template <int S>
__device__ __forceinline__ float max_stage(float v) {
  float o = partner<S>(v);
  return o > v ? o : v;
}

template <int W = kWave>
__device__ __forceinline__ float group_max(float v) {
  if (W > 1) v = max_stage<1>(v);
  if (W > 2) v = max_stage<2>(v);
  if (W > 4) v = max_stage<4>(v);
  if (W > 8) v = max_stage<8>(v);
  if (W > 16) v = max_stage<16>(v);
  if (W > 32) v = max_stage<32>(v);
  return v;
}

// LDS writes of this wave become visible to its other lanes (no workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Total order on floats as integers (Rust's f32::total_cmp).
__device__ __forceinline__ int total_key(float f) {
  int s = __float_as_int(f);
  return s >= 0 ? s : (s ^ 0x7fffffff);
}

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// Quantised matrix in HBM, struct-of-arrays: the payload plane (int8 values for Q8_0, GGML nibble pairs for
// Q4_0, f32 for F32) row-major, then one fp16 scale per 32-element block.
struct DMat {
  const uint8_t* q;
  const uint16_t* d;
  int dtype;
  int rows, cols;
};

enum { DT_F32 = 0, DT_Q8_0 = 1, DT_Q4_0 = 2 };

template <int DT> struct Fmt;
template <> struct Fmt<DT_Q8_0> {
  static constexpr int kElems = 16;  // elements per 16-byte chunk
  __device__ static size_t row_bytes(int cols) { return (size_t)cols; }
};
template <> struct Fmt<DT_Q4_0> {
  static constexpr int kElems = 32;
  __device__ static size_t row_bytes(int cols) { return (size_t)cols / 2; }
};
template <> struct Fmt<DT_F32> {
  static constexpr int kElems = 4;
  __device__ static size_t row_bytes(int cols) { return (size_t)cols * 4; }
};

// A pointer into device memory as a global-address-space pointer. A load through a plain pointer whose origin the
// compiler cannot trace to a kernel argument (one read from a table in memory) becomes a flat load, which also
// counts in the LDS counter (so every LDS wait would wait for it) and needs a 64-bit address per lane; through this
// cast it is a global load.
#define MOERT_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ const MOERT_GLOBAL T* gmem(const T* p) {
  return (const MOERT_GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ MOERT_GLOBAL T* gmem_w(T* p) {
  return (MOERT_GLOBAL T*)p;
}
// 16- and 8-byte vector loads through a global pointer (the HIP vector classes cannot be copied from a qualified
// lvalue, so the native vector is loaded and converted).
typedef unsigned moert_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned moert_u32x2 __attribute__((ext_vector_type(2)));
typedef float moert_f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 gload_u4(const void* p) {
  const moert_u32x4 v = *(const MOERT_GLOBAL moert_u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 gload_u2(const void* p) {
  const moert_u32x2 v = *(const MOERT_GLOBAL moert_u32x2*)p;
  return make_uint2(v.x, v.y);
}
// The same 16-byte load with the non-temporal hint: the line goes into the L2 as the first to be evicted, so that a
// stream read once does not push out lines that a later launch will read.
__device__ __forceinline__ uint4 gload_u4_nt(const void* p) {
  const moert_u32x4 v = __builtin_nontemporal_load((const MOERT_GLOBAL moert_u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 gload_f4(const void* p) {
  const moert_f32x4 v = *(const MOERT_GLOBAL moert_f32x4*)p;
  return make_float4(v.x, v.y, v.z, v.w);
}

// One 16-byte chunk j of a row, loaded raw, with the raw bits of its fp16 scale (converted where it is used, so
// that a run of chunk loads is not broken by a wait for each scale).
struct RawChunk {
  uint4 v;
  uint32_t d;
};

// NT: with the non-temporal hint (rows streamed once per step).
template <int DT, bool NT = false>
__device__ __forceinline__ RawChunk load_chunk(const DMat& m, size_t row, int j) {
  RawChunk c;
  const uint8_t* base = m.q + row * Fmt<DT>::row_bytes(m.cols);
  c.v = NT ? gload_u4_nt(base + (size_t)j * 16) : gload_u4(base + (size_t)j * 16);
  if (DT == DT_Q8_0 || DT == DT_Q4_0) {
    const uint16_t* sp = m.d + row * (size_t)(m.cols / 32) + (DT == DT_Q8_0 ? (j >> 1) : j);
    c.d = NT ? __builtin_nontemporal_load(gmem(sp)) : *gmem(sp);
  } else
    c.d = 0x3c00u;  // 1.0
  return c;
}

// The empty asm keeps the conversion at its use: hoisted up to its load (the compiler pushes the conversion through
// the phi of a conditional load), it would make the wave wait there for every load issued before the scale.
__device__ __forceinline__ float scale_at_use(uint32_t bits) {
  asm("" : "+v"(bits));
  return h2f((uint16_t)bits);
}
__device__ __forceinline__ float chunk_scale(const RawChunk& c) { return scale_at_use(c.d); }

// acc = fma chain over the chunk's elements in index order; x holds the chunk's Fmt<DT>::kElems activations.
template <int DT>
__device__ __forceinline__ float fma_chunk(const RawChunk& c, const float* x, float acc) {
  const uint32_t w[4] = {c.v.x, c.v.y, c.v.z, c.v.w};
  const float d = chunk_scale(c);
  if (DT == DT_Q8_0) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      float q = (float)(int8_t)(w[i >> 2] >> (8 * (i & 3)));
      acc = __builtin_fmaf(q * d, x[i], acc);
    }
  } else if (DT == DT_Q4_0) {
    // GGML Q4_0: byte b holds element b (low nibble) and element b + 16 (high nibble).
#pragma unroll
    for (int i = 0; i < 16; i++) {
      float q = (float)((int)((w[i >> 2] >> (8 * (i & 3))) & 15u) - 8);
      acc = __builtin_fmaf(q * d, x[i], acc);
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
      float q = (float)((int)((w[i >> 2] >> (8 * (i & 3) + 4)) & 15u) - 8);
      acc = __builtin_fmaf(q * d, x[16 + i], acc);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) acc = __builtin_fmaf(__uint_as_float(w[i]), x[i], acc);
  }
  return acc;
}

// Dequantised element i of a chunk (for the dequant kernel).
template <int DT>
__device__ __forceinline__ float chunk_elem(const RawChunk& c, int i) {
  const uint32_t w[4] = {c.v.x, c.v.y, c.v.z, c.v.w};
  if (DT == DT_Q8_0) return (float)(int8_t)(w[i >> 2] >> (8 * (i & 3))) * chunk_scale(c);
  if (DT == DT_Q4_0) {
    int b = i & 15, sh = 8 * (b & 3) + (i >= 16 ? 4 : 0);
    return (float)((int)((w[b >> 2] >> sh) & 15u) - 8) * chunk_scale(c);
  }
  return __uint_as_float(w[i]);
}

}  // namespace moert

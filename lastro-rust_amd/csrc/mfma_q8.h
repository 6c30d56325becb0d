// Device pieces shared by the int8 MFMA kernels of the multi-position step (grouped.hip, grouped_dense.hip): 15-bit
// activation codes, one wave's 16-row MFMA tile over Q8_0 blocks in the tiled layout (TMat), and the staging of
// its operands.
//
// An activation block of 32 elements with scale d = amax / 32639 becomes q = rint(x / d) in [-32639, 32639], split
// into two int8 planes q = 256 hi + lo; a Q8_0 weight block times it is S = 256 (w . hi) + (w . lo), an exact int32
// per block (v_mfma_i32_16x16x32_i8 is one 32-element block per K-step), and acc = fma((float)S, d_w * d_x, acc)
// over the blocks in order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dev_math.h"
#include "grouped.h"

namespace moert {

typedef int v4i __attribute__((ext_vector_type(4)));

// The hi/lo codes of the 32-element block b of row p (8 lanes per block, 4 elements per lane, v[] the lane's
// elements) into xh / xl [.., K] and its scale into xd [.., K/32]. All 64 lanes take part (group_max over 8).
template <int K>
__device__ __forceinline__ void block_codes(const float (&v)[4], bool valid, int p, int b, int part,
                                            int8_t* __restrict__ xh, int8_t* __restrict__ xl, float* __restrict__ xd) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float a = fabsf(v[i]);
    amax = a > amax ? a : amax;
  }
  amax = group_max<8>(amax);
  const float d = amax / 32639.0f;
  uint32_t hw = 0, lw = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int q = d > 0.0f ? (int)__builtin_rintf(v[i] / d) : 0;
    const int h = (q + 128) >> 8;
    hw |= (uint32_t)(uint8_t)(int8_t)h << (8 * i);
    lw |= (uint32_t)(uint8_t)(int8_t)(q - 256 * h) << (8 * i);
  }
  if (valid) {
    reinterpret_cast<uint32_t*>(xh + (size_t)p * K)[8 * b + part] = hw;
    reinterpret_cast<uint32_t*>(xl + (size_t)p * K)[8 * b + part] = lw;
    if (part == 0) xd[(size_t)p * (K / 32) + b] = d;
  }
}

// MFMA tile of one wave: 16 weight rows x NM member columns over NBW 32-element blocks.
//   a[p]  : this lane's weight codes of blocks 2p and 2p+1 (row lane%16, elements 8*(lane/16) .. +8 of each)
//   bh/bl : LDS [NM][stride] hi / lo codes of the members, from the tile's first block
//   sdt   : LDS [NBW][16] fp16 scales of the 16 rows
//   dx    : LDS activation scales, member c's scale of block b at dx[c * dxs + b]
// acc[ct][i] = output (row 4*(lane/16) + i, column 16*ct + lane%16).
template <int NBW, int NM>
__device__ __forceinline__ void mfma_tile(const uint4 (&a)[NBW / 2], const int8_t* bh, const int8_t* bl, int stride,
                                          const uint16_t* sdt, const float* dx, int dxs, float (&acc)[NM / 16][4]) {
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < NM / 16; ct++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[ct][i] = 0.0f;
#pragma unroll
  for (int b = 0; b < NBW; b++) {
    const uint4& ap = a[b / 2];
    const long av = (b & 1) ? (long)(((unsigned long long)ap.w << 32) | ap.z)
                            : (long)(((unsigned long long)ap.y << 32) | ap.x);
    const uint2 s4 = *reinterpret_cast<const uint2*>(sdt + b * 16 + 4 * grp);
    const float dw[4] = {h2f((uint16_t)(s4.x & 0xffff)), h2f((uint16_t)(s4.x >> 16)), h2f((uint16_t)(s4.y & 0xffff)),
                         h2f((uint16_t)(s4.y >> 16))};
#pragma unroll
    for (int ct = 0; ct < NM / 16; ct++) {
      const int c = 16 * ct + col;
      const uint2 h2 = *reinterpret_cast<const uint2*>(bh + (size_t)c * stride + 32 * b + 8 * grp);
      const uint2 l2 = *reinterpret_cast<const uint2*>(bl + (size_t)c * stride + 32 * b + 8 * grp);
      const long hv = (long)(((unsigned long long)h2.y << 32) | h2.x);
      const long lv = (long)(((unsigned long long)l2.y << 32) | l2.x);
      const v4i z = {0, 0, 0, 0};
      const v4i sh = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, hv, z, 0, 0, 0);
      const v4i sl = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, lv, z, 0, 0, 0);
      const float dxc = dx[c * dxs + b];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int S = 256 * sh[i] + sl[i];
        acc[ct][i] = __builtin_fmaf((float)S, dw[i] * dxc, acc[ct][i]);
      }
    }
  }
}

// Operands of one wave's 16-row weight tile and of the member activations, fetched in the order scales,
// activations, weights, so that writing the first two into LDS waits only for them while the weight stream is
// still in flight.
template <int NBW>
struct TileScales {
  static constexpr int N = (4 * NBW + 63) / 64;  // 8-byte pieces (4 scales) per lane
  uint2 v[N];
};

// The [NBW][16] scales of blocks b0 .. b0 + NBW - 1 of tile t16 (of a matrix with NB blocks per row), 8 bytes a
// lane.
template <int NBW>
__device__ __forceinline__ void fetch_scales(const TMat& m, size_t t16, int NB, int b0, TileScales<NBW>& sc) {
  const int lane = threadIdx.x & 63;
  const uint2* p = reinterpret_cast<const uint2*>(m.d + (t16 * NB + b0) * 16);
#pragma unroll
  for (int q = 0; q < TileScales<NBW>::N; q++)
    if (4 * NBW % 64 == 0 || lane + 64 * q < 4 * NBW) sc.v[q] = p[lane + 64 * q];
}
template <int NBW>
__device__ __forceinline__ void store_scales(const TileScales<NBW>& sc, uint16_t* sdt) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int q = 0; q < TileScales<NBW>::N; q++)
    if (4 * NBW % 64 == 0 || lane + 64 * q < 4 * NBW) reinterpret_cast<uint2*>(sdt)[lane + 64 * q] = sc.v[q];
}

// This lane's A operands of blocks b0 .. b0 + NBW - 1 of tile t16 (b0 even): one 16-byte load per pair of blocks,
// 1 KB of consecutive bytes per wave.
template <int NBW>
__device__ __forceinline__ void fetch_tile_q8(const TMat& m, size_t t16, int NB, int b0, uint4 (&a)[NBW / 2]) {
  const uint4* p = reinterpret_cast<const uint4*>(m.q) + (t16 * (NB / 2) + b0 / 2) * 64 + (threadIdx.x & 63);
#pragma unroll
  for (int q = 0; q < NBW / 2; q++) a[q] = p[q * 64];
}

// Member activations: rows row(c) for c in [0, ne) of the hi/lo planes (row length K) and their K/32 block scales;
// row(c) = off + c (member slots, contiguous) or the c-th set bit of `bits` (member positions).
template <int K, int NM, int NT>
struct Members {
  static constexpr int C16 = K / 16;
  static constexpr int PER = (NM * C16 + NT - 1) / NT;
  static constexpr int PERD = (NM * (K / 32) + NT - 1) / NT;
  uint4 h[PER], l[PER];
  float d[PERD];
};

__device__ __forceinline__ int nth_set_bit(unsigned bits, int c) {
  for (int i = 0; i < c; i++) bits &= bits - 1u;
  return __ffs(bits) - 1;
}

template <int K, int NM, int NT, bool CONTIG>
__device__ __forceinline__ void fetch_members(const int8_t* __restrict__ srch, const int8_t* __restrict__ srcl,
                                              const float* __restrict__ srcd, unsigned bits, int off, int ne,
                                              Members<K, NM, NT>& mb) {
  using M = Members<K, NM, NT>;
#pragma unroll
  for (int q = 0; q < M::PER; q++) {
    const int i = threadIdx.x + q * NT, c = i / M::C16, j = i % M::C16;
    mb.h[q] = make_uint4(0, 0, 0, 0);
    mb.l[q] = make_uint4(0, 0, 0, 0);
    if (i < NM * M::C16 && c < ne) {
      const size_t r = CONTIG ? (size_t)(off + c) : (size_t)nth_set_bit(bits, c);
      mb.h[q] = reinterpret_cast<const uint4*>(srch + r * K)[j];
      mb.l[q] = reinterpret_cast<const uint4*>(srcl + r * K)[j];
    }
  }
#pragma unroll
  for (int q = 0; q < M::PERD; q++) {
    const int i = threadIdx.x + q * NT, c = i / (K / 32), b = i % (K / 32);
    mb.d[q] = 0.0f;
    if (i < NM * (K / 32) && c < ne) mb.d[q] = srcd[(CONTIG ? (size_t)(off + c) : (size_t)nth_set_bit(bits, c)) * (K / 32) + b];
  }
}

template <int K, int NM, int NT>
__device__ __forceinline__ void store_members(const Members<K, NM, NT>& mb, int8_t* bh, int8_t* bl, int stride,
                                              float* dx) {
  using M = Members<K, NM, NT>;
#pragma unroll
  for (int q = 0; q < M::PER; q++) {
    const int i = threadIdx.x + q * NT, c = i / M::C16, j = i % M::C16;
    if (i < NM * M::C16) {
      *reinterpret_cast<uint4*>(bh + (size_t)c * stride + 16 * j) = mb.h[q];
      *reinterpret_cast<uint4*>(bl + (size_t)c * stride + 16 * j) = mb.l[q];
    }
  }
#pragma unroll
  for (int q = 0; q < M::PERD; q++) {
    const int i = threadIdx.x + q * NT;
    if (i < NM * (K / 32)) dx[i] = mb.d[q];
  }
}

}  // namespace moert

// MoE-norm partials: the rmsnorm and the router of a layer's MoE half, computed from partial sums that the kernel
// producing the hidden state (the output projection, whose epilogue holds the new residual rows) writes for blocks
// of 8 consecutive rows, so that the router kernel does not restage h, reduce its sum of squares in one wave and
// recompute the whole router before it can rank the experts.
//
// Canonical order (oracle: orc_moe_norm_route). h is cut into blocks b of kNormBlk = 8 rows; for block b
//   zp[e][b] = fma chain over t = 0..7 of Wr[e, 8b + t] * (lnw[8b + t] * h[8b + t])     (e < E)
//   zp[E][b] = fma chain over t = 0..7 of h[8b + t] * h[8b + t]
// each chain from +0 in increasing t. A consumer reduces item i over the blocks: block b goes to lane b % 64, each
// lane adds its blocks in increasing b to +0, then the 64 lanes are summed as the pairwise butterfly tree; this gives
// ss and z_e. Then r = 1 / sqrt(ss / H + eps), logits_e = z_e * r (+ bias_e), xn = lnw * (h * r).
// (rmsnorm then router, rust/moe-rt/src/model.rs:141-145 and block.rs:56-62, with r factored out of the router's
// dot products; the routing then ranks these logits as before.)
#pragma once
#include "dev_math.h"

namespace moert {

constexpr int kNormBlk = 8;       // rows per partial block
constexpr int kNormMaxBlk = 256;  // blocks per item in the partial buffer (hidden <= 2048)
constexpr int kNormItems = 65 * kNormMaxBlk;  // floats of one position's partials: [E + 1 <= 65][kNormMaxBlk]

// Raw weights of 8 consecutive columns [c0, c0 + 8) of row e of a router matrix (c0 a multiple of 8) of dtype DT:
// Q8_0 / Q4_0 8 payload bytes (w[0..1]) and the block's scale bits, f32 the 8 values. The dtype is a template
// parameter: a run-time branch around these loads would split the producer kernel's load run and make it wait.
struct Col8 {
  uint32_t w[8];
  uint32_t d;
};

template <int DT>
__device__ __forceinline__ Col8 load_col8(const DMat& m, int e, int c0) {
  Col8 c;
  const size_t row = (size_t)e;
  if (DT == DT_F32) {
    const uint4* p = reinterpret_cast<const uint4*>(m.q + (row * m.cols + c0) * 4);
    const uint4 a = gload_u4(p), b = gload_u4(p + 1);
    c.w[0] = a.x; c.w[1] = a.y; c.w[2] = a.z; c.w[3] = a.w;
    c.w[4] = b.x; c.w[5] = b.y; c.w[6] = b.z; c.w[7] = b.w;
    c.d = 0x3c00u;
  } else {
    const size_t off =
        DT == DT_Q8_0 ? row * m.cols + c0 : row * (m.cols / 2) + (size_t)(c0 / 32) * 16 + (c0 & 15);
    const uint2 v = gload_u2(m.q + off);
    c.w[0] = v.x;
    c.w[1] = v.y;
    c.w[2] = c.w[3] = c.w[4] = c.w[5] = c.w[6] = c.w[7] = 0u;
    c.d = *gmem(m.d + row * (size_t)(m.cols / 32) + c0 / 32);
  }
  return c;
}

// Element t of a Col8 (c0 says which nibble of a Q4_0 byte holds the columns): q * d, exact.
template <int DT>
__device__ __forceinline__ float col8_elem(const Col8& c, int t, int c0) {
  if (DT == DT_F32) return __uint_as_float(c.w[t]);
  const uint32_t byte = (c.w[t >> 2] >> (8 * (t & 3))) & 0xffu;
  const float d = scale_at_use(c.d);
  if (DT == DT_Q8_0) return (float)(int8_t)byte * d;
  const int nib = (c0 & 31) >= 16 ? (int)(byte >> 4) : (int)(byte & 15u);
  return (float)(nib - 8) * d;
}

// Producer side, for a workgroup of NT threads that owns rows [r0, r0 + RB) of h (RB a multiple of 8) and a router
// of dtype DT: its
// RB / 8 blocks x (E + 1) items, IPT per thread. norm_part_fetch issues the router and norm-weight loads (place it
// before the kernel's own weight loads); norm_part_finish runs once the new rows sit in LDS hn[RB] (after a
// workgroup barrier) and writes the partials of blocks r0/8 ... into zp ([E + 1][kNormMaxBlk]).
template <int RB, int NT>
struct NormPart {
  static constexpr int NBLK = RB / kNormBlk;
  static constexpr int IPT = (NBLK * 65 + NT - 1) / NT;
  Col8 w[IPT];
  float4 l0[IPT], l1[IPT];
};

template <int DT, int RB, int NT>
__device__ __forceinline__ void norm_part_fetch(const DMat& router, const float* __restrict__ lnw, int r0, int H,
                                                NormPart<RB, NT>& np) {
  using NP = NormPart<RB, NT>;
  const int E = router.rows, items = NP::NBLK * (E + 1);
#pragma unroll
  for (int i = 0; i < NP::IPT; i++) {
    int it = threadIdx.x + i * NT;
    it = it < items ? it : 0;  // clamped, not guarded: the loads stay one straight run
    const int blk = it / (E + 1), e = it % (E + 1);
    int c0 = r0 + kNormBlk * blk;
    c0 = c0 < H ? c0 : 0;
    np.w[i] = load_col8<DT>(router, e < E ? e : 0, c0);
    np.l0[i] = *reinterpret_cast<const float4*>(lnw + c0);
    np.l1[i] = *reinterpret_cast<const float4*>(lnw + c0 + 4);
  }
}

template <int DT, int RB, int NT>
__device__ __forceinline__ void norm_part_finish(const NormPart<RB, NT>& np, const float* hn, int E, int r0, int H,
                                                 float* __restrict__ zp) {
  using NP = NormPart<RB, NT>;
  const int items = NP::NBLK * (E + 1);
#pragma unroll
  for (int i = 0; i < NP::IPT; i++) {
    const int it = threadIdx.x + i * NT;
    if (it >= items) continue;
    const int blk = it / (E + 1), e = it % (E + 1);
    const int c0 = r0 + kNormBlk * blk;
    if (c0 >= H) continue;
    const float* hb = hn + kNormBlk * blk;
    const float lw[8] = {np.l0[i].x, np.l0[i].y, np.l0[i].z, np.l0[i].w,
                         np.l1[i].x, np.l1[i].y, np.l1[i].z, np.l1[i].w};
    float acc = 0.0f;
    if (e < E) {
#pragma unroll
      for (int t = 0; t < kNormBlk; t++) acc = __builtin_fmaf(col8_elem<DT>(np.w[i], t, c0), lw[t] * hb[t], acc);
    } else {
#pragma unroll
      for (int t = 0; t < kNormBlk; t++) acc = __builtin_fmaf(hb[t], hb[t], acc);
    }
    zp[(size_t)e * kNormMaxBlk + c0 / kNormBlk] = acc;
  }
}

// Consumer side: item `item` of the partials reduced over nb blocks by one wave (every lane gets the sum). The
// loads are issued by norm_item_fetch (unconditional: entries past nb are allocated and discarded).
struct NormItem {
  float v[kNormMaxBlk / 64];
};

__device__ __forceinline__ void norm_item_fetch(const float* __restrict__ zp, int item, int lane, NormItem& it) {
#pragma unroll
  for (int q = 0; q < kNormMaxBlk / 64; q++) it.v[q] = zp[(size_t)item * kNormMaxBlk + lane + 64 * q];
}

__device__ __forceinline__ float norm_item_sum(const NormItem& it, int nb, int lane) {
  float acc = 0.0f;
#pragma unroll
  for (int q = 0; q < kNormMaxBlk / 64; q++)
    if (lane + 64 * q < nb) acc = acc + it.v[q];
  return group_sum<64>(acc);
}

}  // namespace moert

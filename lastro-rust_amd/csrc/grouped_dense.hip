// Dense half of the multi-position step in grouped mode: the q/k/v and output projections of m <= 32 positions as
// int8 MFMA GEMMs over the tiled Q8_0 weights (the dense kernels of the reference's block prefill,
// rust/moe-rt/src/cuda_dense.rs:236-288, whose per-position GEMVs this replaces by one pass over each weight row),
// the RMSNorms and 15-bit activation codes that feed them, and the experts' combine with the residual.
//
// Arithmetic (the same as the grouped experts): every weight block times the 15-bit codes of the activation block
// is an exact int32, scaled by the two block scales and accumulated in block order; a projection's K range is cut
// into four quarters, one per wave, whose sums are added in quarter order. The results differ from the per-row FMA
// kernels (which equal the decode step bit for bit) by the rounding of the codes, about 3e-5 of each block's
// largest element.
//
// Kernels:
//   k_gd_dense<K, NM, GD_QKV>  grid 2 * rows/64:  rows 16h..16h+15 and 32+16h..32+16h+15 of one head (h = half),
//                                                 RoPE on the (j, j+32) pairs, q in f32, K and V into the fp16 cache
//   k_gd_dense<K, NM, GD_RES>  grid rows/32:      32 rows of the output projection, h += res * (Wo att)
//   k_gd_norm_codes<H>         grid m:            codes of rmsnorm(h[p], lnw)
//   k_gd_combine<H>            grid m:            h[p] += res * (sum over p's experts in list order of w * o), then
//                                                 optionally the codes of rmsnorm(h[p], lnw) for the next layer
#include "dev_rows.h"
#include "grouped.h"
#include "launch.h"
#include "mfma_q8.h"

namespace moert {

enum { GD_QKV = 0, GD_RES = 1 };
constexpr int kGdThreads = 512;  // 8 waves: wave w takes row set w & 1 and K quarter w >> 1

// Epilogue arguments: GD_QKV uses rope .. vc, GD_RES uses h and res.
struct GdEpi {
  const float* rope;  // [max_len, 64]: cos of the 32 frequencies, then sin
  int pos0, heads, kvh, max_len;
  float* q;           // [m, heads * 64]
  uint16_t* kc;       // [kvh, max_len, 64]
  uint16_t* vc;
  float* h;           // [m, rows]
  float res;
};

template <int K, int NM, int EPI>
__global__ __launch_bounds__(kGdThreads) void k_gd_dense(TMat w, int m, const int8_t* __restrict__ xh,
                                                         const int8_t* __restrict__ xl, const float* __restrict__ xd,
                                                         GdEpi ep) {
  constexpr int NB = K / 32, NBW = NB / 4, STR = K + 16;
  static_assert(NB % 8 == 0, "each K quarter is whole pairs of blocks");
  __shared__ __align__(16) int8_t bh[NM * STR];
  __shared__ __align__(16) int8_t bl[NM * STR];
  __shared__ float dx[NM * NB];
  __shared__ __align__(16) uint16_t sdt[kGdThreads / 64][NBW * 16];
  __shared__ float red[4][32][NM + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p = wave & 1, kq = wave >> 1;
  const int row0 = EPI == GD_QKV ? (blockIdx.x >> 1) * 64 + 16 * (blockIdx.x & 1) + 32 * p : 32 * blockIdx.x + 16 * p;
  const size_t t16 = (size_t)row0 / 16;
  TileScales<NBW> sc;
  fetch_scales<NBW>(w, t16, NB, kq * NBW, sc);
  Members<K, NM, kGdThreads> mb;
  fetch_members<K, NM, kGdThreads, true>(xh, xl, xd, 0u, 0, m, mb);
  uint4 a[NBW / 2];
  fetch_tile_q8<NBW>(w, t16, NB, kq * NBW, a);
  store_scales<NBW>(sc, sdt[wave]);
  store_members<K, NM, kGdThreads>(mb, bh, bl, STR, dx);
  __syncthreads();
  float acc[NM / 16][4];
  mfma_tile<NBW, NM>(a, bh + 32 * kq * NBW, bl + 32 * kq * NBW, STR, sdt[wave], dx + kq * NBW, NB, acc);
  const int grp = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < NM / 16; ct++)
#pragma unroll
    for (int i = 0; i < 4; i++) red[kq][16 * p + 4 * grp + i][16 * ct + (lane & 15)] = acc[ct][i];
  __syncthreads();
  auto sum = [&](int r, int c) { return ((red[0][r][c] + red[1][r][c]) + red[2][r][c]) + red[3][r][c]; };
  if (EPI == GD_QKV) {
    // thread (c, jj): the pair (row jp, row jp + 32) of the head for position c, jp = 16 * half + jj
    const int jj = threadIdx.x & 15, c = threadIdx.x >> 4;
    if (c >= NM || c >= m) return;
    const float x1 = sum(jj, c), x2 = sum(16 + jj, c);
    const int head = blockIdx.x >> 1, jp = 16 * (blockIdx.x & 1) + jj;
    const int pos = ep.pos0 + c;
    const float cs = ep.rope[(size_t)pos * 64 + jp], sn = ep.rope[(size_t)pos * 64 + 32 + jp];
    if (head < ep.heads) {
      float* qv = ep.q + (size_t)c * ep.heads * 64 + head * 64;
      qv[jp] = x1 * cs - x2 * sn;
      qv[jp + 32] = x2 * cs + x1 * sn;
    } else if (head < ep.heads + ep.kvh) {
      uint16_t* kp = ep.kc + ((size_t)(head - ep.heads) * ep.max_len + pos) * 64;
      kp[jp] = f2h(x1 * cs - x2 * sn);
      kp[jp + 32] = f2h(x2 * cs + x1 * sn);
    } else {
      uint16_t* vp = ep.vc + ((size_t)(head - ep.heads - ep.kvh) * ep.max_len + pos) * 64;
      vp[jp] = f2h(x1);
      vp[jp + 32] = f2h(x2);
    }
  } else {
    for (int it = threadIdx.x; it < 32 * NM; it += kGdThreads) {
      const int r = it & 31, c = it >> 5;
      if (c < m) {
        float* hp = ep.h + (size_t)c * w.rows + 32 * blockIdx.x + r;
        *hp = *hp + ep.res * sum(r, c);
      }
    }
  }
}

// rmsnorm of the row whose elements 1024 j + 4 t .. +3 (pass j) this thread holds in hv, then the codes of the
// normalised row (block b = 32 j + t / 8, part t % 8). The whole workgroup (256 threads) takes part.
template <int H>
__device__ __forceinline__ void norm_codes_tail(const float (&hv)[(H + 1023) / 1024][4], float ss, int p,
                                                const float* __restrict__ lnw, float eps, GroupBufs g) {
  constexpr int NP = (H + 1023) / 1024;
  __shared__ float wsum[4];
  const int t = threadIdx.x;
  ss = group_sum<64>(ss);
  if ((t & 63) == 0) wsum[t >> 6] = ss;
  __syncthreads();
  const float tot = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  const float r = 1.0f / sqrtf(tot / (float)H + eps);
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const int e0 = 1024 * j + 4 * t;
    const bool valid = e0 < H;
    const float4 lw = *reinterpret_cast<const float4*>(lnw + (valid ? e0 : 0));
    const float v[4] = {lw.x * (hv[j][0] * r), lw.y * (hv[j][1] * r), lw.z * (hv[j][2] * r), lw.w * (hv[j][3] * r)};
    block_codes<H>(v, valid, p, e0 / 32, t & 7, g.xh, g.xl, g.xd);
  }
}

template <int H>
__global__ __launch_bounds__(256) void k_gd_norm_codes(const float* __restrict__ h, const float* __restrict__ lnw,
                                                       float eps, GroupBufs g) {
  constexpr int NP = (H + 1023) / 1024;
  const int p = blockIdx.x, t = threadIdx.x;
  float hv[NP][4];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const int e0 = 1024 * j + 4 * t;
    const bool valid = e0 < H;
    const float4 x = *reinterpret_cast<const float4*>(h + (size_t)p * H + (valid ? e0 : 0));
    hv[j][0] = valid ? x.x : 0.0f;
    hv[j][1] = valid ? x.y : 0.0f;
    hv[j][2] = valid ? x.z : 0.0f;
    hv[j][3] = valid ? x.w : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) ss = __builtin_fmaf(hv[j][i], hv[j][i], ss);
  }
  norm_codes_tail<H>(hv, ss, p, lnw, eps, g);
}

template <int H>
__global__ __launch_bounds__(256) void k_gd_combine(int k, float res, float* __restrict__ h,
                                                    const float* __restrict__ lnw, float eps, GroupBufs g) {
  constexpr int NP = (H + 1023) / 1024;
  const int p = blockIdx.x, t = threadIdx.x;
  int sl[8];
  float wt[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    sl[j] = j < k ? g.grp[GRP_ORD_SLOT + p * 8 + j] : 0;
    wt[j] = j < k ? __int_as_float(g.grp[GRP_ORD_W + p * 8 + j]) : 0.0f;
  }
  float hv[NP][4];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const int e0 = 1024 * j + 4 * t;
    const bool valid = e0 < H;
    const int ec = valid ? e0 : 0;
    float4 ov[8];
#pragma unroll
    for (int u = 0; u < 8; u++)
      ov[u] = u < k ? *reinterpret_cast<const float4*>(g.o + (size_t)sl[u] * H + ec) : make_float4(0, 0, 0, 0);
    float4* hp = reinterpret_cast<float4*>(h + (size_t)p * H + ec);
    const float4 ho = *hp;
    float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (u < k) {
        const float o4[4] = {ov[u].x, ov[u].y, ov[u].z, ov[u].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float tw = wt[u] * o4[i];
          y[i] = y[i] + tw;
        }
      }
    const float hn[4] = {ho.x + res * y[0], ho.y + res * y[1], ho.z + res * y[2], ho.w + res * y[3]};
    if (valid) *hp = make_float4(hn[0], hn[1], hn[2], hn[3]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      hv[j][i] = valid ? hn[i] : 0.0f;
      ss = __builtin_fmaf(hv[j][i], hv[j][i], ss);
    }
  }
  if (lnw) norm_codes_tail<H>(hv, ss, p, lnw, eps, g);
}

// ------------------------------------------------------------------------------------------------------------
template <int K, int EPI>
static void dense_launch(hipStream_t s, int grid, const TMat& w, int m, const GroupBufs& g, const GdEpi& ep) {
  if (m > 16)
    klaunch(k_gd_dense<K, 32, EPI>, grid, kGdThreads, 0, s, w, m, g.xh, g.xl, g.xd, ep);
  else
    klaunch(k_gd_dense<K, 16, EPI>, grid, kGdThreads, 0, s, w, m, g.xh, g.xl, g.xd, ep);
}

hipError_t launch_gd_qkv(hipStream_t s, const Dims& d, int m, int pos0, const float* rope, float* q, uint16_t* kc,
                         uint16_t* vc, const GroupBufs& g) {
  const TMat& w = g.qkv;
  if (m < 1 || m > kGrpMaxPos || !w.q || d.head_dim != 64 || w.rows != (d.heads + 2 * d.kv_heads) * 64 ||
      w.cols != d.hidden || pos0 < 0 || pos0 + m > d.max_len)
    return hipErrorInvalidValue;
  GdEpi ep{rope, pos0, d.heads, d.kv_heads, d.max_len, q, kc, vc, nullptr, 0.0f};
  const int grid = w.rows / 64 * 2;
  switch (w.cols) {
    case 1024: dense_launch<1024, GD_QKV>(s, grid, w, m, g, ep); break;
    case 1536: dense_launch<1536, GD_QKV>(s, grid, w, m, g, ep); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gd_oproj(hipStream_t s, int m, float res, float* h, const GroupBufs& g) {
  const TMat& w = g.oproj;
  if (m < 1 || m > kGrpMaxPos || !w.q || w.rows % 32) return hipErrorInvalidValue;
  GdEpi ep{nullptr, 0, 0, 0, 0, nullptr, nullptr, nullptr, h, res};
  switch (w.cols) {
    case 1024: dense_launch<1024, GD_RES>(s, w.rows / 32, w, m, g, ep); break;
    case 1536: dense_launch<1536, GD_RES>(s, w.rows / 32, w, m, g, ep); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_norm_codes(hipStream_t s, int H, int m, const float* h, const float* lnw, float eps,
                             const GroupBufs& g) {
  if (m < 1 || m > kGrpMaxPos || !lnw) return hipErrorInvalidValue;
  switch (H) {
    case 1024: klaunch(k_gd_norm_codes<1024>, m, 256, 0, s, h, lnw, eps, g); break;
    case 1536: klaunch(k_gd_norm_codes<1536>, m, 256, 0, s, h, lnw, eps, g); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gd_combine(hipStream_t s, int H, int m, int k, float res, float* h, const float* lnw, float eps,
                             const GroupBufs& g) {
  if (m < 1 || m > kGrpMaxPos || k < 1 || k > 8) return hipErrorInvalidValue;
  switch (H) {
    case 1024: klaunch(k_gd_combine<1024>, m, 256, 0, s, k, res, h, lnw, eps, g); break;
    case 1536: klaunch(k_gd_combine<1536>, m, 256, 0, s, k, res, h, lnw, eps, g); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace moert

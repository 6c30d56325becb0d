// Row-streaming building blocks shared by the GEMV-shaped kernels (gfx950, wave64): row geometry, chunk loads
// issued ahead of the activations, the canonical per-row FMA chain, workgroup prologues and the wave top-k.
#pragma once
#include "dev_math.h"

namespace moert {

constexpr int kBlock = 256;  // 4 waves per workgroup
constexpr int kWavesPerBlock = kBlock / kWave;

// Row geometry of a [rows, K] matrix of dtype DT: NCH chunks of CE elements per row. When NCH < 64 a row only
// needs LPR = next power of two >= NCH lanes, so a wave covers RPW = 64 / LPR rows per pass (the canonical
// 64-lane tree then only adds zeros beyond LPR). Lane `sub` of a row owns chunks sub, sub + LPR, ... (NJ of them).
// Lanes per row: the smallest power of two >= NCH, at most 64 (chunk j must sit in lane j % 64).
__host__ __device__ constexpr int lanes_per_row(int nch) {
  return nch > 32 ? 64 : nch > 16 ? 32 : nch > 8 ? 16 : nch > 4 ? 8 : nch > 2 ? 4 : nch > 1 ? 2 : 1;
}

template <int DT, int K>
struct Geo {
  static constexpr int CE = Fmt<DT>::kElems;
  static constexpr int NCH = K / CE;
  static constexpr int LPR = lanes_per_row(NCH);
  static constexpr int RPW = kWave / LPR;
  static constexpr int NJ = (NCH + LPR - 1) / LPR;
  static_assert(K % CE == 0 && K % 32 == 0, "row length must be a multiple of 32");
};

// The activations a lane needs: its chunks of x.
template <int DT, int K>
struct XReg {
  float v[Geo<DT, K>::NJ][Geo<DT, K>::CE];
};

template <int DT, int K>
__device__ __forceinline__ void load_x(XReg<DT, K>& xr, const float* __restrict__ x, int sub) {
  using G = Geo<DT, K>;
#pragma unroll
  for (int jj = 0; jj < G::NJ; jj++) {
    int j = sub + G::LPR * jj;
    if (j < G::NCH) {
      const float4* p = reinterpret_cast<const float4*>(x + j * G::CE);
#pragma unroll
      for (int e = 0; e < G::CE / 4; e++) {
        float4 t = p[e];
        xr.v[jj][4 * e] = t.x;
        xr.v[jj][4 * e + 1] = t.y;
        xr.v[jj][4 * e + 2] = t.z;
        xr.v[jj][4 * e + 3] = t.w;
      }
    }
  }
}

// xn = w * (x * r) on the lane's chunks (rust/moe-rt/src/model.rs:141-145).
template <int DT, int K>
__device__ __forceinline__ void load_xn(XReg<DT, K>& xr, const float* __restrict__ x, const float* __restrict__ w,
                                        float r, int sub) {
  using G = Geo<DT, K>;
#pragma unroll
  for (int jj = 0; jj < G::NJ; jj++) {
    int j = sub + G::LPR * jj;
    if (j < G::NCH) {
      const float4* p = reinterpret_cast<const float4*>(x + j * G::CE);
      const float4* q = reinterpret_cast<const float4*>(w + j * G::CE);
#pragma unroll
      for (int e = 0; e < G::CE / 4; e++) {
        float4 t = p[e], s = q[e];
        xr.v[jj][4 * e] = s.x * (t.x * r);
        xr.v[jj][4 * e + 1] = s.y * (t.y * r);
        xr.v[jj][4 * e + 2] = s.z * (t.z * r);
        xr.v[jj][4 * e + 3] = s.w * (t.w * r);
      }
    }
  }
}

// Canonical sum of squares of x[0, K): 16-element chunks over 64 lanes.
template <int K>
__device__ __forceinline__ float sumsq(const float* __restrict__ x, int lane) {
  constexpr int NCH = K / 16;
  float acc = 0.0f;
#pragma unroll
  for (int jj = 0; jj < (NCH + 63) / 64; jj++) {
    int j = lane + 64 * jj;
    if (j < NCH) {
      const float4* p = reinterpret_cast<const float4*>(x + 16 * j);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float4 t = p[e];
        acc = __builtin_fmaf(t.x, t.x, acc);
        acc = __builtin_fmaf(t.y, t.y, acc);
        acc = __builtin_fmaf(t.z, t.z, acc);
        acc = __builtin_fmaf(t.w, t.w, acc);
      }
    }
  }
  return group_sum<64>(acc);
}

template <int K>
__device__ __forceinline__ float rms_scale(const float* __restrict__ x, float eps, int lane) {
  float ss = sumsq<K>(x, lane);
  return 1.0f / sqrtf(ss / (float)K + eps);
}

// Chunk registers of P rows. rows_load issues every load before any arithmetic (and before the activations are
// ready), rows_fma does the canonical chain per row; out[p] ends up in every lane of the group owning row[p].
template <int DT, int K, int P>
struct Rows {
  RawChunk c[P][Geo<DT, K>::NJ];
};

template <int DT, int K, int P>
__device__ __forceinline__ void rows_load(Rows<DT, K, P>& r, const DMat& m, const size_t (&row)[P],
                                          const bool (&ok)[P], int sub) {
  using G = Geo<DT, K>;
#pragma unroll
  for (int p = 0; p < P; p++)
#pragma unroll
    for (int jj = 0; jj < G::NJ; jj++) {
      int j = sub + G::LPR * jj;
      if (ok[p] && j < G::NCH) r.c[p][jj] = load_chunk<DT>(m, row[p], j);
    }
}

template <int DT, int K, int P>
__device__ __forceinline__ void rows_fma(const Rows<DT, K, P>& r, const bool (&ok)[P], const XReg<DT, K>& xr,
                                         int sub, float (&out)[P]) {
  using G = Geo<DT, K>;
#pragma unroll
  for (int p = 0; p < P; p++) {
    float acc = 0.0f;
#pragma unroll
    for (int jj = 0; jj < G::NJ; jj++) {
      int j = sub + G::LPR * jj;
      if (ok[p] && j < G::NCH) acc = fma_chunk<DT>(r.c[p][jj], xr.v[jj], acc);
    }
    out[p] = group_sum<G::LPR>(acc);
  }
}

// Workgroup prologues: the block's activation vector in LDS, once per workgroup.
// wg_norm: xs = lnw * (x * r), r = 1/sqrt(sum(x^2)/K + eps), the sum in the canonical order by wave 0.
template <int K, int NT>
__device__ __forceinline__ void wg_norm(const float* __restrict__ x, const float* __restrict__ lnw, float eps,
                                        float* xs, float* rs) {
  constexpr int PER = (K + NT - 1) / NT;
  float hv[PER], wv[PER];
#pragma unroll
  for (int e = 0; e < PER; e++) {
    int i = threadIdx.x + e * NT;
    if (i < K) {
      hv[e] = x[i];
      wv[e] = lnw[i];
    }
  }
  if (threadIdx.x < 64) {
    float r = rms_scale<K>(x, eps, threadIdx.x);
    if (threadIdx.x == 0) *rs = r;
  }
  __syncthreads();
  const float r = *rs;
#pragma unroll
  for (int e = 0; e < PER; e++) {
    int i = threadIdx.x + e * NT;
    if (i < K) xs[i] = wv[e] * (hv[e] * r);
  }
  __syncthreads();
}

template <int N, int NT>
__device__ __forceinline__ void wg_copy(const float* __restrict__ x, float* xs) {
  static_assert(N % 4 == 0, "vector copy");
  for (int i = threadIdx.x; i < N / 4; i += NT)
    reinterpret_cast<float4*>(xs)[i] = reinterpret_cast<const float4*>(x)[i];
  __syncthreads();
}

// Top-k of n <= 64 logits held in LDS (lg), by rank: lane e counts the logits that precede it in the order
// (total-order key descending, index ascending) and, if its rank is below k, takes that slot; then
// w_j = exp(l_j - l_top) / sum with the sum taken left to right (Routing::from_logits, block.rs:81-89; route_topk,
// route.rs:18-75). `slot` is 3*64 words of LDS. ids/weights written by lanes j < k.
__device__ __forceinline__ void wave_topk(const float* lg, int n, int k, int lane, float* slot, int* ids,
                                          float* weights) {
  const float v = lane < n ? lg[lane] : 0.0f;
  const int key = total_key(v);
  int rank = 0;
  // all 64 slots read as float4 up front (slots >= n hold stale values and are skipped)
  float4 all[16];
#pragma unroll
  for (int j4 = 0; j4 < 16; j4++) all[j4] = reinterpret_cast<const float4*>(lg)[j4];
#pragma unroll
  for (int j4 = 0; j4 < 16; j4++) {
    const float a4[4] = {all[j4].x, all[j4].y, all[j4].z, all[j4].w};
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int j = 4 * j4 + u;
      const int kj = total_key(a4[u]);
      rank += j < n && ((kj > key) || (kj == key && j < lane));
    }
  }
  float* sval = slot;
  int* sid = reinterpret_cast<int*>(slot + 64);
  float* sex = slot + 128;
  if (lane < n && rank < k) {
    sval[rank] = v;
    sid[rank] = lane;
  }
  wave_lds_sync();
  const float ex = lane < k ? dexp(sval[lane] - sval[0]) : 0.0f;
  sex[lane] = ex;
  wave_lds_sync();
  float sum = 0.0f;
  for (int j = 0; j < k; j++) sum = sum + sex[j];
  if (lane < k) {
    ids[lane] = sid[lane];
    weights[lane] = ex / sum;
  }
}

}  // namespace moert

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

// Loads are unconditional (a row that is not used loads row 0, a chunk past the row end loads the last chunk) so
// that they form one straight run of independent loads; rows_fma skips what is not used.
// NT: the loads carry the non-temporal hint.
template <int DT, int K, int P, bool NT = false>
__device__ __forceinline__ void rows_load(Rows<DT, K, P>& r, const DMat& m, const size_t (&row)[P],
                                          const bool (&ok)[P], int sub) {
  using G = Geo<DT, K>;
#pragma unroll
  for (int p = 0; p < P; p++)
#pragma unroll
    for (int jj = 0; jj < G::NJ; jj++) {
      const int j = sub + G::LPR * jj;
      r.c[p][jj] = load_chunk<DT, NT>(m, ok[p] ? row[p] : 0, j < G::NCH ? j : G::NCH - 1);
    }
}

// rows_load with a matrix per row (rows of routed experts that live in different places).
template <int DT, int K, int P>
__device__ __forceinline__ void rows_load_from(Rows<DT, K, P>& r, const DMat (&m)[P], const size_t (&row)[P],
                                               const bool (&ok)[P], int sub) {
  using G = Geo<DT, K>;
#pragma unroll
  for (int p = 0; p < P; p++)
#pragma unroll
    for (int jj = 0; jj < G::NJ; jj++) {
      const int j = sub + G::LPR * jj;
      r.c[p][jj] = load_chunk<DT>(m[p], ok[p] ? row[p] : 0, j < G::NCH ? j : G::NCH - 1);
    }
}

// Writes the lane's chunks of row p back, as loaded, into row dst_row[p] of `dst` where put[p] (the chunk payload
// and its scale; for Q8_0 the even chunk of a block writes the block's scale).
template <int DT, int K, int P>
__device__ __forceinline__ void rows_store(const Rows<DT, K, P>& r, const DMat& dst, const size_t (&dst_row)[P],
                                           const bool (&put)[P], int sub) {
  using G = Geo<DT, K>;
#pragma unroll
  for (int p = 0; p < P; p++) {
    if (!put[p]) continue;
#pragma unroll
    for (int jj = 0; jj < G::NJ; jj++) {
      const int j = sub + G::LPR * jj;
      if (j >= G::NCH) continue;
      uint8_t* base = const_cast<uint8_t*>(dst.q) + dst_row[p] * Fmt<DT>::row_bytes(dst.cols);
      *reinterpret_cast<uint4*>(base + (size_t)j * 16) = r.c[p][jj].v;
      uint16_t* sc = const_cast<uint16_t*>(dst.d) + dst_row[p] * (size_t)(dst.cols / 32);
      if (DT == DT_Q8_0 && (j & 1) == 0) sc[j >> 1] = (uint16_t)r.c[p][jj].d;
      if (DT == DT_Q4_0) sc[j] = (uint16_t)r.c[p][jj].d;
    }
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

// Workgroup prologues: the block's activation vector in LDS, once per workgroup. Each comes as a fetch, which only
// issues the loads and is placed before a kernel's weight loads, and a finish, which uses them: loads complete in
// issue order, so the prologue then waits only for the activation while the weights are still streaming.
//
// Norm: xs = lnw * (x * r), r = 1/sqrt(sum(x^2)/K + eps), the sum in the canonical order by wave 0 (16-element
// chunks, chunk j in lane j % 64) over x staged in LDS. Fetch loads are unconditional (clamped indices) so that no
// branch join forces an early wait.
template <int K, int NT>
struct NormIn {
  static_assert(K % 4 == 0, "the activation is fetched in 16-byte quads");
  static constexpr int Q = K / 4;                 // quads of the vector
  static constexpr int PER = (Q + NT - 1) / NT;   // quads per thread: quad threadIdx.x + e * NT
  float4 hv[PER], wv[PER];
};

template <int K, int NT>
__device__ __forceinline__ void norm_fetch(const float* __restrict__ x, const float* __restrict__ lnw,
                                           NormIn<K, NT>& in) {
  constexpr int Q = NormIn<K, NT>::Q;
#pragma unroll
  for (int e = 0; e < NormIn<K, NT>::PER; e++) {
    const int q = threadIdx.x + e * NT, qc = q < Q ? q : Q - 1;
    in.hv[e] = reinterpret_cast<const float4*>(x)[qc];
    in.wv[e] = reinterpret_cast<const float4*>(lnw)[qc];
  }
  __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the kernel's weight loads
}

template <int K, int NT>
__device__ __forceinline__ void norm_finish(const NormIn<K, NT>& in, float eps, float* xs, float* rs) {
  constexpr int NCH = K / 16, Q = NormIn<K, NT>::Q;
  float4* xq = reinterpret_cast<float4*>(xs);
#pragma unroll
  for (int e = 0; e < NormIn<K, NT>::PER; e++) {
    const int q = threadIdx.x + e * NT;
    if (q < Q) xq[q] = in.hv[e];
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    float acc = 0.0f;
#pragma unroll
    for (int jj = 0; jj < (NCH + 63) / 64; jj++) {
      const int j = threadIdx.x + 64 * jj;
      if (j < NCH) {
        const float4* p = reinterpret_cast<const float4*>(xs + 16 * j);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float4 t = p[e];
          acc = __builtin_fmaf(t.x, t.x, acc);
          acc = __builtin_fmaf(t.y, t.y, acc);
          acc = __builtin_fmaf(t.z, t.z, acc);
          acc = __builtin_fmaf(t.w, t.w, acc);
        }
      }
    }
    const float ss = group_sum<64>(acc);
    if (threadIdx.x == 0) *rs = 1.0f / sqrtf(ss / (float)K + eps);
  }
  __syncthreads();
  const float r = *rs;
#pragma unroll
  for (int e = 0; e < NormIn<K, NT>::PER; e++) {
    const int q = threadIdx.x + e * NT;
    const float4 h = in.hv[e], w = in.wv[e];
    if (q < Q) xq[q] = make_float4(w.x * (h.x * r), w.y * (h.y * r), w.z * (h.z * r), w.w * (h.w * r));
  }
  __syncthreads();
}

template <int K, int NT>
__device__ __forceinline__ void wg_norm(const float* __restrict__ x, const float* __restrict__ lnw, float eps,
                                        float* xs, float* rs) {
  NormIn<K, NT> in;
  norm_fetch<K, NT>(x, lnw, in);
  norm_finish<K, NT>(in, eps, xs, rs);
}

// Copy: xs = x[0, N).
template <int N, int NT>
struct CopyIn {
  static constexpr int PER = (N / 4 + NT - 1) / NT;
  float4 v[PER];
};

template <int N, int NT>
__device__ __forceinline__ void copy_fetch(const float* __restrict__ x, CopyIn<N, NT>& in) {
  static_assert(N % 4 == 0, "vector copy");
#pragma unroll
  for (int e = 0; e < CopyIn<N, NT>::PER; e++) {
    const int i = threadIdx.x + e * NT;
    in.v[e] = reinterpret_cast<const float4*>(x)[i < N / 4 ? i : 0];
  }
  __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the kernel's weight loads
}

template <int N, int NT>
__device__ __forceinline__ void copy_finish(const CopyIn<N, NT>& in, float* xs) {
#pragma unroll
  for (int e = 0; e < CopyIn<N, NT>::PER; e++) {
    // unconditional store: a thread past the end holds x[0..3] (the clamped fetch) and writes it where thread 0
    // writes the same values; a conditional store would let the compiler sink the fetch below the weight loads
    const int i = threadIdx.x + e * NT;
    reinterpret_cast<float4*>(xs)[i < N / 4 ? i : 0] = in.v[e];
  }
  __syncthreads();
}

template <int N, int NT>
__device__ __forceinline__ void wg_copy(const float* __restrict__ x, float* xs) {
  CopyIn<N, NT> in;
  copy_fetch<N, NT>(x, in);
  copy_finish<N, NT>(in, xs);
}

// Ranks of n <= 64 logits held in LDS (lg[64], visible to the whole workgroup), by all NW waves: wave w counts, for
// every lane e, the 64-bit sort keys of logits [w * 64 / NW, (w + 1) * 64 / NW) above lane e's key (total-order key,
// then 63 - e: descending value, ties to the lower index); the counts meet in LDS (part[wave][lane]: a wave's counts
// in consecutive words, free of bank conflicts) and every wave adds them in wave order. Returns the rank of lane e's
// logit (the same in every wave); contains a workgroup barrier.
template <int NW>
__device__ __forceinline__ int wg_rank(const float* lg, int n, int lane, int wave, int (*part)[64]) {
  constexpr int PER = 64 / NW;
  static_assert(64 % NW == 0, "waves must divide 64");
  // lg[e] is read for every e < 64 and the entries at and past n are discarded afterwards: a read under the
  // condition would be a branch and a wait of its own per key
  auto key = [&](int e) -> unsigned long long {
    const unsigned long long kv =
        ((unsigned long long)((unsigned)total_key(lg[e]) ^ 0x80000000u) << 6) | (unsigned)(63 - e);
    return e < n ? kv : 0ull;
  };
  const unsigned long long mine = key(lane);
  int cnt = 0;
#pragma unroll
  for (int u = 0; u < PER; u++) cnt += key(wave * PER + u) > mine;
  part[wave][lane] = cnt;
  __syncthreads();
  int rank = 0;
#pragma unroll
  for (int w = 0; w < NW; w++) rank += part[w][lane];
  return rank;
}

// The ids of ranks 0..k-1 (k <= 8) as wave-uniform values: id[r] = the lane whose rank is r.
__device__ __forceinline__ void ids_by_rank(bool sel, int rank, int k, int (&id)[8]) {
#pragma unroll
  for (int r = 0; r < 8; r++) {
    const unsigned long long b = __ballot(sel && rank == r);
    id[r] = r < k && b ? __ffsll((long long)b) - 1 : 0;
  }
}

// Routing weights of the selected lanes: w = exp(l - l_top) / sum, the sum over ranks 0..k-1 left to right
// (Routing::from_logits, block.rs:81-89); the lane of rank r writes ids[r] and weights[r].
__device__ __forceinline__ void route_weights(const float* lg, bool sel, int rank, int k, int lane,
                                              const int (&id)[8], int* ids, float* weights) {
  const float v = lg[lane];
  const float ex = sel ? dexp(v - lg[id[0]]) : 0.0f;
  float sum = 0.0f;
#pragma unroll
  for (int r = 0; r < 8; r++)
    if (r < k) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), id[r]));
  if (sel) {
    ids[rank] = lane;
    weights[rank] = ex / sum;
  }
}

// Top-k of n <= 64 logits held in LDS (lg[64]), by one wave. Lane e holds logit e as one 64-bit sort key
// (total-order key, then 63 - e, so that larger means earlier: descending value, ties to the lower index); the keys
// are broadcast through LDS and each lane counts the keys above its own, which is its rank; a lane whose rank is
// below k is selected. Then w_j = exp(l_j - l_top) / sum with the sum taken left to right in rank order
// (Routing::from_logits, block.rs:81-89; route_topk, route.rs:18-75). ids[r] / weights[r] are written by the lane of
// rank r (k <= 8).
struct TopkLds {
  unsigned long long keys[64];
  float val[8];
  float ex[8];
};

__device__ __forceinline__ void wave_topk(const float* lg, int n, int k, int lane, TopkLds& t, int* ids,
                                          float* weights) {
  const float lv = lg[lane];  // read unconditionally (lg holds 64 entries), discarded past n
  const float v = lane < n ? lv : 0.0f;
  const unsigned long long mine =
      ((unsigned long long)((unsigned)total_key(v) ^ 0x80000000u) << 6) | (unsigned)(63 - lane);
  t.keys[lane] = lane < n ? mine : 0ull;
  if (lane < 8) t.ex[lane] = 0.0f;
  wave_lds_sync();
  // the 64 keys in 4 batches of 8 independent 16-byte reads (one round trip per batch, not per read)
  int rank = 0;
#pragma unroll
  for (int b = 0; b < 4; b++) {
    ulonglong2 kk[8];
#pragma unroll
    for (int j2 = 0; j2 < 8; j2++) kk[j2] = reinterpret_cast<const ulonglong2*>(t.keys)[8 * b + j2];
#pragma unroll
    for (int j2 = 0; j2 < 8; j2++) {
      rank += kk[j2].x > mine;
      rank += kk[j2].y > mine;
    }
  }
  const bool sel = lane < n && rank < k;
  if (sel) t.val[rank] = v;
  wave_lds_sync();
  const float ex = sel ? dexp(v - t.val[0]) : 0.0f;
  if (sel) t.ex[rank] = ex;
  wave_lds_sync();
  const float4 e0 = *reinterpret_cast<const float4*>(&t.ex[0]);
  const float4 e1 = *reinterpret_cast<const float4*>(&t.ex[4]);
  const float ev[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
  float sum = 0.0f;
#pragma unroll
  for (int r = 0; r < 8; r++)
    if (r < k) sum = sum + ev[r];
  if (sel) {
    ids[rank] = lane;
    weights[rank] = ex / sum;
  }
}

}  // namespace moert

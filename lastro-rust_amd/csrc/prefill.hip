// Multi-position step of the whole model: m <= 32 consecutive positions in one pass per layer (the block prefill
// `le_ids`, rust/moe-rt/src/motor/leitura.rs:79-85, through begin_step_tokens and the per-position loops of the model
// step, cuda_backend.rs:499-516, 751-917). Every weight row is read from HBM once per block of positions and applied
// to each position's activation with the decode kernels' per-row chain (chunk j of a row accumulated by lane
// j % 64 as an fmaf chain, then the pairwise lane tree), so the step equals m single-position decode steps bit for
// bit: the KV rows it appends, every hidden state and the last position's logits.
//
// Kernels per layer (one stream, in order):
//   k_qkv_b        rmsnorm of each position, [q; k; v] rows of the layer once for all positions, RoPE at each
//                  position, q to qb[v], k and v to row pos0 + v of the KV cache
//   attention      the decode attention kernels over a grid of positions, position v attending to pos0 + v + 1
//   k_oproj_b      output projection once for all positions, h[v] += res * (Wo att[v]); MoE-norm partials of each
//                  position's new rows (moe_norm.h)
//   k_route_b      per position: rmsnorm scale, router logits from the partials, top-k and weights (the decode
//                  router); xn[v] kept
//   k_moe_up_b     per routed expert: its gate/up rows once, applied to the positions routed to it; SwiGLU into
//                  act[v][j] (j = the expert's top-k rank at position v)
//   k_moe_down_b   per routed expert: its down rows once for its positions, o[v][j] = down . act[v][j]
//   k_moe_comb_b   h[v] += res * sum over j in top-k order of w[v][j] * o[v][j]
#include <algorithm>

#include "cache.h"
#include "dev_rows.h"
#include "grouped.h"
#include "launch.h"
#include "moe_norm.h"
#include "prefill.h"

namespace moert {

constexpr int kPfWaves = 8;           // waves per workgroup of the row kernels
constexpr int kPfNT = kPfWaves * 64;
constexpr int kPfGroup = 8;           // positions staged in LDS at a time (one per wave for the norms)

// The dequantised elements of P rows' chunks, formed once and used for every position: element i of a chunk is
// q_i * d (f32 rows: the value itself), the same rounded product the decode chain forms before each fma.
template <int DT, int K, int P>
struct DeqRows {
  float w[P][Geo<DT, K>::NJ][Fmt<DT>::kElems];
};

template <int DT, int K, int P>
__device__ __forceinline__ void deq_rows(const Rows<DT, K, P>& r, DeqRows<DT, K, P>& w) {
  using G = Geo<DT, K>;
#pragma unroll
  for (int p = 0; p < P; p++)
#pragma unroll
    for (int jj = 0; jj < G::NJ; jj++)
#pragma unroll
      for (int i = 0; i < Fmt<DT>::kElems; i++) w.w[p][jj][i] = chunk_elem<DT>(r.c[p][jj], i);
}

// rows_fma over dequantised rows: per row, the lane's fma chain over its chunks' elements in index order, then the
// tree over the row's lanes (the decode kernels' dot, fma_chunk + group_sum, bit for bit).
template <int DT, int K, int P>
__device__ __forceinline__ void deq_fma(const DeqRows<DT, K, P>& w, const bool (&ok)[P], const XReg<DT, K>& xr,
                                        int sub, float (&out)[P]) {
  using G = Geo<DT, K>;
#pragma unroll
  for (int p = 0; p < P; p++) {
    float acc = 0.0f;
#pragma unroll
    for (int jj = 0; jj < G::NJ; jj++) {
      const int j = sub + G::LPR * jj;
      if (ok[p] && j < G::NCH)
#pragma unroll
        for (int i = 0; i < Fmt<DT>::kElems; i++) acc = __builtin_fmaf(w.w[p][jj][i], xr.v[jj][i], acc);
    }
    out[p] = group_sum<G::LPR>(acc);
  }
}

// LDS layout of a staged activation row. Lane `sub` of a row reads whole weight chunks of x (16 floats for Q8_0,
// 32 for Q4_0), so in a plain layout the lanes' 16-byte reads are 64 or 128 bytes apart and fall in the same banks.
// The float4 slots of chunk j are therefore stored with their index xor-ed by sw(j) (slot q of chunk j at
// NQ j + (q ^ sw(j))), which spreads the 8 or 16 lanes one LDS pass serves over distinct bank groups (32 or 64
// banks). The values and the order they are used in do not change.
template <int DT>
__device__ __forceinline__ int xslot(int s) {
  constexpr int NQ = Fmt<DT>::kElems / 4;  // float4 slots per chunk
  if constexpr (NQ == 1) {
    return s;
  } else {
    const int j = s / NQ, q = s % NQ;
    const int sw = NQ == 4 ? ((j >> 1) ^ (j >> 3)) & 3 : (j ^ (j >> 3)) & 7;
    return NQ * j + (q ^ sw);
  }
}

// load_x over a row staged with xslot.
template <int DT, int K>
__device__ __forceinline__ void load_xs(XReg<DT, K>& xr, const float* x, int sub) {
  using G = Geo<DT, K>;
  constexpr int NQ = G::CE / 4;
  const float4* x4 = reinterpret_cast<const float4*>(x);
#pragma unroll
  for (int jj = 0; jj < G::NJ; jj++) {
    const int j = sub + G::LPR * jj;
    if (j < G::NCH) {
#pragma unroll
      for (int e = 0; e < NQ; e++) {
        const float4 t = x4[xslot<DT>(NQ * j + e)];
        xr.v[jj][4 * e] = t.x;
        xr.v[jj][4 * e + 1] = t.y;
        xr.v[jj][4 * e + 2] = t.z;
        xr.v[jj][4 * e + 3] = t.w;
      }
    }
  }
}

// Canonical rmsnorm scale of the K floats at x (LDS, staged with xslot): the sum of squares over 16-element chunks,
// chunk j in lane j % 64, then the lane tree; r = 1 / sqrt(ss / K + eps). One wave.
template <int DT, int K>
__device__ __forceinline__ float wave_rms(const float* x, float eps, int lane) {
  constexpr int NCH = K / 16;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float acc = 0.0f;
#pragma unroll
  for (int jj = 0; jj < (NCH + 63) / 64; jj++) {
    const int j = lane + 64 * jj;
    if (j < NCH) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float4 t = x4[xslot<DT>(4 * j + e)];
        acc = __builtin_fmaf(t.x, t.x, acc);
        acc = __builtin_fmaf(t.y, t.y, acc);
        acc = __builtin_fmaf(t.z, t.z, acc);
        acc = __builtin_fmaf(t.w, t.w, acc);
      }
    }
  }
  const float ss = group_sum<64>(acc);
  return 1.0f / sqrtf(ss / (float)K + eps);
}

// Stages positions [v0, v0 + n) of x ([*, K] rows, global) into xs ([kPfGroup][K], LDS, layout xslot); with lnw,
// each is then normalised in place: xs = lnw * (x * r) (wave w normalises position w of the group). Ends with a
// barrier.
template <int DT, int K>
__device__ __forceinline__ void stage_group(const float* __restrict__ x, int v0, int n, const float* __restrict__ lnw,
                                            float eps, float (*xs)[K], float* rsv) {
  constexpr int K4 = K / 4;
  const float4* src = reinterpret_cast<const float4*>(x + (size_t)v0 * K);
  for (int i = threadIdx.x; i < n * K4; i += kPfNT)
    reinterpret_cast<float4*>(&xs[i / K4][0])[xslot<DT>(i % K4)] = src[i];
  __syncthreads();
  if (!lnw) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave < n) {
    const float r = wave_rms<DT, K>(&xs[wave][0], eps, lane);
    if (lane == 0) rsv[wave] = r;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n * K4; i += kPfNT) {
    const int v = i / K4, s = i % K4;
    float4* p = reinterpret_cast<float4*>(&xs[v][0]) + xslot<DT>(s);
    const float4 w = reinterpret_cast<const float4*>(lnw)[s];
    const float r = rsv[v];
    float4 t = *p;
    t.x = w.x * (t.x * r);
    t.y = w.y * (t.y * r);
    t.z = w.z * (t.z * r);
    t.w = w.w * (t.w * r);
    *p = t;
  }
  __syncthreads();
}

// ------------------------------------------------------------------------------------------------------------
// rmsnorm -> [q; k; v] -> RoPE -> q / KV cache, for positions pos0 .. pos0 + nv - 1 (k_qkv's arithmetic per
// position). A wave owns NP row pairs (j, j + 32) of a head, as in k_qkv.
template <int DT, int K, int NP>
__global__ __launch_bounds__(kPfNT) void k_qkv_b(DMat m, const float* __restrict__ h, const float* __restrict__ lnw,
                                                 float eps, int pos0, int nv, const float* __restrict__ rope,
                                                 int heads, int kvh, int max_len, float* __restrict__ q,
                                                 uint16_t* __restrict__ kc, uint16_t* __restrict__ vc) {
  using G = Geo<DT, K>;
  constexpr int P = 2 * NP;
  __shared__ __align__(16) float xs[kPfGroup][K];
  __shared__ float csv[kPfGroup][64];
  __shared__ float rsv[kPfGroup];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPR, rw = lane / G::LPR;
  const int npairs = m.rows / 2;
  const int wbase = (blockIdx.x * kPfWaves + wave) * (NP * G::RPW);
  size_t row[P];
  bool ok[P];
  int gp[NP];
#pragma unroll
  for (int a = 0; a < NP; a++) {
    gp[a] = wbase + a * G::RPW + rw;
    const bool v = gp[a] < npairs;
    const int head = gp[a] / 32, jp = gp[a] % 32;
    row[2 * a] = (size_t)head * 64 + jp;
    row[2 * a + 1] = row[2 * a] + 32;
    ok[2 * a] = ok[2 * a + 1] = v;
  }
  Rows<DT, K, P> rr;
  rows_load<DT, K, P>(rr, m, row, ok, sub);
  DeqRows<DT, K, P> dw;
  deq_rows<DT, K, P>(rr, dw);
  const int qd = heads * 64;
  for (int v0 = 0; v0 < nv; v0 += kPfGroup) {
    const int n = min(kPfGroup, nv - v0);
    __syncthreads();  // the previous group's activations are no longer read
    for (int i = threadIdx.x; i < n * 64; i += kPfNT) csv[i / 64][i % 64] = rope[(size_t)(pos0 + v0 + i / 64) * 64 + i % 64];
    stage_group<DT, K>(h, v0, n, lnw, eps, xs, rsv);
    for (int v = 0; v < n; v++) {
      XReg<DT, K> xr;
      load_xs<DT, K>(xr, &xs[v][0], sub);
      float out[P];
      deq_fma<DT, K, P>(dw, ok, xr, sub, out);
      if (sub != 0) continue;
      const int pos = pos0 + v0 + v;
#pragma unroll
      for (int a = 0; a < NP; a++) {
        if (!ok[2 * a]) continue;
        const int head = gp[a] / 32, jp = gp[a] % 32;
        const float x1 = out[2 * a], x2 = out[2 * a + 1];
        const float c = csv[v][jp], sn = csv[v][32 + jp];
        if (head < heads) {
          float* qv = q + (size_t)(v0 + v) * qd;
          qv[head * 64 + jp] = x1 * c - x2 * sn;
          qv[head * 64 + jp + 32] = x2 * c + x1 * sn;
        } else if (head < heads + kvh) {
          uint16_t* kp = kc + ((size_t)(head - heads) * max_len + pos) * 64;
          kp[jp] = f2h(x1 * c - x2 * sn);
          kp[jp + 32] = f2h(x2 * c + x1 * sn);
        } else {
          uint16_t* vp = vc + ((size_t)(head - heads - kvh) * max_len + pos) * 64;
          vp[jp] = f2h(x1);
          vp[jp + 32] = f2h(x2);
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------------------
// h[v][r] = h[v][r] + res * (Wo att[v])[r] for every position v (k_oproj's arithmetic per position), then the
// MoE-norm partials of each position's new rows into zp + v * kNormItems (k_oproj's epilogue per position).
template <int DT, int K, int P>
__global__ __launch_bounds__(kPfNT) void k_oproj_b(DMat m, const float* __restrict__ att, int nv, float res,
                                                   float* __restrict__ h, DMat router, const float* __restrict__ lnw,
                                                   float* __restrict__ zp) {
  using G = Geo<DT, K>;
  constexpr int RB = kPfWaves * P * G::RPW;  // rows of the workgroup: [r0, r0 + RB)
  static_assert(RB % kNormBlk == 0, "the workgroup's rows must be whole partial blocks");
  __shared__ __align__(16) float xs[kPfGroup][K];
  __shared__ float hn[kPfGroup][RB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPR, rw = lane / G::LPR;
  const int r0 = blockIdx.x * RB;
  const size_t base = ((size_t)blockIdx.x * kPfWaves + wave) * (P * G::RPW);
  size_t row[P];
  bool ok[P];
#pragma unroll
  for (int p = 0; p < P; p++) {
    row[p] = base + (size_t)p * G::RPW + rw;
    ok[p] = row[p] < (size_t)m.rows;
  }
  Rows<DT, K, P> rr;
  rows_load<DT, K, P>(rr, m, row, ok, sub);
  __builtin_amdgcn_sched_barrier(0);
  NormPart<RB, kPfNT> np;
  norm_part_fetch<DT, RB, kPfNT>(router, lnw, r0, m.rows, np);
  DeqRows<DT, K, P> dw;
  deq_rows<DT, K, P>(rr, dw);
  const int H = m.rows;
  for (int v0 = 0; v0 < nv; v0 += kPfGroup) {
    const int n = min(kPfGroup, nv - v0);
    __syncthreads();
    stage_group<DT, K>(att, v0, n, nullptr, 0.0f, xs, nullptr);
    for (int v = 0; v < n; v++) {
      XReg<DT, K> xr;
      load_xs<DT, K>(xr, &xs[v][0], sub);
      float out[P];
      deq_fma<DT, K, P>(dw, ok, xr, sub, out);
      if (sub != 0) continue;
      float* hv = h + (size_t)(v0 + v) * H;
#pragma unroll
      for (int p = 0; p < P; p++)
        if (ok[p]) {
          const float hold = hv[row[p]];
          const float hnew = hold + res * out[p];
          hv[row[p]] = hnew;
          hn[v][row[p] - r0] = hnew;
        }
    }
    __syncthreads();
    for (int v = 0; v < n; v++)
      norm_part_finish<DT, RB, kPfNT>(np, &hn[v][0], router.rows, r0, H, zp + (size_t)(v0 + v) * kNormItems);
  }
}

// ------------------------------------------------------------------------------------------------------------
// Router of position v = blockIdx.x: xn = rmsnorm(h[v]) (kept in xn[v] for the experts), logits = Wr xn (+ bias),
// ranks, ids and weights in top-k order (k_route_up's router, arithmetic for arithmetic).
// 16 waves, 8 for f32 rows (whose registers would not fit 16), as k_route_up
__host__ __device__ constexpr int route_b_waves(int dt) { return dt == DT_F32 ? 8 : 16; }

template <int DT, int K>
__global__ __launch_bounds__(route_b_waves(DT) * 64) void k_route_b(DMat router, const float* __restrict__ bias,
                                                               const float* __restrict__ h,
                                                               const float* __restrict__ lnw, float eps,
                                                               const float* __restrict__ zp, int k,
                                                               float* __restrict__ xn, int* __restrict__ ids,
                                                               float* __restrict__ wts) {
  constexpr int NW = route_b_waves(DT), NT = NW * 64;
  constexpr int IPW = (64 + NW - 1) / NW;  // router items per wave
  constexpr int XP = (K + NT - 1) / NT;    // elements of h per thread
  __shared__ __align__(16) float lg[64];
  __shared__ int part[NW][64];
  const int v = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int E = router.rows, nb = K / kNormBlk;
  zp += (size_t)v * kNormItems;
  NormItem ssi, it[IPW];
  float bv[IPW], hv[XP], wv[XP];
  norm_item_fetch(zp, E, lane, ssi);
#pragma unroll
  for (int i = 0; i < IPW; i++) {
    const int e = wave + i * NW, ec = e < E ? e : 0;
    norm_item_fetch(zp, ec, lane, it[i]);
    bv[i] = bias ? bias[ec] : 0.0f;
  }
#pragma unroll
  for (int e = 0; e < XP; e++) {
    const int i = threadIdx.x + e * NT, ic = i < K ? i : 0;
    hv[e] = h[(size_t)v * K + ic];
    wv[e] = lnw[ic];
  }
  const float ss = norm_item_sum(ssi, nb, lane);
  const float r = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
  for (int i = 0; i < IPW; i++) {
    const int e = wave + i * NW;
    if (e < E) {
      const float z = norm_item_sum(it[i], nb, lane);
      if (lane == 0) lg[e] = bias ? z * r + bv[i] : z * r;
    }
  }
#pragma unroll
  for (int e = 0; e < XP; e++) {
    const int i = threadIdx.x + e * NT;
    if (i < K) xn[(size_t)v * K + i] = wv[e] * (hv[e] * r);
  }
  __syncthreads();
  int eid[8];
  const int rank = wg_rank<NW>(lg, E, lane, wave, part);
  const bool sel = lane < E && rank < k;
  ids_by_rank(sel, rank, k, eid);
  if (wave == 0) route_weights(lg, sel, rank, k, lane, eid, ids + (size_t)v * k, wts + (size_t)v * k);
}

// ------------------------------------------------------------------------------------------------------------
// The experts routed by the nv positions, in LDS: the u-th expert of the step is the u-th set bit of the used mask
// (ascending expert index; the order of the experts does not enter any sum, each position's combine runs in its
// own top-k order). For expert e: the positions routed to it (bit mask) and, per position, the top-k rank of e.
struct PfPlan {
  unsigned bits[64];          // positions routed to expert e
  unsigned long long used;    // experts routed by any position
  signed char rank[64][kPfMaxPos];  // top-k rank of expert e at position v
};

__device__ __forceinline__ void pf_plan(const int* __restrict__ ids, int nv, int k, PfPlan& pl) {
  const int t = threadIdx.x, n = nv * k;
  if (t < 64) pl.bits[t] = 0u;
  __syncthreads();
  int e = 0;
  if (t < n) {
    e = ids[t];
    atomicOr(&pl.bits[e], 1u << (t / k));
    pl.rank[e][t / k] = (signed char)(t % k);
  }
  __syncthreads();
  if (t < 64) {
    const unsigned long long b = __ballot(pl.bits[t] != 0u);
    if (t == 0) pl.used = b;
  }
  __syncthreads();
}

__device__ __forceinline__ int nth_bit64(unsigned long long b, int u) {
  for (int i = 0; i < u; i++) b &= b - 1ull;
  return b ? __ffsll((long long)b) - 1 : -1;
}

// Gate/up of the u-th routed expert (u = blockIdx.y) for the positions routed to it: rows (r, I + r) of the
// expert for the workgroup's pairs, act[v][j][r] = silu(gate_r . xn[v]) * (up_r . xn[v]) with j the expert's
// rank at v (k_route_up's expert arithmetic per position).
template <int DT, int K, int NP>
__global__ __launch_bounds__(kPfNT) void k_moe_up_b(DMat gu, const float* __restrict__ xn, const int* __restrict__ ids,
                                                    int nv, int k, int inter, float* __restrict__ act) {
  using G = Geo<DT, K>;
  constexpr int P = 2 * NP;
  __shared__ PfPlan pl;
  __shared__ __align__(16) float xs[kPfGroup][K];
  pf_plan(ids, nv, k, pl);
  const int e = nth_bit64(pl.used, blockIdx.y);
  if (e < 0) return;
  const unsigned members = pl.bits[e];
  const int ne = __popc(members);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPR, rw = lane / G::LPR;
  const int wbase = (blockIdx.x * kPfWaves + wave) * (NP * G::RPW);
  size_t row[P];
  bool ok[P];
  int rr_[NP];
#pragma unroll
  for (int a = 0; a < NP; a++) {
    rr_[a] = wbase + a * G::RPW + rw;
    const bool v = rr_[a] < inter;
    row[2 * a] = (size_t)e * 2 * inter + (v ? rr_[a] : 0);
    row[2 * a + 1] = row[2 * a] + inter;
    ok[2 * a] = ok[2 * a + 1] = v;
  }
  Rows<DT, K, P> rr;
  rows_load<DT, K, P>(rr, gu, row, ok, sub);
  DeqRows<DT, K, P> dw;
  deq_rows<DT, K, P>(rr, dw);
  for (int c0 = 0; c0 < ne; c0 += kPfGroup) {
    const int n = min(kPfGroup, ne - c0);
    __syncthreads();
    // members c0 .. c0 + n - 1 (the set bits of `members` in ascending position order) into LDS
    for (int i = threadIdx.x; i < n * K / 4; i += kPfNT) {
      const int c = i / (K / 4), w4 = i % (K / 4);
      const int vpos = nth_bit64(members, c0 + c);
      reinterpret_cast<float4*>(&xs[c][0])[xslot<DT>(w4)] = reinterpret_cast<const float4*>(xn + (size_t)vpos * K)[w4];
    }
    __syncthreads();
    for (int c = 0; c < n; c++) {
      XReg<DT, K> xr;
      load_xs<DT, K>(xr, &xs[c][0], sub);
      float out[P];
      deq_fma<DT, K, P>(dw, ok, xr, sub, out);
      if (sub != 0) continue;
      const int vpos = nth_bit64(members, c0 + c);
      float* av = act + ((size_t)vpos * k + pl.rank[e][vpos]) * inter;
#pragma unroll
      for (int a = 0; a < NP; a++)
        if (ok[2 * a]) av[rr_[a]] = silu_mul(out[2 * a], out[2 * a + 1]);
    }
  }
}

// Down rows of the u-th routed expert for the positions routed to it: o[v][j][r] = down_r . act[v][j]
// (k_expert_down's per-expert dot).
template <int DT, int K, int P>
__global__ __launch_bounds__(kPfNT) void k_moe_down_b(DMat dn, const float* __restrict__ act,
                                                      const int* __restrict__ ids, int nv, int k, int hidden,
                                                      float* __restrict__ o) {
  using G = Geo<DT, K>;
  __shared__ PfPlan pl;
  __shared__ __align__(16) float xs[kPfMaxPos][K];
  pf_plan(ids, nv, k, pl);
  const int e = nth_bit64(pl.used, blockIdx.y);
  if (e < 0) return;
  const unsigned members = pl.bits[e];
  const int ne = __popc(members);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPR, rw = lane / G::LPR;
  const size_t base = ((size_t)blockIdx.x * kPfWaves + wave) * (P * G::RPW);
  size_t row[P];
  bool ok[P];
#pragma unroll
  for (int p = 0; p < P; p++) {
    const size_t r = base + (size_t)p * G::RPW + rw;
    ok[p] = r < (size_t)hidden;
    row[p] = (size_t)e * hidden + (ok[p] ? r : 0);
  }
  Rows<DT, K, P> rr;
  rows_load<DT, K, P>(rr, dn, row, ok, sub);
  DeqRows<DT, K, P> dw;
  deq_rows<DT, K, P>(rr, dw);
  // every member's activation (K = I floats each) into LDS
  for (int i = threadIdx.x; i < ne * K / 4; i += kPfNT) {
    const int c = i / (K / 4), w4 = i % (K / 4);
    const int vpos = nth_bit64(members, c);
    reinterpret_cast<float4*>(&xs[c][0])[xslot<DT>(w4)] =
        reinterpret_cast<const float4*>(act + ((size_t)vpos * k + pl.rank[e][vpos]) * K)[w4];
  }
  __syncthreads();
  for (int c = 0; c < ne; c++) {
    XReg<DT, K> xr;
    load_xs<DT, K>(xr, &xs[c][0], sub);
    float out[P];
    deq_fma<DT, K, P>(dw, ok, xr, sub, out);
    if (sub != 0) continue;
    const int vpos = nth_bit64(members, c);
    float* ov = o + ((size_t)vpos * k + pl.rank[e][vpos]) * hidden;
#pragma unroll
    for (int p = 0; p < P; p++)
      if (ok[p]) ov[base + (size_t)p * G::RPW + rw] = out[p];
  }
}

// h[v][r] = h[v][r] + res * y, y = sum over j = 0 .. k-1 in order of w[v][j] * o[v][j][r] (k_expert_down's combine).
__global__ __launch_bounds__(256) void k_moe_comb_b(const float* __restrict__ o, const float* __restrict__ wts, int k,
                                                    int hidden, float res, float* __restrict__ h) {
  const int v = blockIdx.y, r = blockIdx.x * 256 + threadIdx.x;
  if (r >= hidden) return;
  float y = 0.0f;
  for (int j = 0; j < k; j++) y = y + wts[v * k + j] * o[((size_t)v * k + j) * hidden + r];
  float* hv = h + (size_t)v * hidden;
  const float hold = hv[r];
  hv[r] = hold + res * y;
}

// Embedding rows of the nv tokens (k_embed per position).
template <int DT>
__global__ __launch_bounds__(256) void k_embed_b(DMat e, const int* __restrict__ toks, float mult,
                                                 float* __restrict__ h) {
  const int v = blockIdx.y, tok = toks[v];
  const int H = e.cols;
  float* hv = h + (size_t)v * H;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < H; i += gridDim.x * 256) {
    float x;
    if (DT == DT_Q8_0) {
      x = (float)(int8_t)e.q[(size_t)tok * H + i] * h2f(e.d[(size_t)tok * (H / 32) + i / 32]);
    } else if (DT == DT_Q4_0) {
      const int b = i / 32, w = i % 32;
      const uint8_t byte = e.q[(size_t)tok * (H / 2) + b * 16 + (w & 15)];
      x = (float)((int)(w < 16 ? (byte & 15) : (byte >> 4)) - 8) * h2f(e.d[(size_t)tok * (H / 32) + b]);
    } else {
      x = reinterpret_cast<const float*>(e.q)[(size_t)tok * H + i];
    }
    hv[i] = x * mult;
  }
}

// ------------------------------------------------------------------------------------------------------------
// Launchers.
static inline int cdiv(long a, long b) { return (int)((a + b - 1) / b); }
constexpr int kPfQkvNP = 1;    // row pairs per wave of k_qkv_b
constexpr int kPfOprojP = 1;   // rows per wave of k_oproj_b
constexpr int kPfUpNP = 1;     // row pairs per wave of k_moe_up_b
constexpr int kPfDownP = 1;    // rows per wave of k_moe_down_b

hipError_t launch_embed_b(hipStream_t s, const DMat& emb, const Dims& d, const PfBufs& p, int nv) {
  const dim3 grid((d.hidden + 255) / 256, nv);
  switch (emb.dtype) {
    case DT_Q8_0: klaunch(k_embed_b<DT_Q8_0>, grid, 256, 0, s, emb, p.toks, d.emb_mult, p.h); break;
    case DT_Q4_0: klaunch(k_embed_b<DT_Q4_0>, grid, 256, 0, s, emb, p.toks, d.emb_mult, p.h); break;
    case DT_F32: klaunch(k_embed_b<DT_F32>, grid, 256, 0, s, emb, p.toks, d.emb_mult, p.h); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_layer_b(hipStream_t s, const LayerDev& L, const Dims& d, const PfBufs& p, const int* lenp, int pos0,
                          int nv, const float* rope) {
  if (nv < 1 || nv > kPfMaxPos || d.top_k > 8 || d.experts > 64 || d.head_dim != 64) return hipErrorInvalidValue;
#define BODY(KK)                                                                                         \
  case KK: {                                                                                             \
    constexpr int PB = kPfWaves * kPfQkvNP * Geo<DTC, KK>::RPW;                                          \
    klaunch(k_qkv_b<DTC, KK, kPfQkvNP>, cdiv(L.qkv.rows / 2, PB), kPfNT, 0, s, L.qkv, p.h, L.ln_attn, d.eps, \
            pos0, nv, rope, d.heads, d.kv_heads, d.max_len, p.q, L.k_cache, L.v_cache);                  \
  } break;
  MOERT_DISPATCH(L.qkv.dtype, L.qkv.cols, BODY)
#undef BODY
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // position v attends to pos0 + v + 1 positions: *lenp = pos0 on the device, len_add = 1
  if ((e = launch_attn_batched(s, L, d, lenp, 1, nv, p.q, p.part, p.att)) != hipSuccess) return e;
#define BODY(KK)                                                                                         \
  case KK: {                                                                                             \
    constexpr int RB = kPfWaves * kPfOprojP * Geo<DTC, KK>::RPW;                                         \
    klaunch(k_oproj_b<DTC, KK, kPfOprojP>, cdiv(L.o.rows, RB), kPfNT, 0, s, L.o, p.att, nv, d.res_mult, p.h, \
            L.router, L.ln_moe, p.zpart);                                                                \
  } break;
  MOERT_DISPATCH(L.o.dtype, L.o.cols, BODY)
#undef BODY
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (L.router.dtype != L.gate_up.dtype || L.router.cols != L.gate_up.cols) return hipErrorInvalidValue;
#define BODY(KK)                                                                                         \
  case KK: {                                                                                             \
    klaunch(k_route_b<DTC, KK>, nv, route_b_waves(DTC) * 64, 0, s, L.router, L.router_bias, p.h, L.ln_moe, d.eps, \
            p.zpart, d.top_k, p.xn, p.ids, p.w);                                                         \
  } break;
  MOERT_DISPATCH(L.router.dtype, L.router.cols, BODY)
#undef BODY
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int U = std::min(nv * d.top_k, d.experts);
#define BODY(KK)                                                                                         \
  case KK: {                                                                                             \
    constexpr int PB = kPfWaves * kPfUpNP * Geo<DTC, KK>::RPW;                                           \
    klaunch(k_moe_up_b<DTC, KK, kPfUpNP>, dim3(cdiv(d.inter, PB), U), kPfNT, 0, s, L.gate_up, p.xn, p.ids, nv, \
            d.top_k, d.inter, p.act);                                                                    \
  } break;
  MOERT_DISPATCH(L.gate_up.dtype, L.gate_up.cols, BODY)
#undef BODY
  if ((e = hipGetLastError()) != hipSuccess) return e;
#define BODY(KK)                                                                                         \
  case KK: {                                                                                             \
    constexpr int RB = kPfWaves * kPfDownP * Geo<DTC, KK>::RPW;                                          \
    klaunch(k_moe_down_b<DTC, KK, kPfDownP>, dim3(cdiv(d.hidden, RB), U), kPfNT, 0, s, L.down, p.act, p.ids, nv, \
            d.top_k, d.hidden, p.o);                                                                     \
  } break;
  switch (L.down.dtype) {
    case DT_Q8_0: {
      constexpr int DTC = DT_Q8_0;
      switch (L.down.cols) { MOERT_KDOWN_CASES(BODY) default: return hipErrorInvalidValue; }
    } break;
    case DT_Q4_0: {
      constexpr int DTC = DT_Q4_0;
      switch (L.down.cols) { MOERT_KDOWN_CASES(BODY) default: return hipErrorInvalidValue; }
    } break;
    case DT_F32: {
      constexpr int DTC = DT_F32;
      switch (L.down.cols) { MOERT_KDOWN_CASES(BODY) default: return hipErrorInvalidValue; }
    } break;
    default: return hipErrorInvalidValue;
  }
#undef BODY
  if ((e = hipGetLastError()) != hipSuccess) return e;
  klaunch(k_moe_comb_b, dim3((d.hidden + 255) / 256, nv), 256, 0, s, p.o, p.w, d.top_k, d.hidden, d.res_mult, p.h);
  return hipGetLastError();
}

hipError_t launch_layer_grouped(hipStream_t s, const LayerDev& L, const Dims& d, const PfBufs& p, const int* lenp,
                                int pos0, int nv, const float* rope, const GroupBufs& g, const float* next_lnw) {
  if (nv < 1 || nv > kPfMaxPos || d.top_k > 8 || d.experts > 64 || d.head_dim != 64) return hipErrorInvalidValue;
  GroupBufs gg = g;
  gg.ids = p.ids;
  gg.w = p.w;
  hipError_t e;
  if ((e = launch_gd_qkv(s, d, nv, pos0, rope, p.q, L.k_cache, L.v_cache, gg)) != hipSuccess) return e;
  // position v attends to pos0 + v + 1 positions: *lenp = pos0 on the device, len_add = 1
  if ((e = launch_attn_batched(s, L, d, lenp, 1, nv, p.q, p.part, p.att)) != hipSuccess) return e;
  if ((e = launch_grp_codes(s, d.heads * 64, nv, p.att, gg)) != hipSuccess) return e;
  if ((e = launch_gd_oproj(s, nv, d.res_mult, p.h, gg)) != hipSuccess) return e;
  if ((e = launch_grp_route_norm(s, L, nv, d.top_k, p.h, L.ln_moe, d.eps, gg)) != hipSuccess) return e;
  if ((e = launch_grp_experts(s, d.hidden, d.experts, nv, d.top_k, d.inter, gg)) != hipSuccess) return e;
  return launch_gd_combine(s, d.hidden, nv, d.top_k, d.res_mult, p.h, next_lnw, d.eps, gg);
}

}  // namespace moert

// Decode-step kernels for gfx950 (wave64). The evaluation order of every reduction is the one stated in
// dev_math.h; the reference kernels these replace are cited on each kernel (paths relative to the reference
// root, rust/moe-rt/src).
#include <climits>

#include "kernels.h"

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

// P rows per lane group: all chunk loads are issued before any arithmetic. out[p] ends up in every lane of the
// group that computed row[p].
template <int DT, int K, int P>
__device__ __forceinline__ void rows_dot(const DMat& m, const size_t (&row)[P], const bool (&ok)[P],
                                         const XReg<DT, K>& xr, int sub, float (&out)[P]) {
  using G = Geo<DT, K>;
  RawChunk c[P][G::NJ];
#pragma unroll
  for (int p = 0; p < P; p++)
#pragma unroll
    for (int jj = 0; jj < G::NJ; jj++) {
      int j = sub + G::LPR * jj;
      if (ok[p] && j < G::NCH) c[p][jj] = load_chunk<DT>(m, row[p], j);
    }
#pragma unroll
  for (int p = 0; p < P; p++) {
    float acc = 0.0f;
#pragma unroll
    for (int jj = 0; jj < G::NJ; jj++) {
      int j = sub + G::LPR * jj;
      if (ok[p] && j < G::NCH) acc = fma_chunk<DT>(c[p][jj], xr.v[jj], acc);
    }
    out[p] = group_sum<G::LPR>(acc);
  }
}

// ------------------------------------------------------------------------------------------------------------
// Plain GEMV y = W x (gpu.rs:21-38).
template <int DT, int K, int P>
__global__ __launch_bounds__(kBlock) void k_gemv(DMat m, const float* __restrict__ x, float* __restrict__ y) {
  using G = Geo<DT, K>;
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  XReg<DT, K> xr;
  load_x<DT, K>(xr, x, sub);
  size_t base = ((size_t)blockIdx.x * kWavesPerBlock + wave) * (P * G::RPW);
  size_t row[P];
  bool ok[P];
#pragma unroll
  for (int p = 0; p < P; p++) {
    row[p] = base + (size_t)p * G::RPW + rw;
    ok[p] = row[p] < (size_t)m.rows;
  }
  float out[P];
  rows_dot<DT, K, P>(m, row, ok, xr, sub, out);
#pragma unroll
  for (int p = 0; p < P; p++)
    if (ok[p] && sub == 0) y[row[p]] = out[p];
}

// ------------------------------------------------------------------------------------------------------------
// Embedding row times embedding_multiplier (model.rs:134-138); the token is seq[pos] on the device.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_embed(DMat e, const int* __restrict__ seq, const int* __restrict__ st,
                                                  float mult, float* __restrict__ h) {
  int tok = seq[st[ST_POS]];
  int H = e.cols;
  for (int i = threadIdx.x; i < H; i += kBlock) {
    float v;
    if (DT == DT_Q8_0) {
      v = (float)(int8_t)e.q[(size_t)tok * H + i] * h2f(e.d[(size_t)tok * (H / 32) + i / 32]);
    } else if (DT == DT_Q4_0) {
      int b = i / 32, w = i % 32;
      uint8_t byte = e.q[(size_t)tok * (H / 2) + b * 16 + (w & 15)];
      v = (float)((int)(w < 16 ? (byte & 15) : (byte >> 4)) - 8) * h2f(e.d[(size_t)tok * (H / 32) + b]);
    } else {
      v = reinterpret_cast<const float*>(e.q)[(size_t)tok * H + i];
    }
    h[i] = v * mult;
  }
}

// ------------------------------------------------------------------------------------------------------------
// Attention block input: rmsnorm -> [q; k; v] GEMV -> rotate_half RoPE of q and k -> q to `q` (f32), k and v to
// row `pos` of the fp16 KV cache. Replaces rmsnorm + gemv q/k/v + rope + the two KV copies
// (gpu_model.rs:341-378) and rope_kv / gemv_row (gpu.rs:151-197). A wave owns NP*RPW row pairs (j, j+32) of
// a head, so both halves of a rotation meet in the same lanes.
template <int DT, int K, int NP>
__global__ __launch_bounds__(kBlock) void k_qkv(DMat m, const float* __restrict__ h, const float* __restrict__ lnw,
                                                float eps, const int* __restrict__ st, const float* __restrict__ rope,
                                                int heads, int kvh, int max_len, float* __restrict__ q,
                                                uint16_t* __restrict__ kc, uint16_t* __restrict__ vc) {
  using G = Geo<DT, K>;
  constexpr int P = 2 * NP;
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  float r = rms_scale<K>(h, eps, lane);
  XReg<DT, K> xr;
  load_xn<DT, K>(xr, h, lnw, r, sub);
  int pos = st[ST_POS];
  int npairs = m.rows / 2;
  int wbase = (blockIdx.x * kWavesPerBlock + wave) * (NP * G::RPW);
  size_t row[P];
  bool ok[P];
  int gp[NP];
#pragma unroll
  for (int a = 0; a < NP; a++) {
    gp[a] = wbase + a * G::RPW + rw;
    bool v = gp[a] < npairs;
    int head = gp[a] / 32, jp = gp[a] % 32;
    row[2 * a] = (size_t)head * 64 + jp;
    row[2 * a + 1] = row[2 * a] + 32;
    ok[2 * a] = v;
    ok[2 * a + 1] = v;
  }
  float out[P];
  rows_dot<DT, K, P>(m, row, ok, xr, sub, out);
  if (sub != 0) return;
  const float* cs = rope + (size_t)pos * 64;
#pragma unroll
  for (int a = 0; a < NP; a++) {
    if (!ok[2 * a]) continue;
    int head = gp[a] / 32, jp = gp[a] % 32;
    float x1 = out[2 * a], x2 = out[2 * a + 1];
    float c = cs[jp], s = cs[32 + jp];
    if (head < heads) {
      q[head * 64 + jp] = x1 * c - x2 * s;
      q[head * 64 + jp + 32] = x2 * c + x1 * s;
    } else if (head < heads + kvh) {
      uint16_t* kp = kc + ((size_t)(head - heads) * max_len + pos) * 64;
      kp[jp] = f2h(x1 * c - x2 * s);
      kp[jp + 32] = f2h(x2 * c + x1 * s);
    } else {
      uint16_t* vp = vc + ((size_t)(head - heads - kvh) * max_len + pos) * 64;
      vp[jp] = f2h(x1);
      vp[jp + 32] = f2h(x2);
    }
  }
}

// ------------------------------------------------------------------------------------------------------------
// Split-KV GQA decode attention over the fp16 cache (attn_split + attn_combine, gpu.rs:205-292). Block (g, s)
// serves the G query heads of KV head g against its share of the ceil(len/64) tiles; K is staged transposed and V
// row-major in LDS as f32 and read by the G waves. The last block of a KV head to finish (arrival counter)
// combines the partials of the used blocks in split order, so no second launch is needed.
__global__ __launch_bounds__(kBlock) void k_attn(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                 const uint16_t* __restrict__ vc, const int* __restrict__ lenp,
                                                 int len_add, int heads, int kvh, int max_len, float scale,
                                                 int splits, float* __restrict__ part, int* __restrict__ cnt,
                                                 float* __restrict__ out) {
  __shared__ float KT[64][65];
  __shared__ float Vs[64][64];
  __shared__ float Qs[kWavesPerBlock][64];
  __shared__ float Ps[kWavesPerBlock][64];
  __shared__ int last;
  int g = blockIdx.x / splits, s = blockIdx.x % splits;
  int G = heads / kvh;
  int len = *lenp + len_add;
  int nb = (len + 63) / 64, per = (nb + splits - 1) / splits, used = (nb + per - 1) / per;
  if (s >= used) return;
  int t0 = s * per, t1 = min(t0 + per, nb);
  int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  bool active = w < G;
  int h = g * G + w;
  if (active) Qs[w][lane] = q[h * 64 + lane];
  const uint16_t* K = kc + (size_t)g * max_len * 64;
  const uint16_t* V = vc + (size_t)g * max_len * 64;
  const float NEG_INF = __int_as_float(0xff800000);
  float m = NEG_INF, l = 0.0f, acc = 0.0f, alpha = 0.0f, mn = NEG_INF;
  for (int t = t0; t < t1; t++) {
    __syncthreads();
    for (int sg = tid; sg < 512; sg += kBlock) {
      int i = sg >> 3, c0 = (sg & 7) * 8;
      uint4 kv = *reinterpret_cast<const uint4*>(K + (size_t)(t * 64 + i) * 64 + c0);
      uint4 vv = *reinterpret_cast<const uint4*>(V + (size_t)(t * 64 + i) * 64 + c0);
      const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
      const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        KT[c0 + e][i] = h2f((uint16_t)(kw[e >> 1] >> (16 * (e & 1))));
        Vs[i][c0 + e] = h2f((uint16_t)(vw[e >> 1] >> (16 * (e & 1))));
      }
    }
    __syncthreads();
    int nv = min(64, len - t * 64);
    if (active) {
      float sc = NEG_INF;
      if (lane < nv) {
        float dt = 0.0f;
#pragma unroll 16
        for (int c = 0; c < 64; c++) dt = __builtin_fmaf(Qs[w][c], KT[c][lane], dt);
        sc = dt * scale;
      }
      float tmax = group_max<64>(sc);
      mn = m > tmax ? m : tmax;
      alpha = dexp(m - mn);
      float p = dexp(sc - mn);
      float ts = group_sum<64>(p);
      l = __builtin_fmaf(l, alpha, ts);
      Ps[w][lane] = p;
    }
    __syncthreads();
    if (active) {
      float pv = 0.0f;
      for (int i = 0; i < nv; i++) pv = __builtin_fmaf(Ps[w][i], Vs[i][lane], pv);
      acc = __builtin_fmaf(acc, alpha, pv);
      m = mn;
    }
  }
  if (active) {
    float* pp = part + ((size_t)h * splits + s) * 66;
    if (lane == 0) {
      pp[0] = m;
      pp[1] = l;
    }
    pp[2 + lane] = acc;
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) last = (atomicAdd(&cnt[g], 1) == used - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (active) {
    const float* base = part + (size_t)h * splits * 66;
    float M = NEG_INF;
    for (int s2 = 0; s2 < used; s2++) {
      float ms = __uint_as_float(__hip_atomic_load(reinterpret_cast<const unsigned*>(base + (size_t)s2 * 66),
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      M = ms > M ? ms : M;
    }
    float den = 0.0f, num = 0.0f;
    for (int s2 = 0; s2 < used; s2++) {
      const unsigned* pp = reinterpret_cast<const unsigned*>(base + (size_t)s2 * 66);
      float ms = __uint_as_float(__hip_atomic_load(pp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      float ls = __uint_as_float(__hip_atomic_load(pp + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      float as = __uint_as_float(__hip_atomic_load(pp + 2 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      float wgt = dexp(ms - M);
      den = __builtin_fmaf(wgt, ls, den);
      num = __builtin_fmaf(wgt, as, num);
    }
    out[h * 64 + lane] = num / den;
  }
  if (tid == 0) atomicExch(&cnt[g], 0);
}

// ------------------------------------------------------------------------------------------------------------
// Output projection with the residual in the epilogue: h[r] = h[r] + res * (Wo att)[r] (gemv o + axpby,
// gpu_model.rs:386-394; model.rs:224-227).
template <int DT, int K, int P>
__global__ __launch_bounds__(kBlock) void k_oproj(DMat m, const float* __restrict__ att, float res,
                                                  float* __restrict__ h) {
  using G = Geo<DT, K>;
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  XReg<DT, K> xr;
  load_x<DT, K>(xr, att, sub);
  size_t base = ((size_t)blockIdx.x * kWavesPerBlock + wave) * (P * G::RPW);
  size_t row[P];
  bool ok[P];
#pragma unroll
  for (int p = 0; p < P; p++) {
    row[p] = base + (size_t)p * G::RPW + rw;
    ok[p] = row[p] < (size_t)m.rows;
  }
  float out[P];
  rows_dot<DT, K, P>(m, row, ok, xr, sub, out);
#pragma unroll
  for (int p = 0; p < P; p++)
    if (ok[p] && sub == 0) h[row[p]] = h[row[p]] + res * out[p];
}

// ------------------------------------------------------------------------------------------------------------
// Top-k of one wave's logits (lane e holds expert e, e < n <= 64): repeated max of (total-order key, lower index
// first), then w_j = exp(l_j - l_top) / sum with the sum taken left to right (Routing::from_logits,
// block.rs:81-89; route_topk, route.rs:18-75). ids/weights written by lanes j < k.
__device__ __forceinline__ void wave_topk(float lv, int n, int k, int lane, int* ids, float* weights) {
  int key = lane < n ? total_key(lv) : INT_MIN;
  int my_id = -1;
  float my_val = 0.0f;
  for (int j = 0; j < k; j++) {
    int bk = key, bi = lane;
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
      int ok_ = __shfl_xor(bk, s), oi = __shfl_xor(bi, s);
      if (ok_ > bk || (ok_ == bk && oi < bi)) {
        bk = ok_;
        bi = oi;
      }
    }
    float bv = __shfl(lv, bi);
    if (lane == j) {
      my_id = bi;
      my_val = bv;
    }
    if (lane == bi) key = INT_MIN;
  }
  float top = __shfl(my_val, 0);
  float ex = lane < k ? dexp(my_val - top) : 0.0f;
  float sum = 0.0f;
  for (int j = 0; j < k; j++) sum = sum + __shfl(ex, j);
  if (lane < k) {
    ids[lane] = my_id;
    weights[lane] = ex / sum;
  }
}

// Router of one layer, one workgroup of 16 waves: rmsnorm of h (written to xn for the experts), logits = Wr xn
// (+ bias), then top-k and the softmax weights (forward_cpu's router part, block.rs:56-62; gemv + route_topk,
// cuda_backend.rs:804-835). E <= 64.
// With NORM false, h is already the block input (HostLayer::forward_cpu takes a normalised x) and is copied to xn.
template <int DT, int K, bool NORM>
__global__ __launch_bounds__(1024) void k_router(DMat m, const float* __restrict__ bias,
                                                 const float* __restrict__ h, const float* __restrict__ lnw,
                                                 float eps, int k, float* __restrict__ xn, int* __restrict__ ids,
                                                 float* __restrict__ weights) {
  using G = Geo<DT, K>;
  __shared__ float lg[64];
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  XReg<DT, K> xr;
  if (NORM) {
    float r = rms_scale<K>(h, eps, lane);
    load_xn<DT, K>(xr, h, lnw, r, sub);
  } else {
    load_x<DT, K>(xr, h, sub);
  }
  if (wave == 0 && rw == 0) {
#pragma unroll
    for (int jj = 0; jj < G::NJ; jj++) {
      int j = sub + G::LPR * jj;
      if (j < G::NCH)
#pragma unroll
        for (int e = 0; e < G::CE; e++) xn[j * G::CE + e] = xr.v[jj][e];
    }
  }
  int E = m.rows;
  for (int base = 0; base < E; base += 16 * G::RPW) {
    size_t row[1] = {(size_t)(base + wave * G::RPW + rw)};
    bool ok[1] = {row[0] < (size_t)E};
    float out[1];
    rows_dot<DT, K, 1>(m, row, ok, xr, sub, out);
    if (ok[0] && sub == 0) lg[row[0]] = bias ? out[0] + bias[row[0]] : out[0];
  }
  __syncthreads();
  if (wave == 0) wave_topk(lane < E ? lg[lane] : 0.0f, E, k, lane, ids, weights);
}

// ------------------------------------------------------------------------------------------------------------
// Gate/up rows of the k routed experts with SwiGLU: act[j, r] = silu(gate_r . xn) * (up_r . xn) for expert
// ids[j] (gemv_swiglu gpu.rs:46-74, grouped as moe_gate_up hits.rs:67-105; Cpu::experts cpu.rs:116-137).
template <int DT, int K, int NP>
__global__ __launch_bounds__(kBlock) void k_expert_up(DMat m, const float* __restrict__ xn, const int* __restrict__ ids,
                                                      int k, int inter, float* __restrict__ act) {
  using G = Geo<DT, K>;
  constexpr int P = 2 * NP;
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  XReg<DT, K> xr;
  load_x<DT, K>(xr, xn, sub);
  int npairs = k * inter;
  int wbase = (blockIdx.x * kWavesPerBlock + wave) * (NP * G::RPW);
  size_t row[P];
  bool ok[P];
  int gp[NP];
#pragma unroll
  for (int a = 0; a < NP; a++) {
    gp[a] = wbase + a * G::RPW + rw;
    bool v = gp[a] < npairs;
    int j = v ? gp[a] / inter : 0, r = gp[a] % inter;
    size_t e = (size_t)ids[j];
    row[2 * a] = e * 2 * inter + r;
    row[2 * a + 1] = e * 2 * inter + inter + r;
    ok[2 * a] = v;
    ok[2 * a + 1] = v;
  }
  float out[P];
  rows_dot<DT, K, P>(m, row, ok, xr, sub, out);
  if (sub != 0) return;
#pragma unroll
  for (int a = 0; a < NP; a++)
    if (ok[2 * a]) act[gp[a]] = silu_mul(out[2 * a], out[2 * a + 1]);
}

// Down rows of the k routed experts, combined in top-k order, residual in the epilogue:
// h[r] = h[r] + res * sum_j w_j * (down_{ids[j]}[r] . act_j) (gemv_axpby gpu.rs:80-103 / moe_down hits.rs:109-148;
// Cpu::experts cpu.rs:138-148). One output row per wave; expert slot j = pass * RPW + group.
template <int DT, int K>
__global__ __launch_bounds__(kBlock) void k_expert_down(DMat m, const float* __restrict__ act,
                                                        const int* __restrict__ ids, const float* __restrict__ wts,
                                                        int k, int hidden, float res, bool accumulate,
                                                        float* __restrict__ h) {
  using G = Geo<DT, K>;
  constexpr int KMAX = 8;
  constexpr int KP = (KMAX + G::RPW - 1) / G::RPW;
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  int r = blockIdx.x * kWavesPerBlock + wave;
  if (r >= hidden) return;
  XReg<DT, K> xr[KP];
  RawChunk c[KP][G::NJ];
#pragma unroll
  for (int p = 0; p < KP; p++) {
    int j = p * G::RPW + rw;
    if (j < k) {
      size_t row = (size_t)ids[j] * hidden + r;
#pragma unroll
      for (int jj = 0; jj < G::NJ; jj++) {
        int ch = sub + G::LPR * jj;
        if (ch < G::NCH) c[p][jj] = load_chunk<DT>(m, row, ch);
      }
      load_x<DT, K>(xr[p], act + (size_t)j * K, sub);
    }
  }
  float dsum[KP];
#pragma unroll
  for (int p = 0; p < KP; p++) {
    int j = p * G::RPW + rw;
    float acc = 0.0f;
    if (j < k) {
#pragma unroll
      for (int jj = 0; jj < G::NJ; jj++) {
        int ch = sub + G::LPR * jj;
        if (ch < G::NCH) acc = fma_chunk<DT>(c[p][jj], xr[p].v[jj], acc);
      }
    }
    dsum[p] = group_sum<G::LPR>(acc);
  }
  float y = 0.0f;
#pragma unroll
  for (int p = 0; p < KP; p++) {
#pragma unroll
    for (int g2 = 0; g2 < G::RPW; g2++) {
      int j = p * G::RPW + g2;
      float dj = __shfl(dsum[p], g2 * G::LPR);
      if (j < k) y = y + wts[j] * dj;
    }
  }
  if (lane == 0) h[r] = accumulate ? h[r] + res * y : y;
}

// ------------------------------------------------------------------------------------------------------------
// Final rmsnorm, tied LM head, division by logits_scaling, and greedy argmax (last index on ties): each block
// reduces its rows, the last block to arrive reduces the blocks, records the token and advances the position
// (final rmsnorm + gemv, gpu_model.rs:414-439; argmax, bin/m1b-gulosa.rs:22-24).
__device__ __forceinline__ bool later_better(int ak, int ai, int bk, int bi) { return ak > bk || (ak == bk && ai > bi); }

template <int DT, int K, int P>
__global__ __launch_bounds__(kBlock) void k_head(DMat m, const float* __restrict__ h, const float* __restrict__ lnw,
                                                 float eps, float ls, float* __restrict__ logits, int2* __restrict__ best,
                                                 int* __restrict__ cnt, int* __restrict__ st, int* __restrict__ seq,
                                                 int* __restrict__ hist, int max_len) {
  using G = Geo<DT, K>;
  __shared__ int sk[kWavesPerBlock], si[kWavesPerBlock];
  __shared__ int last;
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  float r = rms_scale<K>(h, eps, lane);
  XReg<DT, K> xr;
  load_xn<DT, K>(xr, h, lnw, r, sub);
  size_t base = ((size_t)blockIdx.x * kWavesPerBlock + wave) * (P * G::RPW);
  size_t row[P];
  bool ok[P];
#pragma unroll
  for (int p = 0; p < P; p++) {
    row[p] = base + (size_t)p * G::RPW + rw;
    ok[p] = row[p] < (size_t)m.rows;
  }
  float out[P];
  rows_dot<DT, K, P>(m, row, ok, xr, sub, out);
  int bk = INT_MIN, bi = -1;
#pragma unroll
  for (int p = 0; p < P; p++) {
    if (ok[p]) {
      float v = out[p] / ls;
      if (sub == 0) logits[row[p]] = v;
      int kk = total_key(v);
      if (later_better(kk, (int)row[p], bk, bi)) {
        bk = kk;
        bi = (int)row[p];
      }
    }
  }
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) {
    int ok_ = __shfl_xor(bk, s), oi = __shfl_xor(bi, s);
    if (later_better(ok_, oi, bk, bi)) {
      bk = ok_;
      bi = oi;
    }
  }
  if (lane == 0) {
    sk[wave] = bk;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWavesPerBlock; w++)
      if (later_better(sk[w], si[w], bk, bi)) {
        bk = sk[w];
        bi = si[w];
      }
    best[blockIdx.x] = make_int2(bk, bi);
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) last = (atomicAdd(cnt, 1) == (int)gridDim.x - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();
  bk = INT_MIN;
  bi = -1;
  for (int i = threadIdx.x; i < (int)gridDim.x; i += kBlock) {
    int ck = (int)__hip_atomic_load(reinterpret_cast<const unsigned*>(&best[i].x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int ci = (int)__hip_atomic_load(reinterpret_cast<const unsigned*>(&best[i].y), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (later_better(ck, ci, bk, bi)) {
      bk = ck;
      bi = ci;
    }
  }
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) {
    int ok_ = __shfl_xor(bk, s), oi = __shfl_xor(bi, s);
    if (later_better(ok_, oi, bk, bi)) {
      bk = ok_;
      bi = oi;
    }
  }
  __syncthreads();
  if (lane == 0) {
    sk[wave] = bk;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWavesPerBlock; w++)
      if (later_better(sk[w], si[w], bk, bi)) {
        bk = sk[w];
        bi = si[w];
      }
    int pos = st[ST_POS];
    hist[pos] = bi;
    st[ST_ARGMAX] = bi;
    if (pos + 1 < max_len && pos + 1 >= st[ST_FIXED]) seq[pos + 1] = bi;
    st[ST_POS] = pos + 1;
    atomicExch(cnt, 0);
  }
}

// ------------------------------------------------------------------------------------------------------------
// Unit kernels.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_dequant(DMat m, float* __restrict__ out) {
  constexpr int CE = Fmt<DT>::kElems;
  size_t nch = (size_t)m.cols / CE;
  size_t id = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (id >= (size_t)m.rows * nch) return;
  size_t row = id / nch;
  int j = (int)(id % nch);
  RawChunk c = load_chunk<DT>(m, row, j);
#pragma unroll
  for (int i = 0; i < CE; i++) out[row * m.cols + (size_t)j * CE + i] = chunk_elem<DT>(c, i);
}

// One wave; n a multiple of 16.
__global__ void k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w, int n, float eps,
                          float* __restrict__ out) {
  int lane = threadIdx.x;
  float acc = 0.0f;
  for (int j = lane; j < n / 16; j += 64)
    for (int e = 0; e < 16; e++) acc = __builtin_fmaf(x[16 * j + e], x[16 * j + e], acc);
  float ss = group_sum<64>(acc);
  float r = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = lane; i < n; i += 64) out[i] = w[i] * (x[i] * r);
}

__global__ void k_rope(float* __restrict__ x, int heads, int half, const float* __restrict__ cs) {
  int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= heads * half) return;
  int hd = id / half, j = id % half;
  float* p = x + (size_t)hd * 2 * half;
  float x1 = p[j], x2 = p[j + half], c = cs[j], s = cs[half + j];
  p[j] = x1 * c - x2 * s;
  p[j + half] = x2 * c + x1 * s;
}

__global__ void k_topk(const float* __restrict__ logits, const float* __restrict__ bias, int n, int k,
                       int* __restrict__ ids, float* __restrict__ w) {
  int lane = threadIdx.x;
  float v = 0.0f;
  if (lane < n) v = bias ? logits[lane] + bias[lane] : logits[lane];
  wave_topk(v, n, k, lane, ids, w);
}

__global__ __launch_bounds__(kBlock) void k_argmax(const float* __restrict__ v, int n, int2* __restrict__ best,
                                                   int* __restrict__ cnt, int* __restrict__ outp) {
  __shared__ int sk[kWavesPerBlock], si[kWavesPerBlock];
  __shared__ int last;
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int bk = INT_MIN, bi = -1;
  for (int i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock) {
    int kk = total_key(v[i]);
    if (later_better(kk, i, bk, bi)) {
      bk = kk;
      bi = i;
    }
  }
  for (int s = 1; s < 64; s <<= 1) {
    int ok_ = __shfl_xor(bk, s), oi = __shfl_xor(bi, s);
    if (later_better(ok_, oi, bk, bi)) {
      bk = ok_;
      bi = oi;
    }
  }
  if (lane == 0) {
    sk[wave] = bk;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWavesPerBlock; w++)
      if (later_better(sk[w], si[w], bk, bi)) {
        bk = sk[w];
        bi = si[w];
      }
    best[blockIdx.x] = make_int2(bk, bi);
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) last = (atomicAdd(cnt, 1) == (int)gridDim.x - 1);
  __syncthreads();
  if (!last || threadIdx.x != 0) return;
  __threadfence();
  bk = INT_MIN;
  bi = -1;
  for (int i = 0; i < (int)gridDim.x; i++) {
    int ck = (int)__hip_atomic_load(reinterpret_cast<const unsigned*>(&best[i].x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int ci = (int)__hip_atomic_load(reinterpret_cast<const unsigned*>(&best[i].y), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (later_better(ck, ci, bk, bi)) {
      bk = ck;
      bi = ci;
    }
  }
  *outp = bi < 0 ? 0 : bi;
  atomicExch(cnt, 0);
}

__global__ void k_exp(const float* __restrict__ x, float* __restrict__ y, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = dexp(x[i]);
}

// ------------------------------------------------------------------------------------------------------------
// Launchers. Row lengths are compile-time; the switch covers the shapes of the Granite-MoE family and the small
// test models.
#define MOERT_K_CASES(X) X(128) X(256) X(512) X(1024) X(1536)
#define MOERT_KDOWN_CASES(X) X(128) X(256) X(512)

#define MOERT_DISPATCH(dt, K, BODY)                                   \
  switch (dt) {                                                       \
    case DT_Q8_0: {                                                   \
      constexpr int DTC = DT_Q8_0;                                    \
      switch (K) { MOERT_K_CASES(BODY) default: return hipErrorInvalidValue; } \
    } break;                                                          \
    case DT_Q4_0: {                                                   \
      constexpr int DTC = DT_Q4_0;                                    \
      switch (K) { MOERT_K_CASES(BODY) default: return hipErrorInvalidValue; } \
    } break;                                                          \
    case DT_F32: {                                                    \
      constexpr int DTC = DT_F32;                                     \
      switch (K) { MOERT_K_CASES(BODY) default: return hipErrorInvalidValue; } \
    } break;                                                          \
    default:                                                          \
      return hipErrorInvalidValue;                                    \
  }

template <int DT, int K, int P>
constexpr int rows_per_block() { return kWavesPerBlock * P * Geo<DT, K>::RPW; }

static inline int cdiv(long a, long b) { return (int)((a + b - 1) / b); }

constexpr int kGemvP = 4;
constexpr int kQkvNP = 1;
constexpr int kUpNP = 1;
constexpr int kHeadP = 4;
constexpr int kOprojP = 2;

hipError_t launch_gemv(hipStream_t s, const DMat& w, const float* x, float* y) {
#define BODY(KK)                                                                                    \
  case KK: {                                                                                        \
    constexpr int RB = rows_per_block<DTC, KK, kGemvP>();                                           \
    k_gemv<DTC, KK, kGemvP><<<cdiv(w.rows, RB), kBlock, 0, s>>>(w, x, y);                           \
  } break;
  MOERT_DISPATCH(w.dtype, w.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_embed(hipStream_t s, const DMat& emb, const Dims& d, const StepBufs& b) {
  switch (emb.dtype) {
    case DT_Q8_0: k_embed<DT_Q8_0><<<1, kBlock, 0, s>>>(emb, b.seq, b.state, d.emb_mult, b.h); break;
    case DT_Q4_0: k_embed<DT_Q4_0><<<1, kBlock, 0, s>>>(emb, b.seq, b.state, d.emb_mult, b.h); break;
    case DT_F32: k_embed<DT_F32><<<1, kBlock, 0, s>>>(emb, b.seq, b.state, d.emb_mult, b.h); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_qkv(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b) {
#define BODY(KK)                                                                                            \
  case KK: {                                                                                                \
    constexpr int PB = kWavesPerBlock * kQkvNP * Geo<DTC, KK>::RPW; /* pairs per block */                   \
    k_qkv<DTC, KK, kQkvNP><<<cdiv(L.qkv.rows / 2, PB), kBlock, 0, s>>>(                                     \
        L.qkv, b.h, L.ln_attn, d.eps, b.state, b.rope, d.heads, d.kv_heads, d.max_len, b.q, L.k_cache,      \
        L.v_cache);                                                                                         \
  } break;
  MOERT_DISPATCH(L.qkv.dtype, L.qkv.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_attn(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b) {
  k_attn<<<d.kv_heads * d.splits, kBlock, 0, s>>>(b.q, L.k_cache, L.v_cache, b.state + ST_POS, 1, d.heads,
                                                 d.kv_heads, d.max_len, d.attn_mult, d.splits, b.part,
                                                 b.attn_cnt, b.att);
  return hipGetLastError();
}

hipError_t launch_attn_unit(hipStream_t s, const float* q, const uint16_t* kc, const uint16_t* vc, int heads,
                            int kv_heads, int max_len, const int* len_dev, float scale, int splits, float* part,
                            int* cnt, float* out) {
  k_attn<<<kv_heads * splits, kBlock, 0, s>>>(q, kc, vc, len_dev, 0, heads, kv_heads, max_len, scale, splits,
                                              part, cnt, out);
  return hipGetLastError();
}

hipError_t launch_oproj(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b) {
#define BODY(KK)                                                                            \
  case KK: {                                                                                \
    constexpr int RB = rows_per_block<DTC, KK, kOprojP>();                                  \
    k_oproj<DTC, KK, kOprojP><<<cdiv(L.o.rows, RB), kBlock, 0, s>>>(L.o, b.att, d.res_mult, b.h); \
  } break;
  MOERT_DISPATCH(L.o.dtype, L.o.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_router(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                         bool normalize) {
#define BODY(KK)                                                                                          \
  case KK:                                                                                                \
    if (normalize)                                                                                        \
      k_router<DTC, KK, true><<<1, 1024, 0, s>>>(L.router, L.router_bias, b.h, L.ln_moe, d.eps, d.top_k,  \
                                                 b.xn, b.route_ids + layer * d.top_k,                     \
                                                 b.route_w + layer * d.top_k);                            \
    else                                                                                                  \
      k_router<DTC, KK, false><<<1, 1024, 0, s>>>(L.router, L.router_bias, b.h, L.ln_moe, d.eps, d.top_k, \
                                                  b.xn, b.route_ids + layer * d.top_k,                    \
                                                  b.route_w + layer * d.top_k);                           \
    break;
  MOERT_DISPATCH(L.router.dtype, L.router.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_expert_up(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer) {
#define BODY(KK)                                                                                         \
  case KK: {                                                                                             \
    constexpr int PB = kWavesPerBlock * kUpNP * Geo<DTC, KK>::RPW;                                       \
    k_expert_up<DTC, KK, kUpNP><<<cdiv((long)d.top_k * d.inter, PB), kBlock, 0, s>>>(                   \
        L.gate_up, b.xn, b.route_ids + layer * d.top_k, d.top_k, d.inter, b.act);                        \
  } break;
  MOERT_DISPATCH(L.gate_up.dtype, L.gate_up.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_expert_down(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                              bool accumulate) {
#define BODY(KK)                                                                                          \
  case KK:                                                                                                \
    k_expert_down<DTC, KK><<<cdiv(d.hidden, kWavesPerBlock), kBlock, 0, s>>>(                             \
        L.down, b.act, b.route_ids + layer * d.top_k, b.route_w + layer * d.top_k, d.top_k, d.hidden,     \
        d.res_mult, accumulate, accumulate ? b.h : b.logits);                                             \
    break;
  switch (L.down.dtype) {
    case DT_Q8_0: { constexpr int DTC = DT_Q8_0; switch (L.down.cols) { MOERT_KDOWN_CASES(BODY) default: return hipErrorInvalidValue; } } break;
    case DT_Q4_0: { constexpr int DTC = DT_Q4_0; switch (L.down.cols) { MOERT_KDOWN_CASES(BODY) default: return hipErrorInvalidValue; } } break;
    case DT_F32: { constexpr int DTC = DT_F32; switch (L.down.cols) { MOERT_KDOWN_CASES(BODY) default: return hipErrorInvalidValue; } } break;
    default: return hipErrorInvalidValue;
  }
#undef BODY
  return hipGetLastError();
}

int head_blocks(const DMat& head) {
  int rpw;
  int ce = head.dtype == DT_Q8_0 ? 16 : head.dtype == DT_Q4_0 ? 32 : 4;
  rpw = kWave / lanes_per_row(head.cols / ce);
  return cdiv(head.rows, kWavesPerBlock * kHeadP * rpw);
}

hipError_t launch_head(hipStream_t s, const DMat& head, const float* norm, const Dims& d, const StepBufs& b) {
#define BODY(KK)                                                                                        \
  case KK: {                                                                                            \
    constexpr int RB = rows_per_block<DTC, KK, kHeadP>();                                               \
    k_head<DTC, KK, kHeadP><<<cdiv(head.rows, RB), kBlock, 0, s>>>(head, b.h, norm, d.eps,              \
                                                                   d.logits_scaling, b.logits, b.best,  \
                                                                   b.head_cnt, b.state, b.seq,          \
                                                                   b.argmax_hist, d.max_len);           \
  } break;
  MOERT_DISPATCH(head.dtype, head.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_dequant(hipStream_t s, const DMat& w, float* out) {
  size_t n;
  switch (w.dtype) {
    case DT_Q8_0: n = (size_t)w.rows * (w.cols / 16); k_dequant<DT_Q8_0><<<cdiv(n, kBlock), kBlock, 0, s>>>(w, out); break;
    case DT_Q4_0: n = (size_t)w.rows * (w.cols / 32); k_dequant<DT_Q4_0><<<cdiv(n, kBlock), kBlock, 0, s>>>(w, out); break;
    case DT_F32: n = (size_t)w.rows * (w.cols / 4); k_dequant<DT_F32><<<cdiv(n, kBlock), kBlock, 0, s>>>(w, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rmsnorm(hipStream_t s, const float* x, const float* w, int n, float eps, float* out) {
  k_rmsnorm<<<1, 64, 0, s>>>(x, w, n, eps, out);
  return hipGetLastError();
}

hipError_t launch_rope(hipStream_t s, float* x, int heads, int head_dim, const float* cs) {
  int n = heads * head_dim / 2;
  k_rope<<<cdiv(n, 256), 256, 0, s>>>(x, heads, head_dim / 2, cs);
  return hipGetLastError();
}

hipError_t launch_topk(hipStream_t s, const float* logits, const float* bias, int n, int k, int* ids, float* w) {
  k_topk<<<1, 64, 0, s>>>(logits, bias, n, k, ids, w);
  return hipGetLastError();
}

hipError_t launch_argmax(hipStream_t s, const float* v, int n, int2* best, int* cnt, int* out) {
  int blocks = cdiv(n, kBlock * 4);
  if (blocks > 1024) blocks = 1024;
  if (blocks < 1) blocks = 1;
  k_argmax<<<blocks, kBlock, 0, s>>>(v, n, best, cnt, out);
  return hipGetLastError();
}

hipError_t launch_exp(hipStream_t s, const float* x, float* y, int n) {
  k_exp<<<cdiv(n, 256), 256, 0, s>>>(x, y, n);
  return hipGetLastError();
}

}  // namespace moert

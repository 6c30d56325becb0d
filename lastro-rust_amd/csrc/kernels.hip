// Decode-step kernels for gfx950 (wave64). The evaluation order of every reduction is the one stated in
// dev_math.h; the reference kernels these replace are cited on each kernel (paths relative to the reference
// root, rust/moe-rt/src).
#include <algorithm>
#include <climits>

#include "cache_dev.h"
#include "dev_rows.h"
#include "kernels.h"
#include "launch.h"
#include "moe_norm.h"
#include "attn_dev.h"
#include "timeline.h"

namespace moert {

namespace {
thread_local hipEvent_t t_armed[2] = {nullptr, nullptr};
}
void arm_launch_events(hipEvent_t start, hipEvent_t stop) {
  t_armed[0] = start;
  t_armed[1] = stop;
}
bool take_armed_events(hipEvent_t* start, hipEvent_t* stop) {
  if (!t_armed[0]) return false;
  *start = t_armed[0];
  *stop = t_armed[1];
  t_armed[0] = t_armed[1] = nullptr;
  return true;
}

// ------------------------------------------------------------------------------------------------------------
// Plain GEMV y = W x (gpu.rs:21-38).
template <int DT, int K, int P>
__global__ __launch_bounds__(kBlock) void k_gemv(DMat m, const float* __restrict__ x, float* __restrict__ y) {
  using G = Geo<DT, K>;
  __shared__ float xs[K];
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  size_t base = ((size_t)blockIdx.x * kWavesPerBlock + wave) * (P * G::RPW);
  size_t row[P];
  bool ok[P];
#pragma unroll
  for (int p = 0; p < P; p++) {
    row[p] = base + (size_t)p * G::RPW + rw;
    ok[p] = row[p] < (size_t)m.rows;
  }
  CopyIn<K, kBlock> xin;
  copy_fetch<K, kBlock>(x, xin);
  Rows<DT, K, P> rr;
  rows_load<DT, K, P>(rr, m, row, ok, sub);
  copy_finish<K, kBlock>(xin, xs);
  XReg<DT, K> xr;
  load_x<DT, K>(xr, xs, sub);
  float out[P];
  rows_fma<DT, K, P>(rr, ok, xr, sub, out);
#pragma unroll
  for (int p = 0; p < P; p++)
    if (ok[p] && sub == 0) y[row[p]] = out[p];
}

// ------------------------------------------------------------------------------------------------------------
// Embedding row times embedding_multiplier (model.rs:134-138); the token is seq[pos] on the device.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_embed(DMat e, const int* __restrict__ seq, const int* __restrict__ st,
                                                  float mult, float* __restrict__ h, unsigned* __restrict__ step_ctr,
                                                  const float* __restrict__ rope, float* __restrict__ rope_cur,
                                                  Tl tl) {
  TL_START(tl);
  if (step_ctr && threadIdx.x == 0) *step_ctr += 1u;
  static_assert(kBlock >= 64, "one thread per rope element");
  if (rope_cur && threadIdx.x < 64) rope_cur[threadIdx.x] = rope[(size_t)st[ST_POS] * 64 + threadIdx.x];
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
  TL_END(tl);
}

constexpr int kQkvWaves = 8;  // waves per workgroup of k_qkv

// ------------------------------------------------------------------------------------------------------------
// Attention block input: rmsnorm -> [q; k; v] GEMV -> rotate_half RoPE of q and k -> q to `q` (f32), k and v to
// row `pos` of the fp16 KV cache. Replaces rmsnorm + gemv q/k/v + rope + the two KV copies
// (gpu_model.rs:341-378) and rope_kv / gemv_row (gpu.rs:151-197). A wave owns NP*RPW row pairs (j, j+32) of
// a head, so both halves of a rotation meet in the same lanes.
template <int DT, int K, int NP>
__global__ __launch_bounds__(kQkvWaves * 64) void k_qkv(DMat m, const float* __restrict__ h, const float* __restrict__ lnw,
                                                float eps, const int* __restrict__ st, const float* __restrict__ rope,
                                                int heads, int kvh, int max_len, float* __restrict__ q,
                                                uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, Tl tl) {
  TL_START(tl);
  using G = Geo<DT, K>;
  constexpr int P = 2 * NP;
  __shared__ float xs[K];
  __shared__ float rs;
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  int npairs = m.rows / 2;
  int wbase = (blockIdx.x * kQkvWaves + wave) * (NP * G::RPW);
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
  // position first, then the activation, then this lane's cos/sin (they depend only on the position), then the
  // weights: each wait below covers only what was issued before the thing waited for
  const int pos = st[ST_POS];
  NormIn<K, (kQkvWaves * 64)> hin;
  norm_fetch<K, (kQkvWaves * 64)>(h, lnw, hin);
  const float* cs = rope + (size_t)pos * 64;
  float cv[NP], sv[NP];
#pragma unroll
  for (int a = 0; a < NP; a++) {
    const int jp = gp[a] % 32;
    cv[a] = cs[jp];
    sv[a] = cs[32 + jp];
  }
  __builtin_amdgcn_sched_barrier(0);
  Rows<DT, K, P> rr;
  rows_load<DT, K, P>(rr, m, row, ok, sub);
  norm_finish<K, (kQkvWaves * 64)>(hin, eps, xs, &rs);
  TL_PHASE(tl, 2);
  XReg<DT, K> xr;
  load_x<DT, K>(xr, xs, sub);
  float out[P];
  rows_fma<DT, K, P>(rr, ok, xr, sub, out);
  TL_PHASE(tl, 3);
  if (sub != 0) return;
#pragma unroll
  for (int a = 0; a < NP; a++) {
    if (!ok[2 * a]) continue;
    int head = gp[a] / 32, jp = gp[a] % 32;
    float x1 = out[2 * a], x2 = out[2 * a + 1];
    float c = cv[a], sn = sv[a];
    if (head < heads) {
      q[head * 64 + jp] = x1 * c - x2 * sn;
      q[head * 64 + jp + 32] = x2 * c + x1 * sn;
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
  TL_END(tl);
}

// ------------------------------------------------------------------------------------------------------------
// Split-KV GQA decode attention over the fp16 cache, two kernels (attn_split + attn_combine, gpu.rs:205-292).
// k_attn_split: one wave per (KV head g, split s) serves all G query heads of g, so each K/V byte is read once.
// Lane i holds the K row of position i of a tile in registers (scores: lane = position); V goes straight from HBM
// to the wave's LDS (p.v: lane = dim), double buffered: the next tile's K and V are requested before the current
// tile's scores are computed. Partials (m, l, acc[64]) per (head, split).
// k_attn_combine: one wave per query head merges the used splits in split order, all partials loaded at once.

// A 128-byte row held in named registers (an array copied to LDS in a loop is turned into a memcpy from a stack
// slot by the compiler).
struct Row8 {
  uint4 a, b, c, d, e, f, g, h;
  __device__ __forceinline__ void load(const uint4* p) {
    a = p[0]; b = p[1]; c = p[2]; d = p[3]; e = p[4]; f = p[5]; g = p[6]; h = p[7];
  }
  // member i for a compile-time i (unrolled loops)
  __device__ __forceinline__ uint4 at(int i) const {
    return i == 0 ? a : i == 1 ? b : i == 2 ? c : i == 3 ? d : i == 4 ? e : i == 5 ? f : i == 6 ? g : h;
  }
};

template <int G>
__global__ __launch_bounds__(256) void k_attn_split(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                   const uint16_t* __restrict__ vc, const int* __restrict__ lenp,
                                                   int len_add, int max_len, float scale, int tps, int splits,
                                                   float* __restrict__ part) {
  // workgroup = G waves, wave w serves query head g*G + w; the K rows are read by every wave (L2 after the first),
  // the V tile is moved into LDS once, each wave carrying a share of its rows
  __shared__ uint4 Vs[2][64][8];  // fp16 V tiles, row i = position
  __shared__ float Qs[G][64];
  __shared__ float Ps[G][64];
  const int g = blockIdx.x / splits, s = blockIdx.x % splits;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  {  // position blockIdx.y of a multi-position step: its own query, partials and length
    const int nh = gridDim.x / splits * G;
    q += (size_t)blockIdx.y * nh * 64;
    part += (size_t)blockIdx.y * nh * splits * 66;
    len_add += blockIdx.y;
  }
  const int h = g * G + w;
  const float NEG_INF = __int_as_float(0xff800000);
  const uint16_t* K = kc + (size_t)g * max_len * 64;
  const uint16_t* V = vc + (size_t)g * max_len * 64;
  auto v_share = [&](int t, int buf) {
    const uint16_t* src = V + ((size_t)t * 64 + (lane >> 3)) * 64 + (lane & 7) * 8;
    for (int e = w; e < 8; e += G)
      __builtin_amdgcn_global_load_lds(src + (size_t)e * 8 * 64, &Vs[buf][8 * e][0], 16, 0, 0);
  };
  // split s covers tiles [s*tps, s*tps + tps); its first tile is requested before the length is known (the grid
  // only covers tiles inside the cache)
  const int t0 = s * tps;
  // q and the length first (loads complete in issue order), then the first tile's K rows and V shares
  const float qv = q[h * 64 + lane];
  const int len = *lenp + len_add;
  __builtin_amdgcn_sched_barrier(0);
  Row8 kn;
  kn.load(reinterpret_cast<const uint4*>(K + (size_t)(t0 * 64 + lane) * 64));
  v_share(t0, 0);
  Qs[w][lane] = qv;
  const int nb = (len + 63) / 64;
  if (t0 >= nb) {
    __builtin_amdgcn_s_waitcnt(0);  // the tile copy into LDS has finished before the wave ends
    return;
  }
  const int t1 = min(t0 + tps, nb);
  float m = NEG_INF, l = 0.0f, acc = 0.0f;
  for (int t = t0; t < t1; t++) {
    const int nv = min(64, len - t * 64), buf = (t - t0) & 1;
    const Row8 kr = kn;
    __syncthreads();  // Qs written; every wave is done with the buffer the prefetch overwrites
    if (t + 1 < t1) {
      kn.load(reinterpret_cast<const uint4*>(K + (size_t)((t + 1) * 64 + lane) * 64));
      v_share(t + 1, buf ^ 1);
    }
    // scores: lane = position, chain over the 64 dims in order
    float dt = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint4 ke = kr.at(e);
      const uint32_t wv[4] = {ke.x, ke.y, ke.z, ke.w};
#pragma unroll
      for (int hh = 0; hh < 2; hh++) {
        const float4 qv = *reinterpret_cast<const float4*>(&Qs[w][8 * e + 4 * hh]);
        const float qa[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const uint32_t word = wv[2 * hh + (c >> 1)];
          dt = __builtin_fmaf(qa[c], h2f((uint16_t)(word >> (16 * (c & 1)))), dt);
        }
      }
    }
    const float sc = lane < nv ? dt * scale : NEG_INF;
    const float tmax = group_max<64>(sc);
    const float mn = m > tmax ? m : tmax;
    const float alpha = dexp(m - mn);
    const float p = dexp(sc - mn);
    const float ts = group_sum<64>(p);
    l = __builtin_fmaf(l, alpha, ts);
    Ps[w][lane] = p;
    m = mn;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's share of the tile's V rows has landed in LDS
    __syncthreads();                // every share has
    // p.v: lane = dim, chain over the valid positions in order; LDS reads batched 8 positions at a time
    const uint16_t* vcol = reinterpret_cast<const uint16_t*>(&Vs[buf][0][0]) + lane;
    float pv = 0.0f;
#pragma unroll
    for (int i0 = 0; i0 < 64; i0 += 8) {
      if (i0 < nv) {
        float vf[8];
#pragma unroll
        for (int u = 0; u < 8; u++) vf[u] = h2f(vcol[(i0 + u) * 64]);
        const float4 p0 = *reinterpret_cast<const float4*>(&Ps[w][i0]);
        const float4 p1 = *reinterpret_cast<const float4*>(&Ps[w][i0 + 4]);
        const float pa[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
        for (int u = 0; u < 8; u++)
          if (i0 + u < nv) pv = __builtin_fmaf(pa[u], vf[u], pv);
      }
    }
    acc = __builtin_fmaf(acc, alpha, pv);
  }
  float* pp = part + ((size_t)h * splits + s) * 66;
  if (lane == 0) {
    pp[0] = m;
    pp[1] = l;
  }
  pp[2 + lane] = acc;
}

// Tile-parallel form of k_attn_split for a split of exactly T tiles: workgroup = G x T waves, wave (wh, wt) takes
// query head g*G + wh and tile t0 + wt. Every wave computes its tile's scores and tile max at once; the running max
// m_{t-1} each tile's online-softmax step needs is the max of the earlier tiles' maxima (exchanged through LDS), so
// alpha_t = exp(m_{t-1} - m_t), p_t = exp(s - m_t), the tile sum and p.v are formed in parallel; the first wave of
// each head then applies l = fma(l, alpha_t, sum_t) and acc = fma(acc, alpha_t, pv_t) over the tiles in order.
// Every operation and its order are those of the sequential kernel, so the partials are the same bit for bit.
template <int G, int T>
__global__ __launch_bounds__(G * T * 64) void k_attn_tiles(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                          const uint16_t* __restrict__ vc, const int* __restrict__ lenp,
                                                          int len_add, int max_len, float scale, int splits,
                                                          float* __restrict__ part, Tl tl) {
  TL_START(tl);
  constexpr int TR = 8 % G == 0 ? 64 : 72;  // tile rows (64..71: padding for VShare when G does not divide 8)
  constexpr int KS = 68;                     // K row stride in floats: 16-byte rows, conflict-free row reads
  __shared__ __align__(16) float Vs[T][TR][64];  // V tiles in f32, row i = position
  __shared__ __align__(16) float Ks[T][TR][KS];  // K tiles in f32, row i = position
  __shared__ float Qs[G][64];
  __shared__ float Ps[G][T][64];
  __shared__ float Pv[G][T][64];
  __shared__ float Tm[G][T], Al[G][T], Ts[G][T];
  const int g = blockIdx.x / splits, s = blockIdx.x % splits;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  {  // position blockIdx.y of a multi-position step: its own query, partials and length
    const int nh = gridDim.x / splits * G;
    q += (size_t)blockIdx.y * nh * 64;
    part += (size_t)blockIdx.y * nh * splits * 66;
    len_add += blockIdx.y;
  }
  const int wh = wid % G, wt = wid / G;
  const int h = g * G + wh;
  const float NEG_INF = __int_as_float(0xff800000);
  const uint16_t* K = kc + (size_t)g * max_len * 64;
  const uint16_t* V = vc + (size_t)g * max_len * 64;
  const int t0 = s * T, t = t0 + wt;
  // the tile's rows are requested before the length is known; a tile past the end of the cache (last split, when
  // T does not divide the tile count) reads the cache's last tile instead and is never used
  const int tc = min(t, max_len / 64 - 1);
  // q and the length first (loads complete in issue order), then this wave's shares of the tile's K and V (the G
  // waves of a tile move it together, each element is loaded and converted once)
  const float qv = q[h * 64 + lane];
  const int len = *lenp + len_add;
  __builtin_amdgcn_sched_barrier(0);
  VShare<G> ksh;
  ksh.load(K, tc, lane, wh);
  __builtin_amdgcn_sched_barrier(0);  // K (needed first) ahead of V
  VShare<G> vsh;
  vsh.load(V, tc, lane, wh);
  Qs[wh][lane] = qv;  // every wave of head wh stores the same q (an unconditional store keeps the q load first)
  const int nb = (len + 63) / 64;
  const int used = min(T, nb - t0);  // tiles of this split inside the length (>= 1 when the split is used)
  const bool active = wt < used;
  const int nv = active ? min(64, len - t * 64) : 0;
  ksh.template store<KS>(&Ks[wt][0][0], lane, wh, nv);
  __syncthreads();  // Qs, K tiles
  TL_PHASE(tl, 2);
  // scores: lane = position, chain over the 64 dims in order (an inactive tile's scores are discarded)
  float sc;
  {
    float dt = 0.0f;
    const float* krow = &Ks[wt][lane][0];
#pragma unroll
    for (int d4 = 0; d4 < 16; d4++) {
      const float4 kk = *reinterpret_cast<const float4*>(krow + 4 * d4);
      const float4 qq = *reinterpret_cast<const float4*>(&Qs[wh][4 * d4]);
      dt = __builtin_fmaf(qq.x, kk.x, dt);
      dt = __builtin_fmaf(qq.y, kk.y, dt);
      dt = __builtin_fmaf(qq.z, kk.z, dt);
      dt = __builtin_fmaf(qq.w, kk.w, dt);
    }
    sc = lane < nv ? dt * scale : NEG_INF;  // nv = 0 for an inactive tile
  }
  const float tmax = group_max<64>(sc);
  if (lane == 0) Tm[wh][wt] = tmax;
  __syncthreads();  // tile maxima
  TL_PHASE(tl, 3);
  float pv = 0.0f;
  if (active) {
    float mprev = NEG_INF;
    for (int u = 0; u < wt; u++) mprev = mprev > Tm[wh][u] ? mprev : Tm[wh][u];
    const float mn = mprev > tmax ? mprev : tmax;
    const float alpha = dexp(mprev - mn);
    const float p = dexp(sc - mn);
    const float ts = group_sum<64>(p);
    Ps[wh][wt][lane] = p;
    if (lane == 0) {
      Al[wh][wt] = alpha;
      Ts[wh][wt] = ts;
    }
  }
  vsh.template store<64>(&Vs[wt][0][0], lane, wh, nv);
  __syncthreads();  // every share of every V tile stored; P written
  TL_PHASE(tl, 4);
  if (active) {
    // p.v: lane = dim, chain over the positions in order, without branches so that every LDS read can be issued
    // ahead of the chain. A position past the length has p = exp(-inf) = 0 and its V element is stored as 0, so
    // its step fma(0, 0, pv) returns pv unchanged (pv starts at +0 and an exact zero sum is +0, so pv is never -0):
    // the chain equals the one over the valid positions only, bit for bit.
    const float* vcol = &Vs[wt][0][lane];
    if constexpr (G * T < 16) {
#pragma unroll
      for (int i0 = 0; i0 < 64; i0 += 4) {
        const float4 p4 = *reinterpret_cast<const float4*>(&Ps[wh][wt][i0]);
        const float pa[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
        for (int u = 0; u < 4; u++) pv = __builtin_fmaf(pa[u], vcol[(i0 + u) * 64], pv);
      }
    } else {
      // 16 waves leave 128 VGPRs a lane, too few to hoist every read: batches of 8 positions, valid ones only
#pragma unroll
      for (int i0 = 0; i0 < 64; i0 += 8) {
        if (i0 < nv) {
          float vf[8];
#pragma unroll
          for (int u = 0; u < 8; u++) vf[u] = vcol[(i0 + u) * 64];
          const float4 p0 = *reinterpret_cast<const float4*>(&Ps[wh][wt][i0]);
          const float4 p1 = *reinterpret_cast<const float4*>(&Ps[wh][wt][i0 + 4]);
          const float pa[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
          for (int u = 0; u < 8; u++)
            if (i0 + u < nv) pv = __builtin_fmaf(pa[u], vf[u], pv);
        }
      }
    }
    if (wt > 0) Pv[wh][wt][lane] = pv;
  }
  __syncthreads();  // p.v of every tile
  TL_PHASE(tl, 5);
  if (wt != 0 || used <= 0) {
    TL_END(tl);
    return;
  }
  float m = NEG_INF, l = 0.0f, acc = 0.0f;
  for (int u = 0; u < used; u++) {
    const float a = Al[wh][u];
    l = __builtin_fmaf(l, a, Ts[wh][u]);
    acc = __builtin_fmaf(acc, a, u == 0 ? pv : Pv[wh][u][lane]);
    m = m > Tm[wh][u] ? m : Tm[wh][u];
  }
  float* pp = part + ((size_t)h * splits + s) * 66;
  if (lane == 0) {
    pp[0] = m;
    pp[1] = l;
  }
  pp[2 + lane] = acc;
  TL_END(tl);
}

// Multi-position form of k_attn_tiles for the block step: one workgroup per (KV head g, split s, group of up to
// kMqMaxPos consecutive positions of the block), one wave per tile of the split. The split's K and V tiles are read
// once for the whole group and every (position, query head) unit of the group goes through the three steps of
// k_attn_tiles: (1) scores (lane = position of the tile, the K row in registers) and tile maxima, (2) alpha, p and
// the tile sum, then p.v (lane = dim, the V column in registers), (3) the in-order combine of the tiles into the
// split's partial. The K row is needed only in (1) and the V column only from (2) on, so they share registers and
// several units run side by side: two score chains, p of four units, four p.v chains. Queries, scores, p and p.v
// go through LDS (a unit's score row becomes its p row, then its p.v row), and the V tile is moved into registers
// through LDS in two halves; the small footprint keeps five workgroups on a compute unit. Position y of the block
// sees the first len + y cache positions, so its valid rows differ per tile: rows at and past its tile length get
// score -inf (p = 0) and V element +0, which is what k_attn_tiles' zeroed rows give; the partials are the same bit
// for bit.
constexpr int kMqMaxPos = 6;
template <int G, int T>
__global__ __launch_bounds__(T * 64) void k_attn_mq(const float* __restrict__ q, const uint16_t* __restrict__ kc,
                                                   const uint16_t* __restrict__ vc, const int* __restrict__ lenp,
                                                   int len_add, int max_len, float scale, int splits, int ny, int npw,
                                                   float* __restrict__ part) {
  constexpr int NU = kMqMaxPos * G;  // units of a group: unit u = position u / G, query head g * G + u % G
  __shared__ __align__(16) float Vt[T][32 * 32];  // wave wt: half of its fp16 V tile, [32][64]
  __shared__ __align__(16) float Sp[T][NU][64];    // wave wt: its scores, then p, then p.v, row = unit
  __shared__ __align__(16) float Qs[NU][64];
  __shared__ float Tm[NU][T], Al[NU][T], Ts[NU][T];
  const int g = blockIdx.x / splits, s = blockIdx.x % splits;
  const int lane = threadIdx.x & 63, wt = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: SGPRs
  const int nh = gridDim.x / splits * G;
  const int y0 = blockIdx.y * npw, yn = min(ny, y0 + npw) - y0;  // positions y0 .. y0 + yn - 1 of the block
  const int units = yn * G;
  const float NEG_INF = __int_as_float(0xff800000);
  const uint16_t* K = kc + (size_t)g * max_len * 64;
  const uint16_t* V = vc + (size_t)g * max_len * 64;
  const int t0 = s * T, t = t0 + wt;
  const int tl = min(t, max_len / 64 - 1);  // a tile past the end of the cache is never used by any position
  // the group's queries and the first length, then the K row of this lane and the V tile in 8 pieces of 8 rows
  for (int u = wt; u < units; u += T) Qs[u][lane] = q[((size_t)(y0 + u / G) * nh + g * G + u % G) * 64 + lane];
  const int len0 = *lenp + len_add + y0;  // length seen by the group's first position; position y sees len0 + y
  __builtin_amdgcn_sched_barrier(0);
  Row8 kn;
  kn.load(reinterpret_cast<const uint4*>(K + (size_t)(tl * 64 + lane) * 64));
  Row8 vp;
  {
    const uint4* src = reinterpret_cast<const uint4*>(V + ((size_t)tl * 64 + (lane >> 3)) * 64 + (lane & 7) * 8);
    vp.a = src[0 * 64]; vp.b = src[1 * 64]; vp.c = src[2 * 64]; vp.d = src[3 * 64];
    vp.e = src[4 * 64]; vp.f = src[5 * 64]; vp.g = src[6 * 64]; vp.h = src[7 * 64];
  }
  if (t0 * 64 >= len0 + yn - 1) {  // no position of the group reaches this split
    __builtin_amdgcn_s_waitcnt(0);
    return;
  }
  uint4* const vt = reinterpret_cast<uint4*>(&Vt[wt][0]);  // row i = 8 uint4
#pragma unroll
  for (int e = 0; e < 4; e++) vt[(8 * e + (lane >> 3)) * 8 + (lane & 7)] = vp.at(e);  // rows 0..31
  // valid rows of this wave's tile for unit u (0: the tile is past the position's length)
  auto valid = [&](int u) { return max(0, min(64, len0 + u / G - t * 64)); };
  float* const sp = &Sp[wt][0][0];
  {
    float kr[64];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint4 ke = kn.at(e);
      const uint32_t wv[4] = {ke.x, ke.y, ke.z, ke.w};
#pragma unroll
      for (int j = 0; j < 8; j++) kr[8 * e + j] = h2f((uint16_t)(wv[j >> 1] >> (16 * (j & 1))));
    }
    __syncthreads();  // queries
    // (1) scores: lane = position, chain over the 64 dims in order; the tile maximum. Two units at a time; the
    // second of an odd count repeats the first and is not stored.
    for (int k = 0; k < units; k += 2) {
      const int kb = k + 1 < units ? k + 1 : k;
      const int na = valid(k), nb = k + 1 < units ? valid(kb) : 0;
      float sa = NEG_INF, sb = NEG_INF, ta = NEG_INF, tb = NEG_INF;
      if (na > 0 || nb > 0) {
        float da = 0.0f, db = 0.0f;
#pragma unroll
        for (int d4 = 0; d4 < 16; d4++) {
          const float4 qa = *reinterpret_cast<const float4*>(&Qs[k][4 * d4]);
          const float4 qb = *reinterpret_cast<const float4*>(&Qs[kb][4 * d4]);
          da = __builtin_fmaf(qa.x, kr[4 * d4], da);
          db = __builtin_fmaf(qb.x, kr[4 * d4], db);
          da = __builtin_fmaf(qa.y, kr[4 * d4 + 1], da);
          db = __builtin_fmaf(qb.y, kr[4 * d4 + 1], db);
          da = __builtin_fmaf(qa.z, kr[4 * d4 + 2], da);
          db = __builtin_fmaf(qb.z, kr[4 * d4 + 2], db);
          da = __builtin_fmaf(qa.w, kr[4 * d4 + 3], da);
          db = __builtin_fmaf(qb.w, kr[4 * d4 + 3], db);
        }
        sa = lane < na ? da * scale : NEG_INF;
        sb = lane < nb ? db * scale : NEG_INF;
        ta = group_max<64>(sa);
        tb = group_max<64>(sb);
      }
      sp[k * 64 + lane] = sa;
      if (k + 1 < units) sp[(k + 1) * 64 + lane] = sb;
      if (lane == 0) {
        Tm[k][wt] = ta;
        if (k + 1 < units) Tm[k + 1][wt] = tb;
      }
    }
  }
  float vr[64];  // the V column of this lane, f32
  {
    const uint16_t* col = reinterpret_cast<const uint16_t*>(vt) + lane;
#pragma unroll
    for (int i = 0; i < 32; i++) vr[i] = h2f(col[i * 64]);
    wave_lds_sync();  // the first half is read
#pragma unroll
    for (int e = 4; e < 8; e++) vt[(8 * (e - 4) + (lane >> 3)) * 8 + (lane & 7)] = vp.at(e);  // rows 32..63
    wave_lds_sync();
#pragma unroll
    for (int i = 32; i < 64; i++) vr[i] = h2f(col[(i - 32) * 64]);
  }
  __syncthreads();  // tile maxima
  // (2) lane u < units: m_prev, m and alpha of unit u for this tile
  float mu = NEG_INF;
  if (lane < units) {
    float mprev = NEG_INF;
#pragma unroll
    for (int v = 0; v < T; v++)
      if (v < wt) mprev = mprev > Tm[lane][v] ? mprev : Tm[lane][v];
    const float tmax = Tm[lane][wt];
    mu = mprev > tmax ? mprev : tmax;
    if (valid(lane) > 0) Al[lane][wt] = dexp_sel(mprev - mu);
  }
  // p = exp(s - m) over the score rows and the tile sums, four units at a time (a unit whose tile is past its
  // length gets a p row and sum that nothing reads)
  for (int k0 = 0; k0 < units; k0 += 4) {
    float pj[4], tj[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int k = min(k0 + j, units - 1);
      const float m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mu), k));
      pj[j] = dexp_sel(sp[k * 64 + lane] - m);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) tj[j] = group_sum<64>(pj[j]);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if (k0 + j < units) {
        sp[(k0 + j) * 64 + lane] = pj[j];
        if (lane == 0) Ts[k0 + j][wt] = tj[j];
      }
    }
  }
  wave_lds_sync();  // this wave's p rows
  // p.v: lane = dim, chain over the positions in order, the V elements of rows past the position's length as +0;
  // four units at a time (past the last unit, the last unit's row again, not stored). Each result replaces its
  // unit's p row (all of the row's reads come first: the result depends on them).
  for (int k0 = 0; k0 < units; k0 += 4) {
    int nv[4], row[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      row[j] = min(k0 + j, units - 1);
      nv[j] = valid(row[j]);
    }
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (nv[0] == 64 && nv[1] == 64 && nv[2] == 64 && nv[3] == 64) {
#pragma unroll
      for (int i0 = 0; i0 < 64; i0 += 4) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float4 p4 = *reinterpret_cast<const float4*>(&sp[row[j] * 64 + i0]);
          acc[j] = __builtin_fmaf(p4.x, vr[i0], acc[j]);
          acc[j] = __builtin_fmaf(p4.y, vr[i0 + 1], acc[j]);
          acc[j] = __builtin_fmaf(p4.z, vr[i0 + 2], acc[j]);
          acc[j] = __builtin_fmaf(p4.w, vr[i0 + 3], acc[j]);
        }
      }
    } else {  // a tile the positions see in part (the last of the group's lengths)
#pragma unroll
      for (int i0 = 0; i0 < 64; i0 += 4) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float4 p4 = *reinterpret_cast<const float4*>(&sp[row[j] * 64 + i0]);
          acc[j] = __builtin_fmaf(p4.x, i0 < nv[j] ? vr[i0] : 0.0f, acc[j]);
          acc[j] = __builtin_fmaf(p4.y, i0 + 1 < nv[j] ? vr[i0 + 1] : 0.0f, acc[j]);
          acc[j] = __builtin_fmaf(p4.z, i0 + 2 < nv[j] ? vr[i0 + 2] : 0.0f, acc[j]);
          acc[j] = __builtin_fmaf(p4.w, i0 + 3 < nv[j] ? vr[i0 + 3] : 0.0f, acc[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
      if (k0 + j < units && nv[j] > 0) sp[(k0 + j) * 64 + lane] = acc[j];
  }
  __syncthreads();  // p.v, alpha and sums of every tile
  // (3) the split's partial of each unit: l and acc over the used tiles in order
  for (int k = wt; k < units; k += T) {
    const int y = k / G, hh = k % G;
    const int used = min(T, (len0 + y + 63) / 64 - t0);
    if (used <= 0) continue;
    float m = NEG_INF, l = 0.0f, acc = 0.0f;
#pragma unroll
    for (int v = 0; v < T; v++) {
      if (v < used) {
        const float a = Al[k][v];
        l = __builtin_fmaf(l, a, Ts[k][v]);
        acc = __builtin_fmaf(acc, a, Sp[v][k][lane]);
        m = m > Tm[k][v] ? m : Tm[k][v];
      }
    }
    float* pp = part + (((size_t)(y0 + y) * nh + g * G + hh) * splits + s) * 66;
    if (lane == 0) {
      pp[0] = m;
      pp[1] = l;
    }
    pp[2 + lane] = acc;
  }
}

// One wave per query head: M = max m_s; w_s = exp(m_s - M); den = fma chain of w_s * l_s; num_c = fma chain of
// w_s * acc_sc, both over s = 0..used-1 in order; out_c = num_c / den. used <= splits <= 64.
template <int SP>
__global__ __launch_bounds__(64) void k_attn_combine(const float* __restrict__ part, const int* __restrict__ lenp,
                                                    int len_add, int tps, int splits, float* __restrict__ out, Tl tl) {
  TL_START(tl);
  __shared__ float Cw[2][64];
  const int h = blockIdx.x, lane = threadIdx.x;
  const float NEG_INF = __int_as_float(0xff800000);
  part += (size_t)blockIdx.y * gridDim.x * splits * 66;  // position blockIdx.y of a multi-position step
  out += (size_t)blockIdx.y * gridDim.x * 64;
  len_add += blockIdx.y;
  const float* base = part + (size_t)h * splits * 66;
  // every split's partial is requested before the length (and so the number of used splits) is known; indices
  // are clamped instead of guarded (SP >= splits), so the loads form one straight run
  float av[SP];
#pragma unroll
  for (int s2 = 0; s2 < SP; s2++) av[s2] = base[(size_t)min(s2, splits - 1) * 66 + 2 + lane];
  const int sl = min(lane, splits - 1);
  float ms = base[(size_t)sl * 66];
  float ls = base[(size_t)sl * 66 + 1];
  const int len = *lenp + len_add;
  const int nb = (len + 63) / 64, used = (nb + tps - 1) / tps;
  if (lane >= used) {
    ms = NEG_INF;
    ls = 0.0f;
  }
  const float M = group_max<64>(ms);
  TL_PHASE(tl, 2);
  Cw[0][lane] = lane < used ? dexp(ms - M) : 0.0f;
  Cw[1][lane] = ls;
  wave_lds_sync();
  float den = 0.0f, num = 0.0f;
#pragma unroll
  for (int s2 = 0; s2 < SP; s2++) {
    if (s2 < used) {
      const float ws = Cw[0][s2];
      den = __builtin_fmaf(ws, Cw[1][s2], den);
      num = __builtin_fmaf(ws, av[s2], num);
    }
  }
  out[h * 64 + lane] = num / den;
  TL_END(tl);
}

// ------------------------------------------------------------------------------------------------------------
// Output projection with the residual in the epilogue: h[r] = h[r] + res * (Wo att)[r] (gemv o + axpby,
// gpu_model.rs:386-394; model.rs:224-227). The epilogue also writes the MoE-norm partials of the workgroup's rows
// (moe_norm.h: the router dots and the sum of squares of its 8-row blocks of the new h) for the router kernel; the
// router has the output projection's dtype DT.
template <int DT, int K, int P>
__global__ __launch_bounds__(kBlock) void k_oproj(DMat m, const float* __restrict__ att, float res,
                                                  const float* hin, float* __restrict__ h, DMat router,
                                                  const float* __restrict__ lnw, float* __restrict__ zp, Tl tl) {
  TL_START(tl);
  using G = Geo<DT, K>;
  constexpr int RB = kWavesPerBlock * P * G::RPW;  // rows of the workgroup: [r0, r0 + RB)
  static_assert(RB % kNormBlk == 0, "the workgroup's rows must be whole partial blocks");
  __shared__ float xs[K];
  __shared__ float hn[RB];
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  const int r0 = blockIdx.x * RB;
  size_t base = ((size_t)blockIdx.x * kWavesPerBlock + wave) * (P * G::RPW);
  size_t row[P];
  bool ok[P];
#pragma unroll
  for (int p = 0; p < P; p++) {
    row[p] = base + (size_t)p * G::RPW + rw;
    ok[p] = row[p] < (size_t)m.rows;
  }
  CopyIn<K, kBlock> ain;
  copy_fetch<K, kBlock>(att, ain);
  float hold[P];
#pragma unroll
  for (int p = 0; p < P; p++) hold[p] = hin[ok[p] ? row[p] : 0];  // clamped, not guarded: no branch in the load run
  Rows<DT, K, P> rr;
  rows_load<DT, K, P>(rr, m, row, ok, sub);
  copy_finish<K, kBlock>(ain, xs);
  // the router columns and norm weights of the epilogue after the activation has arrived: loads complete in issue
  // order, so they must not sit in front of it (they arrive with the weight rows, before the epilogue)
  NormPart<RB, kBlock> np;
  norm_part_fetch<DT, RB, kBlock>(router, lnw, r0, m.rows, np);
  TL_PHASE(tl, 2);
  XReg<DT, K> xr;
  load_x<DT, K>(xr, xs, sub);
  float out[P];
  rows_fma<DT, K, P>(rr, ok, xr, sub, out);
  TL_PHASE(tl, 3);
#pragma unroll
  for (int p = 0; p < P; p++)
    if (ok[p] && sub == 0) {
      const float hv = hold[p] + res * out[p];
      h[row[p]] = hv;
      hn[row[p] - r0] = hv;
    }
  __syncthreads();
  norm_part_finish<DT, RB, kBlock>(np, hn, router.rows, r0, m.rows, zp);
  TL_END(tl);
}

// ------------------------------------------------------------------------------------------------------------
// Router and gate/up of the routed experts in one kernel. Every workgroup computes the router itself (its 40-65 KB
// of weights stay in L2 after the first read): xn = rmsnorm(h) (or h as is), logits = Wr xn (+ bias), top-k and the
// softmax weights (forward_cpu's router, block.rs:56-62; gemv + route_topk, cuda_backend.rs:804-835); workgroup 0
// publishes ids/weights for the down kernel. Then its pairs (slot j, row r): act[j, r] = silu(gate_r . xn) *
// (up_r . xn) for expert ids[j] (gemv_swiglu gpu.rs:46-74, grouped as moe_gate_up hits.rs:67-105; Cpu::experts
// cpu.rs:116-137). E <= 64, k <= 8.
// Waves per workgroup: 16 (4 per SIMD, so that the router's FMA chains of the 4 waves of a SIMD interleave); 8 for
// f32 rows, whose registers would not fit 16 waves. Rows per wave (NP pairs) make 16 pairs per workgroup either way.
__host__ __device__ constexpr int route_waves(int dt) { return dt == DT_F32 ? 8 : 16; }
__host__ __device__ constexpr int route_np(int dt) { return 16 / route_waves(dt); }

// CACHED (expert-cache path): after the top-k, wave 0 of every workgroup makes the layer step's LRU decision from
// the current copy of the slot tables (all workgroups read the same copy, so they all decide alike); workgroup 0
// writes the updated tables into the other copy, the counters and the routed slots for the down kernel. Rows of a
// routed expert come from its pool slot, or, when it missed, from its record in the host store; those rows are also
// written into the slot.
template <int DT, int K, int NP, bool PART, bool CACHED>
__global__ __launch_bounds__(route_waves(DT) * 64) void k_route_up(DMat router, const float* __restrict__ bias, DMat gu,
                                                               const float* __restrict__ h,
                                                               const float* __restrict__ lnw, float eps,
                                                               const float* __restrict__ zp, int k, int inter,
                                                               int layer, int* __restrict__ ids_out,
                                                               float* __restrict__ w_out, float* __restrict__ act,
                                                               CacheDev c, Tl tl) {
  TL_START(tl);
  using G = Geo<DT, K>;
  constexpr int NW = route_waves(DT);
  constexpr int NT = NW * 64;
  constexpr int RP = PART ? 1 : (64 + NW * G::RPW - 1) / (NW * G::RPW);  // router passes for 64 rows
  constexpr int P = 2 * NP;
  constexpr int SMAX = CACHED ? kCacheMaxSlots : 1;
  __shared__ float xs[K];
  __shared__ __align__(16) float lg[64];
  __shared__ int part[NW][64];
  __shared__ int skey[SMAX];
  __shared__ int slast[SMAX];
  __shared__ int lslot[8], lmiss[8], lfound[8];
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  const int E = router.rows;
  XReg<DT, K> xr;
  if (PART) {
    // Model step: the rmsnorm and the router from the MoE-norm partials of the output projection (moe_norm.h).
    // Loads first: the sum-of-squares partials (every wave forms r itself), this wave's router items and their
    // bias, this thread's elements of h and of the norm weights, the slot tables.
    constexpr int IPW = (64 + NW - 1) / NW;  // router items per wave
    constexpr int XP = (K + NT - 1) / NT;    // elements of h per thread
    const int nb = K / kNormBlk;
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
      hv[e] = h[ic];
      wv[e] = lnw[ic];
    }
    __builtin_amdgcn_sched_barrier(0);
    if (CACHED) {
      const int cur = *c.cur, S = c.slots;
      for (int i = threadIdx.x; i < S; i += NT) {
        skey[i] = c.slot_key[cur * S + i];
        slast[i] = c.slot_last[cur * S + i];
      }
    }
    const float ss = norm_item_sum(ssi, nb, lane);
    const float r = 1.0f / sqrtf(ss / (float)K + eps);
    TL_PHASE(tl, 2);
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
      if (i < K) xs[i] = wv[e] * (hv[e] * r);
    }
  } else {
    // Standalone block: x is the already normalised input; the router's dots in the canonical order.
    CopyIn<K, NT> cin;
    copy_fetch<K, NT>(h, cin);
    size_t row[RP];
    bool ok[RP];
#pragma unroll
    for (int p = 0; p < RP; p++) {
      row[p] = (size_t)(p * NW + wave) * G::RPW + rw;
      ok[p] = row[p] < (size_t)E;
    }
    Rows<DT, K, RP> rr;
    rows_load<DT, K, RP>(rr, router, row, ok, sub);
    float bv[RP];
#pragma unroll
    for (int p = 0; p < RP; p++) bv[p] = bias ? bias[ok[p] ? row[p] : 0] : 0.0f;  // clamped, not guarded: one run of loads
    copy_finish<K, NT>(cin, xs);
    TL_PHASE(tl, 2);
    load_x<DT, K>(xr, xs, sub);
    float out[RP];
    rows_fma<DT, K, RP>(rr, ok, xr, sub, out);
#pragma unroll
    for (int p = 0; p < RP; p++)
      if (ok[p] && sub == 0) lg[row[p]] = bias ? out[p] + bv[p] : out[p];
  }
  __syncthreads();
  TL_PHASE(tl, 3);
  // routed ids as wave-uniform values, ranked by all waves
  int eid[8];
  const int rank = wg_rank<NW>(lg, E, lane, wave, part);
  const bool sel = lane < E && rank < k;
  ids_by_rank(sel, rank, k, eid);
  TL_PHASE(tl, 4);
  if (blockIdx.x == 0 && wave == 0) route_weights(lg, sel, rank, k, lane, eid, ids_out, w_out);
  // expert-cache path: slots of the routed experts (eid becomes slot ids) and the keys of the misses
  int mk[8];
#pragma unroll
  for (int r = 0; r < 8; r++) mk[r] = -1;
  if (CACHED && c.table) {
    // hybrid: the slot of each routed expert from the token's table; an expert without one is computed on the host
    int e = 0;
#pragma unroll
    for (int r = 0; r < 8; r++) e = lane == r ? eid[r] : e;
    if (wave == 0 && lane < k) lslot[lane] = c.table[layer * c.experts + e];
    if (blockIdx.x == 0 && wave == 0 && lane < k) {
      c.route[lane] = lslot[lane];
      c.route[8 + lane] = -1;
    }
    if (blockIdx.x == 0)
      for (int i = threadIdx.x; i < K; i += NT) c.xn[i] = xs[i];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 8; r++) eid[r] = r < k ? lslot[r] : 0;
  } else if (CACHED) {
    const int cur = *c.cur, S = c.slots;
    if (wave == 0) {
      int key = 0;
#pragma unroll
      for (int r = 0; r < 8; r++) key = lane == r ? layer * c.experts + eid[r] : key;
      const int clock = c.clock[cur] + 1;
      int slot, miss_key, hits, misses;
      lru_decide(skey, slast, lfound, S, clock, k, lane, key, slot, miss_key, hits, misses);
      if (lane < k) {
        lslot[lane] = slot;
        lmiss[lane] = miss_key;
      }
      if (blockIdx.x == 0) {
        if (lane < k) {
          c.route[lane] = slot;
          c.route[8 + lane] = miss_key;
        }
        if (lane == 0) {
          c.clock[cur ^ 1] = clock;
          c.stats[CS_HITS] += (unsigned long long)hits;
          c.stats[CS_COPIES] += (unsigned long long)misses;
          int* th = c.tok_hist + ((size_t)c.state[ST_POS] * c.layers + layer) * 4;
          th[0] = hits;
          th[1] = misses;
        }
      }
    }
    __syncthreads();
    if (blockIdx.x == 0)
      for (int i = threadIdx.x; i < S; i += NT) {
        c.slot_key[(cur ^ 1) * S + i] = skey[i];
        c.slot_last[(cur ^ 1) * S + i] = slast[i];
      }
#pragma unroll
    for (int r = 0; r < 8; r++) {
      eid[r] = r < k ? lslot[r] : 0;
      mk[r] = r < k ? lmiss[r] : -1;
    }
  }
  const int npairs = k * inter;
  const int wbase = (blockIdx.x * NW + wave) * (NP * G::RPW);
  size_t row[P], prow[P];
  bool ok[P], put[P];
  DMat src[P];
  int gp[NP];
#pragma unroll
  for (int a = 0; a < NP; a++) {
    gp[a] = wbase + a * G::RPW + rw;
    bool v = gp[a] < npairs;
    int j = v ? gp[a] / inter : 0, r = gp[a] % inter;
    int ej = eid[0], mj = mk[0];
#pragma unroll
    for (int q = 1; q < 8; q++) {
      ej = j == q ? eid[q] : ej;
      mj = j == q ? mk[q] : mj;
    }
    if (CACHED && ej < 0) v = false;  // hybrid: an expert the host computes
    size_t r0 = (size_t)ej * 2 * inter;
    src[2 * a] = src[2 * a + 1] = CACHED ? expert_source(c, 0, ej, mj, r0) : gu;
    row[2 * a] = r0 + r;
    row[2 * a + 1] = r0 + inter + r;
    prow[2 * a] = (size_t)ej * 2 * inter + r;
    prow[2 * a + 1] = prow[2 * a] + inter;
    ok[2 * a] = v;
    ok[2 * a + 1] = v;
    put[2 * a] = put[2 * a + 1] = CACHED && v && mj >= 0;
  }
  Rows<DT, K, P> rr;
  if (CACHED)
    rows_load_from<DT, K, P>(rr, src, row, ok, sub);
  else
    rows_load<DT, K, P>(rr, gu, row, ok, sub);
  if (PART) load_x<DT, K>(xr, xs, sub);  // the normalised input, staged before the rank's barrier
  float out[P];
  rows_fma<DT, K, P>(rr, ok, xr, sub, out);
  TL_PHASE(tl, 5);
  if (CACHED) rows_store<DT, K, P>(rr, c.pool_gu, prow, put, sub);  // a missed expert's rows into its slot
  if (sub != 0) return;
#pragma unroll
  for (int a = 0; a < NP; a++)
    if (ok[2 * a]) act[gp[a]] = silu_mul(out[2 * a], out[2 * a + 1]);
  TL_END(tl);
}

// Down rows of the k routed experts, combined in top-k order, residual in the epilogue:
// h[r] = h[r] + res * sum_j w_j * (down_{ids[j]}[r] . act_j) (gemv_axpby gpu.rs:80-103 / moe_down hits.rs:109-148;
// Cpu::experts cpu.rs:138-148). One output row per wave; expert slot j = pass * RPW + group.
// CACHED: expert j's rows come from pool slot c.route[j], or, when it missed, from its record c.route[8 + j] in the
// host store (and are written into the slot); workgroup 0 then makes the other copy of the slot tables current.
template <int DT, int K, bool CACHED>
__global__ __launch_bounds__(kBlock) void k_expert_down(DMat m, const float* __restrict__ act,
                                                        const int* __restrict__ ids, const float* __restrict__ wts,
                                                        int k, int hidden, float res, bool accumulate,
                                                        float* __restrict__ h, CacheDev c, Tl tl) {
  TL_START(tl);
  using G = Geo<DT, K>;
  constexpr int KMAX = 8;
  constexpr int KP = (KMAX + G::RPW - 1) / G::RPW;
  __shared__ float xs[KMAX * K];
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  int r = blockIdx.x * kWavesPerBlock + wave;
  bool rok = r < hidden;
  // routed ids, then activations (loads complete in issue order, so waiting for the ids does not wait for the
  // activations), then the expert rows, then the activations into LDS
  int idj[KP], mkj[KP];
#pragma unroll
  for (int p = 0; p < KP; p++) {
    const int j = p * G::RPW + rw;
    idj[p] = CACHED ? c.route[j < k ? j : 0] : ids[j < k ? j : 0];
    mkj[p] = CACHED ? c.route[8 + (j < k ? j : 0)] : -1;
  }
  constexpr int AP = (KMAX * K / 4 + kBlock - 1) / kBlock;
  float4 av[AP];
#pragma unroll
  for (int q = 0; q < AP; q++) {
    const int i = threadIdx.x + q * kBlock;
    av[q] = reinterpret_cast<const float4*>(act)[i < k * K / 4 ? i : 0];
  }
  float hold = (rok && lane == 0 && accumulate) ? h[r] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);  // ids and activations ahead of the expert rows
  Rows<DT, K, KP> rows;
  size_t srow[KP], prow[KP];
  bool all[KP], put[KP];
  DMat src[KP];
#pragma unroll
  for (int p = 0; p < KP; p++) {
    const int sl = CACHED && idj[p] < 0 ? 0 : idj[p];  // hybrid: an expert the host computes (rows unused)
    size_t r0 = (size_t)sl * hidden;
    src[p] = CACHED ? expert_source(c, 1, sl, mkj[p], r0) : m;
    srow[p] = r0 + (rok ? r : 0);
    prow[p] = (size_t)sl * hidden + (rok ? r : 0);
    all[p] = true;
    put[p] = CACHED && rok && mkj[p] >= 0 && p * G::RPW + rw < k;
  }
  rows_load_from<DT, K, KP>(rows, src, srow, all, sub);
#pragma unroll
  for (int q = 0; q < AP; q++) {
    // unconditional store (past the end: act[0..3] again, where thread 0 writes it), so that the activation
    // loads stay ahead of the expert rows instead of being sunk into a branch below them
    const int i = threadIdx.x + q * kBlock;
    reinterpret_cast<float4*>(xs)[i < k * K / 4 ? i : 0] = av[q];
  }
  __syncthreads();
  TL_PHASE(tl, 2);
  if (CACHED) {
    if (blockIdx.x == 0 && threadIdx.x == 0) *c.cur ^= 1;
    rows_store<DT, K, KP>(rows, c.pool_dn, prow, put, sub);  // a missed expert's rows into its slot
  }
  if (!rok) {
    TL_END(tl);
    return;
  }
  float dsum[KP];
#pragma unroll
  for (int p = 0; p < KP; p++) {
    int j = p * G::RPW + rw;
    float acc = 0.0f;
    if (j < k && (!CACHED || idj[p] >= 0)) {
      XReg<DT, K> xr;
      load_x<DT, K>(xr, xs + (size_t)j * K, sub);
#pragma unroll
      for (int jj = 0; jj < G::NJ; jj++) {
        int ch = sub + G::LPR * jj;
        if (ch < G::NCH) acc = fma_chunk<DT>(rows.c[p][jj], xr.v[jj], acc);
      }
    }
    dsum[p] = group_sum<G::LPR>(acc);
  }
  TL_PHASE(tl, 3);
  float y = 0.0f;
#pragma unroll
  for (int p = 0; p < KP; p++) {
#pragma unroll
    for (int g2 = 0; g2 < G::RPW; g2++) {
      int j = p * G::RPW + g2;
      float dj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dsum[p]), g2 * G::LPR));
      const bool live = !CACHED || __builtin_amdgcn_readlane(idj[p], g2 * G::LPR) >= 0;
      if (j < k && live) y = y + wts[j] * dj;
    }
  }
  if (lane == 0) h[r] = accumulate ? hold + res * y : y;
  TL_END(tl);
}

// ------------------------------------------------------------------------------------------------------------
// Final rmsnorm, tied LM head, division by logits_scaling, and greedy argmax (last index on ties): each block
// reduces its rows, the last block to arrive reduces the blocks, records the token and advances the position
// (final rmsnorm + gemv, gpu_model.rs:414-439; argmax, bin/m1b-gulosa.rs:22-24).
__device__ __forceinline__ bool later_better(int ak, int ai, int bk, int bi) { return ak > bk || (ak == bk && ai > bi); }

template <int S>
__device__ __forceinline__ void argmax_stage(int& bk, int& bi) {
  int ok_ = partner<S>(bk), oi = partner<S>(bi);
  if (later_better(ok_, oi, bk, bi)) {
    bk = ok_;
    bi = oi;
  }
}

// (key, index) maximum over the wave, the later index winning ties (max_by keeps the last maximum).
__device__ __forceinline__ void wave_argmax(int& bk, int& bi) {
  argmax_stage<1>(bk, bi);
  argmax_stage<2>(bk, bi);
  argmax_stage<4>(bk, bi);
  argmax_stage<8>(bk, bi);
  argmax_stage<16>(bk, bi);
  argmax_stage<32>(bk, bi);
}

// The rows are cut into slots of RPW rows (one pass of a wave) and the slots are dealt out to the grid's waves in
// contiguous runs, as evenly as possible (the first S % W waves take one more): with at most as many workgroups as
// are resident at once, 49155 rows on 3072 waves is 16 slots each and 17 for three waves, instead of a workgroup
// waiting for a free compute unit. A wave streams its run in batches of P slots, the next batch's loads issued
// before the current batch's arithmetic.
// One workgroup of NT threads per compute unit: its activation loads are the first requests of the compute unit
// (every wave's, ahead of any row, through a bare barrier), so the norm completes at once instead of behind the rows
// of other workgroups on the same compute unit.
template <int DT, int K, int P, int NT>
__global__ __launch_bounds__(NT) void k_head(DMat m, const float* __restrict__ h, const float* __restrict__ lnw,
                                             float eps, float ls, float* __restrict__ logits,
                                             int2* __restrict__ best, Tl tl) {
  TL_START(tl);
  using G = Geo<DT, K>;
  constexpr int NWB = NT / kWave;
  __shared__ float xs[K];
  __shared__ float rs;
  __shared__ int sk[NWB], si[NWB];
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int sub = lane % G::LPR, rw = lane / G::LPR;
  const int slots = (m.rows + G::RPW - 1) / G::RPW, waves = gridDim.x * NWB;
  const int wv = blockIdx.x * NWB + wave;
  const int base = slots / waves, extra = slots % waves;
  const int s0 = wv * base + min(wv, extra), ns = base + (wv < extra ? 1 : 0);
  const int nbat = (ns + P - 1) / P;
  size_t row[P];
  bool ok[P];
  auto batch_rows = [&](int bt) {
#pragma unroll
    for (int p = 0; p < P; p++) {
      row[p] = (size_t)(s0 + bt * P + p) * G::RPW + rw;
      ok[p] = bt * P + p < ns && row[p] < (size_t)m.rows;
    }
  };
  batch_rows(0);
  NormIn<K, NT> hin;
  norm_fetch<K, NT>(h, lnw, hin);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  Rows<DT, K, P> cur, nxt;
  rows_load<DT, K, P>(cur, m, row, ok, sub);
  norm_finish<K, NT>(hin, eps, xs, &rs);
  TL_PHASE(tl, 2);
  XReg<DT, K> xr;
  load_x<DT, K>(xr, xs, sub);
  int bk = INT_MIN, bi = -1;
  for (int bt = 0; bt < nbat; bt++) {
    size_t rcur[P];
    bool ocur[P];
#pragma unroll
    for (int p = 0; p < P; p++) {
      rcur[p] = row[p];
      ocur[p] = ok[p];
    }
    if (bt + 1 < nbat) {
      batch_rows(bt + 1);
      rows_load<DT, K, P>(nxt, m, row, ok, sub);
    }
    float out[P];
    rows_fma<DT, K, P>(cur, ocur, xr, sub, out);
#pragma unroll
    for (int p = 0; p < P; p++) {
      if (ocur[p]) {
        float v = out[p] / ls;
        if (sub == 0) logits[rcur[p]] = v;
        int kk = total_key(v);
        if (later_better(kk, (int)rcur[p], bk, bi)) {
          bk = kk;
          bi = (int)rcur[p];
        }
      }
    }
    cur = nxt;
  }
  wave_argmax(bk, bi);
  if (lane == 0) {
    sk[wave] = bk;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < NWB; w++)
      if (later_better(sk[w], si[w], bk, bi)) {
        bk = sk[w];
        bi = si[w];
      }
    best[blockIdx.x] = make_int2(bk, bi);
  }
  TL_END(tl);
}

// Greedy token from the per-block maxima of k_head (one block); records it, feeds it to the next position unless
// that position holds a forced prompt token, and advances the position.
__global__ __launch_bounds__(kBlock) void k_head_argmax(const int2* __restrict__ best, int nblocks,
                                                        int* __restrict__ st, int* __restrict__ seq,
                                                        int* __restrict__ hist, int max_len, Tl tl) {
  TL_START(tl);
  __shared__ int sk[kWavesPerBlock], si[kWavesPerBlock];
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int bk = INT_MIN, bi = -1;
  for (int i = threadIdx.x; i < nblocks; i += kBlock) {
    int2 c = best[i];
    if (later_better(c.x, c.y, bk, bi)) {
      bk = c.x;
      bi = c.y;
    }
  }
  wave_argmax(bk, bi);
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
  }
  TL_END(tl);
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
  __shared__ __align__(16) float lg[64];
  __shared__ __align__(16) TopkLds tk;
  int lane = threadIdx.x;
  if (lane < n) lg[lane] = bias ? logits[lane] + bias[lane] : logits[lane];
  wave_lds_sync();
  wave_topk(lg, n, k, lane, tk, ids, w);
}

__global__ __launch_bounds__(kBlock) void k_argmax(const float* __restrict__ v, int n, int2* __restrict__ best) {
  __shared__ int sk[kWavesPerBlock], si[kWavesPerBlock];
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int bk = INT_MIN, bi = -1;
  for (int i = blockIdx.x * kBlock + threadIdx.x; i < n; i += gridDim.x * kBlock) {
    int kk = total_key(v[i]);
    if (later_better(kk, i, bk, bi)) {
      bk = kk;
      bi = i;
    }
  }
  wave_argmax(bk, bi);
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
}

__global__ void k_argmax_final(const int2* __restrict__ best, int nblocks, int* __restrict__ outp) {
  int bk = INT_MIN, bi = -1;
  for (int i = threadIdx.x; i < nblocks; i += 64) {
    int2 c = best[i];
    if (later_better(c.x, c.y, bk, bi)) {
      bk = c.x;
      bi = c.y;
    }
  }
  wave_argmax(bk, bi);
  if (threadIdx.x == 0) *outp = bi < 0 ? 0 : bi;
}

__global__ void k_exp(const float* __restrict__ x, float* __restrict__ y, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = dexp(x[i]);
}

// ------------------------------------------------------------------------------------------------------------
// Launchers. Row lengths are compile-time; the switch covers the shapes of the Granite-MoE family and the small
// test models.

template <int DT, int K, int P>
constexpr int rows_per_block() { return kWavesPerBlock * P * Geo<DT, K>::RPW; }

static inline int cdiv(long a, long b) { return (int)((a + b - 1) / b); }

constexpr int kGemvP = 4;
constexpr int kQkvNP = 1;
constexpr int kHeadP = 4;
constexpr int kOprojP = 2;

hipError_t launch_gemv(hipStream_t s, const DMat& w, const float* x, float* y) {
#define BODY(KK)                                                                                    \
  case KK: {                                                                                        \
    constexpr int RB = rows_per_block<DTC, KK, kGemvP>();                                           \
    klaunch(k_gemv<DTC, KK, kGemvP>, cdiv(w.rows, RB), kBlock, 0, s, w, x, y);                           \
  } break;
  MOERT_DISPATCH(w.dtype, w.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_embed(hipStream_t s, const DMat& emb, const Dims& d, const StepBufs& b, unsigned* step_ctr,
                        float* rope_cur, Tl tl) {
  if (rope_cur && d.head_dim != 64) return hipErrorInvalidValue;
#define EMB(DD) klaunch(k_embed<DD>, 1, kBlock, 0, s, emb, b.seq, b.state, d.emb_mult, b.h, step_ctr, b.rope, rope_cur, tl)
  switch (emb.dtype) {
    case DT_Q8_0: EMB(DT_Q8_0); break;
    case DT_Q4_0: EMB(DT_Q4_0); break;
    case DT_F32: EMB(DT_F32); break;
    default: return hipErrorInvalidValue;
  }
#undef EMB
  return hipGetLastError();
}

hipError_t launch_qkv(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, Tl tl) {
#define BODY(KK)                                                                                            \
  case KK: {                                                                                                \
    constexpr int PB = kQkvWaves * kQkvNP * Geo<DTC, KK>::RPW; /* pairs per block */                   \
    klaunch(k_qkv<DTC, KK, kQkvNP>, cdiv(L.qkv.rows / 2, PB), kQkvWaves * 64, 0, s,                                      \
        L.qkv, b.h, L.ln_attn, d.eps, b.state, b.rope, d.heads, d.kv_heads, d.max_len, b.q, L.k_cache,      \
        L.v_cache, tl);                                                                                     \
  } break;
  MOERT_DISPATCH(L.qkv.dtype, L.qkv.cols, BODY)
#undef BODY
  return hipGetLastError();
}

int attn_splits_for(int max_len, int tps) { return ((max_len + 63) / 64 + tps - 1) / tps; }

static hipError_t attn_split_dispatch(hipStream_t s, int G, int kvh, int tps, const float* q, const uint16_t* kc,
                                      const uint16_t* vc, const int* lenp, int len_add, int max_len, float scale,
                                      float* part, int ny = 1, Tl tl = {}) {
  const int splits = attn_splits_for(max_len, tps);
  if (splits > 64 || max_len % 64 || ny < 1) return hipErrorInvalidValue;
  const dim3 blocks(kvh * splits, ny);
#define TILES_CASE(GG, TT)                                                                                   \
  if (G == GG && tps == TT) {                                                                                \
    klaunch(k_attn_tiles<GG, TT>, blocks, GG * TT * 64, 0, s, q, kc, vc, lenp, len_add, max_len, scale, splits, part, tl); \
    return hipGetLastError();                                                                                \
  }
  TILES_CASE(1, 1) TILES_CASE(2, 1) TILES_CASE(3, 1) TILES_CASE(4, 1)
  TILES_CASE(1, 2) TILES_CASE(2, 2) TILES_CASE(3, 2) TILES_CASE(4, 2)
  TILES_CASE(1, 3) TILES_CASE(2, 3) TILES_CASE(3, 3) TILES_CASE(4, 3)
  TILES_CASE(1, 4) TILES_CASE(2, 4) TILES_CASE(3, 4) TILES_CASE(4, 4)
#undef TILES_CASE
  switch (G) {
    case 1: klaunch(k_attn_split<1>, blocks, 64, 0, s, q, kc, vc, lenp, len_add, max_len, scale, tps, splits, part); break;
    case 2: klaunch(k_attn_split<2>, blocks, 128, 0, s, q, kc, vc, lenp, len_add, max_len, scale, tps, splits, part); break;
    case 3: klaunch(k_attn_split<3>, blocks, 192, 0, s, q, kc, vc, lenp, len_add, max_len, scale, tps, splits, part); break;
    case 4: klaunch(k_attn_split<4>, blocks, 256, 0, s, q, kc, vc, lenp, len_add, max_len, scale, tps, splits, part); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

static hipError_t attn_combine_dispatch(hipStream_t s, int heads, int tps, int max_len, const int* lenp, int len_add,
                                        const float* part, float* out, int ny = 1, Tl tl = {}) {
  const int splits = attn_splits_for(max_len, tps);
  if (splits > 64 || max_len % 64 || ny < 1) return hipErrorInvalidValue;
  const dim3 grid(heads, ny);
  if (splits <= 8)
    klaunch(k_attn_combine<8>, grid, 64, 0, s, part, lenp, len_add, tps, splits, out, tl);
  else if (splits <= 16)
    klaunch(k_attn_combine<16>, grid, 64, 0, s, part, lenp, len_add, tps, splits, out, tl);
  else if (splits <= 32)
    klaunch(k_attn_combine<32>, grid, 64, 0, s, part, lenp, len_add, tps, splits, out, tl);
  else
    klaunch(k_attn_combine<64>, grid, 64, 0, s, part, lenp, len_add, tps, splits, out, tl);
  return hipGetLastError();
}

// Positions per workgroup of k_attn_mq: at most kMqMaxPos, and fewer when that brings the grid to about five
// workgroups per compute unit (the LDS and register footprint allows five: 15 waves).
static int mq_positions(int ny, int wgs) {
  const int groups = std::min(ny, std::max(cdiv(ny, kMqMaxPos), cdiv(1280, wgs)));
  return cdiv(ny, groups);
}

static bool attn_mq_dispatch(hipStream_t s, int G, int kvh, int tps, const float* q, const uint16_t* kc,
                             const uint16_t* vc, const int* lenp, int len_add, int max_len, float scale, int ny,
                             float* part) {
  const int splits = attn_splits_for(max_len, tps);
  if (G > 4 || tps > 4 || ny < 1 || splits > 64 || max_len % 64) return false;
  const int npw = mq_positions(ny, kvh * splits);
  const dim3 blocks(kvh * splits, cdiv(ny, npw));
#define MQ_CASE(GG, TT)                                                                                           \
  if (G == GG && tps == TT) {                                                                                     \
    klaunch(k_attn_mq<GG, TT>, blocks, TT * 64, 0, s, q, kc, vc, lenp, len_add, max_len, scale, splits, ny,      \
            npw, part);                                                                                           \
    return true;                                                                                                  \
  }
  MQ_CASE(1, 1) MQ_CASE(2, 1) MQ_CASE(3, 1) MQ_CASE(4, 1)
  MQ_CASE(1, 2) MQ_CASE(2, 2) MQ_CASE(3, 2) MQ_CASE(4, 2)
  MQ_CASE(1, 3) MQ_CASE(2, 3) MQ_CASE(3, 3) MQ_CASE(4, 3)
  MQ_CASE(1, 4) MQ_CASE(2, 4) MQ_CASE(3, 4) MQ_CASE(4, 4)
#undef MQ_CASE
  return false;
}

hipError_t launch_attn_batched(hipStream_t s, const LayerDev& L, const Dims& d, const int* lenp, int len_add, int ny,
                               const float* q, float* part, float* att) {
  hipError_t e = hipSuccess;
  if (attn_mq_dispatch(s, d.heads / d.kv_heads, d.kv_heads, d.tps, q, L.k_cache, L.v_cache, lenp, len_add,
                       d.max_len, d.attn_mult, ny, part))
    e = hipGetLastError();
  else
    e = attn_split_dispatch(s, d.heads / d.kv_heads, d.kv_heads, d.tps, q, L.k_cache, L.v_cache, lenp, len_add,
                            d.max_len, d.attn_mult, part, ny);
  if (e != hipSuccess) return e;
  return attn_combine_dispatch(s, d.heads, d.tps, d.max_len, lenp, len_add, part, att, ny);
}

hipError_t launch_attn_split(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, Tl tl) {
  return attn_split_dispatch(s, d.heads / d.kv_heads, d.kv_heads, d.tps, b.q, L.k_cache, L.v_cache, b.state + ST_POS,
                             1, d.max_len, d.attn_mult, b.part, 1, tl);
}

hipError_t launch_attn_combine(hipStream_t s, const Dims& d, const StepBufs& b, Tl tl) {
  return attn_combine_dispatch(s, d.heads, d.tps, d.max_len, b.state + ST_POS, 1, b.part, b.att, 1, tl);
}

hipError_t launch_attn_unit(hipStream_t s, const float* q, const uint16_t* kc, const uint16_t* vc, int heads,
                            int kv_heads, int max_len, const int* len_dev, float scale, int tps, float* part,
                            float* out) {
  hipError_t e = attn_split_dispatch(s, heads / kv_heads, kv_heads, tps, q, kc, vc, len_dev, 0, max_len, scale, part);
  if (e != hipSuccess) return e;
  return attn_combine_dispatch(s, heads, tps, max_len, len_dev, 0, part, out);
}

hipError_t launch_oproj(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, Tl tl, bool from_hc) {
  const float* hin = from_hc ? b.hc : b.h;
#define BODY(KK)                                                                            \
  case KK: {                                                                                \
    constexpr int RB = rows_per_block<DTC, KK, kOprojP>();                                  \
    klaunch(k_oproj<DTC, KK, kOprojP>, cdiv(L.o.rows, RB), kBlock, 0, s, L.o, b.att, d.res_mult, hin, b.h,     \
            L.router, L.ln_moe, b.zpart, tl);                                                       \
  } break;
  MOERT_DISPATCH(L.o.dtype, L.o.cols, BODY)
#undef BODY
  return hipGetLastError();
}


hipError_t launch_route_up(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                           bool partials, Tl tl) {
  if (L.router.dtype != L.gate_up.dtype || L.router.cols != L.gate_up.cols) return hipErrorInvalidValue;
  const CacheDev none{};
#define BODY(KK)                                                                                           \
  case KK: {                                                                                               \
    constexpr int NW = route_waves(DTC), NP = route_np(DTC), PB = NW * NP * Geo<DTC, KK>::RPW;             \
    const int blocks = cdiv((long)d.top_k * d.inter, PB);                                                  \
    if (partials)                                                                                          \
      klaunch(k_route_up<DTC, KK, NP, true, false>, blocks, NW * 64, 0, s,                                 \
          L.router, L.router_bias, L.gate_up, b.h, L.ln_moe, d.eps, b.zpart, d.top_k, d.inter, layer,      \
          b.route_ids + layer * d.top_k, b.route_w + layer * d.top_k, b.act, none, tl);                    \
    else                                                                                                   \
      klaunch(k_route_up<DTC, KK, NP, false, false>, blocks, NW * 64, 0, s,                                \
          L.router, L.router_bias, L.gate_up, b.h, L.ln_moe, d.eps, (const float*)nullptr, d.top_k, d.inter, \
          layer, b.route_ids + layer * d.top_k, b.route_w + layer * d.top_k, b.act, none, tl);             \
  } break;
  MOERT_DISPATCH(L.router.dtype, L.router.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_route_up_cached(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                                  const CacheDev& c, Tl tl) {
  if (L.router.dtype != c.pool_gu.dtype || L.router.cols != c.pool_gu.cols || (!c.table && c.slots < d.top_k) ||
      c.slots > kCacheMaxSlots || L.router.rows > 64 || d.top_k > 8)
    return hipErrorInvalidValue;
#define BODY(KK)                                                                                           \
  case KK: {                                                                                               \
    constexpr int NW = route_waves(DTC), NP = route_np(DTC), PB = NW * NP * Geo<DTC, KK>::RPW;             \
    const int blocks = cdiv((long)d.top_k * d.inter, PB);                                                  \
    klaunch(k_route_up<DTC, KK, NP, true, true>, blocks, NW * 64, 0, s, L.router,                          \
            L.router_bias, c.pool_gu, b.h, L.ln_moe, d.eps, b.zpart, d.top_k, d.inter, layer,              \
            b.route_ids + layer * d.top_k, b.route_w + layer * d.top_k, b.act, c, tl);                     \
  } break;
  MOERT_DISPATCH(L.router.dtype, L.router.cols, BODY)
#undef BODY
  return hipGetLastError();
}

#define DOWN_DISPATCH(dt, cols, BODY)                                                                     \
  switch (dt) {                                                                                           \
    case DT_Q8_0: { constexpr int DTC = DT_Q8_0; switch (cols) { MOERT_KDOWN_CASES(BODY) default: return hipErrorInvalidValue; } } break; \
    case DT_Q4_0: { constexpr int DTC = DT_Q4_0; switch (cols) { MOERT_KDOWN_CASES(BODY) default: return hipErrorInvalidValue; } } break; \
    case DT_F32: { constexpr int DTC = DT_F32; switch (cols) { MOERT_KDOWN_CASES(BODY) default: return hipErrorInvalidValue; } } break;   \
    default: return hipErrorInvalidValue;                                                                 \
  }

hipError_t launch_expert_down_cached(hipStream_t s, const Dims& d, const StepBufs& b, int layer, const CacheDev& c,
                                     Tl tl) {
#define BODY(KK)                                                                                          \
  case KK:                                                                                                \
    klaunch(k_expert_down<DTC, KK, true>, cdiv(d.hidden, kWavesPerBlock), kBlock, 0, s, c.pool_dn, b.act,  \
            (const int*)nullptr, b.route_w + layer * d.top_k, d.top_k, d.hidden, d.res_mult, true, b.h, c, tl); \
    break;
  DOWN_DISPATCH(c.pool_dn.dtype, c.pool_dn.cols, BODY)
#undef BODY
  return hipGetLastError();
}

// h[i] += res * y[i] (the host-computed experts of a hybrid layer step, y in mapped host memory)
__global__ __launch_bounds__(256) void k_add_scaled(float* __restrict__ h, const float* __restrict__ y, float res,
                                                    int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) h[i] = h[i] + res * y[i];
}

hipError_t launch_add_scaled(hipStream_t s, float* h, const float* y, float res, int n) {
  klaunch(k_add_scaled, cdiv(n, 256), 256, 0, s, h, y, res, n);
  return hipGetLastError();
}

// The doorbell of a hybrid layer (the reference's stream wait on a host-written value, cuda_backend.rs:919-927):
// thread 0 of each workgroup polls the layer's flag word in coherent host memory until it carries the token's
// sequence number (flag = seq << 1 | any host expert), then h[i] += res * y[i] when the host computed any expert.
// The poll is bounded (kHyDoorbellSpin polls of about a microsecond each, far beyond a layer's host work): a flag
// that never comes sets bit 256 of *err and adds nothing, so the kernel always ends.
constexpr int kHyDoorbellSpin = 1 << 23;
__global__ __launch_bounds__(256) void k_hy_doorbell_add(float* __restrict__ h, const float* __restrict__ y,
                                                         float res, int n, const unsigned* __restrict__ flag,
                                                         unsigned seq, unsigned* __restrict__ err) {
  __shared__ unsigned any_s;
  if (threadIdx.x == 0) {
    unsigned v = 0;
    int it = 0;
    for (; it < kHyDoorbellSpin; it++) {
      v = __hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
      if ((v >> 1) == seq) break;
      __builtin_amdgcn_s_sleep(4);
    }
    if (it == kHyDoorbellSpin) {
      if (blockIdx.x == 0) atomicOr(err, 256u);
      v = 0u;
    }
    any_s = v & 1u;
  }
  __syncthreads();
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (any_s && i < n) h[i] = h[i] + res * __hip_atomic_load(y + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

hipError_t launch_hy_doorbell_add(hipStream_t s, float* h, const float* y, float res, int n, const unsigned* flag,
                                  unsigned seq, unsigned* err) {
  klaunch(k_hy_doorbell_add, cdiv(n, 256), 256, 0, s, h, y, res, n, flag, seq, err);
  return hipGetLastError();
}

hipError_t launch_expert_down(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                              bool accumulate, Tl tl) {
  const CacheDev none{};
#define BODY(KK)                                                                                          \
  case KK:                                                                                                \
    klaunch(k_expert_down<DTC, KK, false>, cdiv(d.hidden, kWavesPerBlock), kBlock, 0, s,                      \
        L.down, b.act, b.route_ids + layer * d.top_k, b.route_w + layer * d.top_k, d.top_k, d.hidden,     \
        d.res_mult, accumulate, accumulate ? b.h : b.logits, none, tl);                                   \
    break;
  DOWN_DISPATCH(L.down.dtype, L.down.cols, BODY)
#undef BODY
  return hipGetLastError();
}
#undef DOWN_DISPATCH

constexpr int kHeadNB = 4;
constexpr int kHeadNT = 768;  // threads of a k_head workgroup

// Rows of the head per workgroup at kHeadNB batches per wave (the grid's upper bound: the rows are then dealt out
// to the resident waves).
static int head_groups(const DMat& head) {
  int ce = head.dtype == DT_Q8_0 ? 16 : head.dtype == DT_Q4_0 ? 32 : 4;
  int rpw = kWave / lanes_per_row(head.cols / ce);
  return cdiv(head.rows, kHeadNT / kWave * kHeadNB * kHeadP * rpw);
}

// Workgroups of k_head<DT, K> resident on the device at once (occupancy x compute units; one per compute unit at
// 768 threads).
template <int DT, int K>
static int head_resident() {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_head<DT, K, kHeadP, kHeadNT>, kHeadNT, 0) != hipSuccess ||
      cus < 1 || per_cu < 1)
    return 1 << 30;  // unknown: the group count alone
  return cus * per_cu;
}

int head_blocks(const DMat& head) {
  int resident = 1 << 30;
#define HB(DTC, KK) \
  case KK:          \
    resident = head_resident<DTC, KK>(); \
    break;
  switch (head.dtype) {
    case DT_Q8_0: switch (head.cols) { HB(DT_Q8_0, 128) HB(DT_Q8_0, 256) HB(DT_Q8_0, 512) HB(DT_Q8_0, 1024) HB(DT_Q8_0, 1536) } break;
    case DT_Q4_0: switch (head.cols) { HB(DT_Q4_0, 128) HB(DT_Q4_0, 256) HB(DT_Q4_0, 512) HB(DT_Q4_0, 1024) HB(DT_Q4_0, 1536) } break;
    case DT_F32: switch (head.cols) { HB(DT_F32, 128) HB(DT_F32, 256) HB(DT_F32, 512) HB(DT_F32, 1024) HB(DT_F32, 1536) } break;
  }
#undef HB
  return std::min(head_groups(head), resident);
}

hipError_t launch_head(hipStream_t s, const DMat& head, const float* norm, const Dims& d, const StepBufs& b, Tl tl) {
  const int grid = head_blocks(head);
#define BODY(KK)                                                                                        \
  case KK:                                                                                              \
    klaunch(k_head<DTC, KK, kHeadP, kHeadNT>, grid, kHeadNT, 0, s, head, b.h, norm, d.eps, d.logits_scaling, b.logits, \
            b.best, tl);                                                                                \
    break;
  MOERT_DISPATCH(head.dtype, head.cols, BODY)
#undef BODY
  return hipGetLastError();
}

hipError_t launch_head_argmax(hipStream_t s, const DMat& head, const Dims& d, const StepBufs& b, Tl tl) {
  klaunch(k_head_argmax, 1, kBlock, 0, s, b.best, head_blocks(head), b.state, b.seq, b.argmax_hist, d.max_len, tl);
  return hipGetLastError();
}

hipError_t launch_dequant(hipStream_t s, const DMat& w, float* out) {
  size_t n;
  switch (w.dtype) {
    case DT_Q8_0: n = (size_t)w.rows * (w.cols / 16); klaunch(k_dequant<DT_Q8_0>, cdiv(n, kBlock), kBlock, 0, s, w, out); break;
    case DT_Q4_0: n = (size_t)w.rows * (w.cols / 32); klaunch(k_dequant<DT_Q4_0>, cdiv(n, kBlock), kBlock, 0, s, w, out); break;
    case DT_F32: n = (size_t)w.rows * (w.cols / 4); klaunch(k_dequant<DT_F32>, cdiv(n, kBlock), kBlock, 0, s, w, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rmsnorm(hipStream_t s, const float* x, const float* w, int n, float eps, float* out) {
  klaunch(k_rmsnorm, 1, 64, 0, s, x, w, n, eps, out);
  return hipGetLastError();
}

hipError_t launch_rope(hipStream_t s, float* x, int heads, int head_dim, const float* cs) {
  int n = heads * head_dim / 2;
  klaunch(k_rope, cdiv(n, 256), 256, 0, s, x, heads, head_dim / 2, cs);
  return hipGetLastError();
}

hipError_t launch_topk(hipStream_t s, const float* logits, const float* bias, int n, int k, int* ids, float* w) {
  klaunch(k_topk, 1, 64, 0, s, logits, bias, n, k, ids, w);
  return hipGetLastError();
}

hipError_t launch_argmax(hipStream_t s, const float* v, int n, int2* best, int* cnt, int* out) {
  int blocks = cdiv(n, kBlock * 4);
  if (blocks > 1024) blocks = 1024;
  if (blocks < 1) blocks = 1;
  (void)cnt;
  klaunch(k_argmax, blocks, kBlock, 0, s, v, n, best);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  klaunch(k_argmax_final, 1, 64, 0, s, best, blocks, out);
  return hipGetLastError();
}

// Plain streaming copy (16 B per lane per iteration): the reference point for achievable HBM bandwidth and for
// scaling the FETCH_SIZE / WRITE_SIZE counters of the other kernels.
__global__ __launch_bounds__(256) void k_copy(const float4* __restrict__ src, float4* __restrict__ dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

hipError_t launch_copy(hipStream_t s, const void* src, void* dst, size_t bytes) {
  const size_t n = bytes / 16;
  const int blocks = (int)std::min<size_t>((n + 255) / 256, 8192);
  klaunch(k_copy, blocks, 256, 0, s, (const float4*)src, (float4*)dst, n);
  return hipGetLastError();
}

// Streaming read of n 16-byte words (four loads in flight per thread and pass), one word of output per thread so
// that the loads are live.
__global__ __launch_bounds__(256) void k_read(const uint4* __restrict__ src, size_t n, unsigned* __restrict__ out) {
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  unsigned acc = 0;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a.x ^ b.y ^ c.z ^ d.w;
  }
  for (; i < n; i += stride) acc ^= src[i].x;
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

int read_probe_blocks(size_t bytes) { return bytes >= ((size_t)256 << 20) ? 256 : 1024; }

hipError_t launch_read(hipStream_t s, const void* src, size_t bytes, unsigned* out) {
  klaunch(k_read, read_probe_blocks(bytes), 256, 0, s, (const uint4*)src, bytes / 16, out);
  return hipGetLastError();
}

hipError_t launch_exp(hipStream_t s, const float* x, float* y, int n) {
  klaunch(k_exp, cdiv(n, 256), 256, 0, s, x, y, n);
  return hipGetLastError();
}

}  // namespace moert

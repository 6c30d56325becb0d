// Attention block of the decode step in one launch: rmsnorm -> [q; k; v] rows -> rotate_half RoPE -> KV append,
// the split-KV GQA attention, and the merge of the splits. It does the work of k_qkv, k_attn_tiles and
// k_attn_combine (kernels.hip) with their operations in their order, so its results are the same bit for bit; the
// reference sequence it replaces is gpu_model.rs:341-384 (rmsnorm, gemv q/k/v, rope_kv, the KV copies,
// attention_b = attn_split + attn_combine, gpu.rs:133-292; paths relative to rust/moe-rt/src).
//
// The chip dispatches the workgroups of a launch to its 8 XCDs in round-robin order, continuing from where the
// previous launch left off: workgroup b runs on XCD (c + b) % 8 for some c. So the workgroups 8s + r (s = 0, 1, ...)
// of one residue r share an XCD, and workgroup b serves KV head g = its XCD (hardware register XCC_ID) and split
// s = b / 8: all workgroups of KV head g run on XCD g and share its L2. They exchange their data through that L2
// (attn_dev.h) as 8-byte entries that carry the launch's epoch beside the value, so a consumer polls exactly the
// entries it needs, and a producer stores and goes on; this costs far less than a kernel boundary:
//   1. the group's q/k/v row pairs ((G + 2) * 32 of them: G query heads, one K and one V head) are dealt out over
//      its splits; each workgroup normalises h, computes its pairs with RoPE, and writes q and the new K/V row into
//      the group's L2 area (and K, V into row `pos` of the cache);
//   2. meanwhile its split's K and V tiles have been loaded and staged in LDS; it polls its queries and (when the
//      split holds position pos) the new K/V row until they carry the epoch, and computes the split's partials
//      (m, l, acc) per query head as k_attn_tiles does, into the group's L2 area;
//   3. workgroup s < G then polls the partials of query head g*G + s over the used splits and merges them as
//      k_attn_combine does, into `att`.
// Every wait is bounded: an entry that does not arrive in time (which is what a dispatch that is not round-robin,
// or a group that is not all resident at once, would cause) sets a bit of `err` and the kernel still ends; the host
// turns a set bit into an error.
#include "attn_dev.h"
#include "cache_pf.h"
#include "dev_rows.h"
#include "kernels.h"
#include "launch.h"
#include "timeline.h"

namespace moert {

namespace {

constexpr int kAbSpin = 1 << 18;  // polls before a wait gives up (each poll is an L2 round trip)

// Wave-level wait until the entry at byte offset off0 of r (and with TWO the one at off1) carries `epoch`, read from
// the XCD's L2; returns the values. Clears *ok when the wait gave up.
template <bool TWO>
__device__ __forceinline__ uint2 poll_entries(__amdgpu_buffer_rsrc_t r, unsigned off0, unsigned off1, unsigned epoch,
                                              int spin, bool* ok) {
  for (int it = 0; it < spin; it++) {
    poll_fence();
    const uint2 a = l2_load_u64(r, off0);
    const uint2 b = TWO ? l2_load_u64(r, off1) : make_uint2(0u, epoch);
    if (__ballot(a.y != epoch || b.y != epoch) == 0) return make_uint2(a.x, b.x);
    __builtin_amdgcn_s_sleep(1);
  }
  *ok = false;
  return make_uint2(0u, 0u);
}

}  // namespace

// CMB: the input is h + res * (sum over j < 8, in order, of yw[j] * ys[j]) (the previous layer's experts left by
// k_moe_xcd; k_expert_down's epilogue arithmetic), and workgroup 0 writes it to hc.
template <int DT, int K, int G, int T, int NP, int SP, bool CMB>
__device__ __forceinline__ void attn_block_body(DMat m, const float* __restrict__ h,
                                                const float* __restrict__ lnw, float eps,
                                                const int* __restrict__ st, const float* __restrict__ rope_cur,
                                                int heads, int max_len, uint16_t* __restrict__ kc,
                                                uint16_t* __restrict__ vc, float scale, int splits, int pp,
                                                AbGroup* __restrict__ xg_all,
                                                const unsigned* __restrict__ step_ctr, unsigned layer,
                                                unsigned* __restrict__ err, float* __restrict__ att,
                                                const float* __restrict__ ys, const float* __restrict__ yw,
                                                float res, float* __restrict__ hc, Tl tl) {
  TL_START(tl);
  using Ge = Geo<DT, K>;
  static_assert(Ge::RPW == 1, "one q/k/v row per wave and pass");
  constexpr int NW = G * T, NT = NW * 64, P = 2 * NP;
  constexpr int TR = 8 % G == 0 ? 64 : 72;  // K tile rows (64..71: padding for VShare when G does not divide 8)
  constexpr int KHS = 72;                    // K row stride in halves: 144-byte rows, conflict-free row reads
  // The K and V tiles stay fp16 in LDS (the FMAs take a half operand exactly, v_fma_mix): K row-major, V transposed
  // (dim-major, VShare::vt_col), so that a lane reads its position's K row and its dim's V column 8 halves at a time.
  __shared__ __align__(16) uint16_t Vt[T][64][64];
  __shared__ __align__(16) uint16_t Kh[T][TR][KHS];
  __shared__ float rs;
  static_assert(T * 64 * 64 / 2 >= K, "the normalised input is staged in the V tiles' LDS");
  float* xs = reinterpret_cast<float*>(&Vt[0][0][0]);  // the normalised input, until the V tiles are staged
  __shared__ __align__(16) float Qs[G][64];
  __shared__ __align__(16) float Ps[G][T][64];
  __shared__ float Pv[G][T][64];
  __shared__ float Tm[G][T], Al[G][T], Ts[G][T];
  __shared__ float Cw[2][64];
  // wid as a wave-uniform value, so that what derives from it (the wave's row pairs, their cos/sin) is scalar
  const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = (int)xcc_id() & 7, s = blockIdx.x >> 3;
  const int wh = wid % G, wt = wid / G;
  AbGroup* xg = xg_all + g;
  uint16_t* Kc = kc + (size_t)g * max_len * 64;
  uint16_t* Vc = vc + (size_t)g * max_len * 64;
  const float NEG_INF = __int_as_float(0xff800000);

  // this wave's q/k/v row pairs: pair l of the group (l = s * pp + wid + NW * a) is row pair (jp, jp + 32) of the
  // group's head l / 32 (query heads g*G .. g*G + G - 1, then K head g, then V head g)
  constexpr int NPAIR = (G + 2) * 32;
  size_t row[P];
  bool ok[P];
  int lh[NP], jp[NP];
#pragma unroll
  for (int a = 0; a < NP; a++) {
    const int li = wid + NW * a, l = s * pp + li;
    const bool v = li < pp && l < NPAIR;
    const int lc = v ? l : 0;
    lh[a] = lc / 32;
    jp[a] = lc % 32;
    const int gh = lh[a] < G ? g * G + lh[a] : lh[a] == G ? heads + g : heads + 8 + g;
    row[2 * a] = (size_t)gh * 64 + jp[a];
    row[2 * a + 1] = row[2 * a] + 32;
    ok[2 * a] = ok[2 * a + 1] = v;
  }
  // The values earlier launches wrote that every wave needs as scalars (the position, the step counter, the
  // previous layer's routing weights) are the first vector loads (lane j: weight j), so waiting for them waits for
  // nothing else (vector loads complete in issue order); read back as scalars after the bulk loads are issued.
  const unsigned pos_v = __builtin_amdgcn_raw_buffer_load_b32(l2_buffer(st, 4 * ST_WORDS), 4 * ST_POS, 0, 0);
  const unsigned sctr_v = __builtin_amdgcn_raw_buffer_load_b32(l2_buffer(step_ctr, 4), 0, 0, 0);
  const auto err_v = __builtin_amdgcn_raw_buffer_load_b64(l2_buffer(err, 8), 0, 0, 0);  // error bits, test mask
  const float yw_v = CMB ? yw[lane & 7] : 0.0f;
  const float rc_v = rope_cur[lane];  // the rope row of the position: cos 0..31, sin 32..63
  __builtin_amdgcn_sched_barrier(0);
  // Vector loads in the order they are needed: the activation, the q/k/v rows, then the split's K and V tiles
  // (used after the first barrier). A compute unit passes requests to its L1 at a fixed rate of bytes, so the
  // activation loads of every wave go first (a bare workgroup barrier orders them before any wave's rows), and a
  // wave whose threads hold no quad of the activation issues none.
  NormIn<K, NT> hin;
  constexpr int PER = NormIn<K, NT>::PER, NQ = NormIn<K, NT>::Q;
  float4 yv[CMB ? 8 : 1][PER];
#pragma unroll
  for (int e = 0; e < PER; e++) {
    const int q = threadIdx.x + e * NT, qc = q < NQ ? q : NQ - 1;
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    hin.hv[e] = hin.wv[e] = z4;
#pragma unroll
    for (int j = 0; j < (CMB ? 8 : 1); j++) yv[j][e] = z4;
    if (wid * 64 + e * NT < NQ) {  // wave-uniform: some thread of the wave holds a quad (clamped, not guarded)
      hin.hv[e] = reinterpret_cast<const float4*>(h)[qc];
      hin.wv[e] = reinterpret_cast<const float4*>(lnw)[qc];
      if (CMB) {
#pragma unroll
        for (int j = 0; j < 8; j++) yv[j][e] = reinterpret_cast<const float4*>(ys)[(size_t)j * NQ + qc];
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  Rows<DT, K, P> rr;
  if (ok[0]) {  // a wave with no pair (wave-uniform) loads no row
    rows_load<DT, K, P>(rr, m, row, ok, lane);
    // the wave's rows in before its tiles are requested (vmcnt(0)): the rows come first, and the pairs' dot does not
    // wait for the tiles
    __builtin_amdgcn_s_waitcnt(0x0F70);
  }
  __builtin_amdgcn_sched_barrier(0);
  const int t0 = s * T, t = t0 + wt;
  const int tc = min(t, max_len / 64 - 1);  // a tile past the cache's end (never used) reads the last tile
  VShare<G> ksh, vsh;
  ksh.load(Kc, tc, lane, wh);
  vsh.load(Vc, tc, lane, wh);
  __builtin_amdgcn_sched_barrier(0);
  // the scalars, and the wave's cos/sin
  const int pos = (int)__builtin_amdgcn_readfirstlane(pos_v);
  const unsigned sctr = __builtin_amdgcn_readfirstlane(sctr_v);
  float wj[8];
#pragma unroll
  for (int j = 0; j < 8; j++) wj[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(yw_v), j));
  float cv[NP], sv[NP];
#pragma unroll
  for (int a = 0; a < NP; a++) {
    cv[a] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(rc_v), jp[a]));
    sv[a] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(rc_v), 32 + jp[a]));
  }
  const unsigned epoch = sctr * 64u + layer + 1u;
  // an earlier launch's failure: no wait here (and no further bit); a test mask: short waits, the masked ones for an
  // epoch no launch writes
  const unsigned err0 = __builtin_amdgcn_readfirstlane(err_v[0]), inj = __builtin_amdgcn_readfirstlane(err_v[1]);
  const int spin = err0 ? 0 : inj ? kInjectSpin : kAbSpin;
  const unsigned ep_q = (inj & 2u) ? kNoEpoch : epoch, ep_p = (inj & 4u) ? kNoEpoch : epoch;

  // 1. q/k/v pairs of the group
  if (CMB) {
#pragma unroll
    for (int e = 0; e < PER; e++) {
      float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        y.x = y.x + wj[j] * yv[j][e].x;
        y.y = y.y + wj[j] * yv[j][e].y;
        y.z = y.z + wj[j] * yv[j][e].z;
        y.w = y.w + wj[j] * yv[j][e].w;
      }
      float4& hv = hin.hv[e];
      hv = make_float4(hv.x + res * y.x, hv.y + res * y.y, hv.z + res * y.z, hv.w + res * y.w);
      const int q = threadIdx.x + e * NT;
      if (blockIdx.x == 0 && q < NQ) reinterpret_cast<float4*>(hc)[q] = hv;
    }
  }
  norm_finish<K, NT>(hin, eps, xs, &rs);
  XReg<DT, K> xr;
  load_x<DT, K>(xr, xs, lane);
  float out[P];
  rows_fma<DT, K, P>(rr, ok, xr, lane, out);
  TL_PHASE(tl, 2);
  if (lane == 0) {
#pragma unroll
    for (int a = 0; a < NP; a++) {
      if (!ok[2 * a]) continue;
      const float x1 = out[2 * a], x2 = out[2 * a + 1], c = cv[a], sn = sv[a];
      const int j = jp[a];
      if (lh[a] < G) {
        put_entry(&xg->q[lh[a]][j], __float_as_uint(x1 * c - x2 * sn), epoch);
        put_entry(&xg->q[lh[a]][j + 32], __float_as_uint(x2 * c + x1 * sn), epoch);
      } else {
        const bool isk = lh[a] == G;
        const uint16_t e1 = f2h(isk ? x1 * c - x2 * sn : x1), e2 = f2h(isk ? x2 * c + x1 * sn : x2);
        put_entry(&xg->kv[isk ? 0 : 1][j], e1, epoch);
        put_entry(&xg->kv[isk ? 0 : 1][j + 32], e2, epoch);
        uint16_t* row = (isk ? Kc : Vc) + (size_t)pos * 64;
        row[j] = e1;
        row[j + 32] = e2;
      }
    }
  }
  // the split's tiles into LDS while the other workgroups finish their pairs (every wave has read xs)
  __syncthreads();
  const int len = pos + 1;
  const int nb = (len + 63) / 64;
  const int used = min(T, nb - t0);  // tiles of this split inside the length (>= 1 when the split is used)
  const bool active = wt < used;
  const int nv = active ? min(64, len - t * 64) : 0;
  ksh.template store_h<KHS>(&Kh[wt][0][0], lane, wh, nv);
  vsh.store_ht(&Vt[wt][0][0], lane, wh, nv);
  TL_PHASE(tl, 3);
  __syncthreads();  // the staged tiles, before the new row goes over row pos

  // 2. the split's partials: queries of the group from the L2, the new K/V row (written by this group in phase 1)
  // over the stale row `pos` of the staged tiles
  {
    bool okw = true;
    if (wt == 0) {  // the queries of head wh
      const __amdgpu_buffer_rsrc_t rq = l2_buffer(&xg->q[0][0], sizeof(xg->q));
      const uint2 qv = poll_entries<false>(rq, 8u * (wh * 64 + lane), 0u, ep_q, spin, &okw);
      Qs[wh][lane] = __uint_as_float(qv.x);
    }
    const int tp = pos / 64 - t0;
    if (tp >= 0 && tp < T && wid == tp * G) {
      const __amdgpu_buffer_rsrc_t rk = l2_buffer(&xg->kv[0][0], sizeof(xg->kv));
      const uint2 kv = poll_entries<true>(rk, 8u * lane, 8u * (64 + lane), ep_q, spin, &okw);
      Kh[tp][pos & 63][lane] = (uint16_t)kv.x;
      Vt[tp][lane][VShare<G>::vt_col(pos & 63, lane)] = (uint16_t)kv.y;
    }
    if (!okw && lane == 0 && !err0) atomicOr(err, 2u);
  }
  __syncthreads();  // Qs, the new row
  TL_PHASE(tl, 4);
  // scores: lane = position, chain over the 64 dims in order (an inactive tile's scores are discarded)
  float sc;
  {
    float dt = 0.0f;
    const uint4* krow = reinterpret_cast<const uint4*>(&Kh[wt][lane][0]);
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const uint4 k8 = krow[c];
      const float4 q0 = *reinterpret_cast<const float4*>(&Qs[wh][8 * c]);
      const float4 q1 = *reinterpret_cast<const float4*>(&Qs[wh][8 * c + 4]);
      dt = __builtin_fmaf(q0.x, h2f((uint16_t)k8.x), dt);
      dt = __builtin_fmaf(q0.y, h2f((uint16_t)(k8.x >> 16)), dt);
      dt = __builtin_fmaf(q0.z, h2f((uint16_t)k8.y), dt);
      dt = __builtin_fmaf(q0.w, h2f((uint16_t)(k8.y >> 16)), dt);
      dt = __builtin_fmaf(q1.x, h2f((uint16_t)k8.z), dt);
      dt = __builtin_fmaf(q1.y, h2f((uint16_t)(k8.z >> 16)), dt);
      dt = __builtin_fmaf(q1.z, h2f((uint16_t)k8.w), dt);
      dt = __builtin_fmaf(q1.w, h2f((uint16_t)(k8.w >> 16)), dt);
    }
    sc = lane < nv ? dt * scale : NEG_INF;  // nv = 0 for an inactive tile
  }
  const float tmax = group_max<64>(sc);
  if (lane == 0) Tm[wh][wt] = tmax;
  __syncthreads();  // tile maxima
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
    wave_lds_sync();  // the wave's own p row, read back below by every lane of the same wave
    // p.v: lane = dim, chain over the positions in order; past the length p = 0 and V = +0, so those steps leave
    // pv unchanged (the chain equals the one over the valid positions only)
    const uint4* vrow = reinterpret_cast<const uint4*>(&Vt[wt][lane][0]);
    const int sd = (lane ^ (lane >> 3)) & 7;  // positions 8cj..8cj+7 of dim `lane` sit in 16-byte slot cj ^ sd
#pragma unroll
    for (int cj = 0; cj < 8; cj++) {
      const uint4 v8 = vrow[cj ^ sd];
      const float4 p0 = *reinterpret_cast<const float4*>(&Ps[wh][wt][8 * cj]);
      const float4 p1 = *reinterpret_cast<const float4*>(&Ps[wh][wt][8 * cj + 4]);
      pv = __builtin_fmaf(p0.x, h2f((uint16_t)v8.x), pv);
      pv = __builtin_fmaf(p0.y, h2f((uint16_t)(v8.x >> 16)), pv);
      pv = __builtin_fmaf(p0.z, h2f((uint16_t)v8.y), pv);
      pv = __builtin_fmaf(p0.w, h2f((uint16_t)(v8.y >> 16)), pv);
      pv = __builtin_fmaf(p1.x, h2f((uint16_t)v8.z), pv);
      pv = __builtin_fmaf(p1.y, h2f((uint16_t)(v8.z >> 16)), pv);
      pv = __builtin_fmaf(p1.z, h2f((uint16_t)v8.w), pv);
      pv = __builtin_fmaf(p1.w, h2f((uint16_t)(v8.w >> 16)), pv);
    }
    if (wt > 0) Pv[wh][wt][lane] = pv;
  }
  __syncthreads();  // p.v of every tile
  if (wt == 0 && used > 0) {
    float mm = NEG_INF, l = 0.0f, acc = 0.0f;
    for (int u = 0; u < used; u++) {
      const float a = Al[wh][u];
      l = __builtin_fmaf(l, a, Ts[wh][u]);
      acc = __builtin_fmaf(acc, a, u == 0 ? pv : Pv[wh][u][lane]);
      mm = mm > Tm[wh][u] ? mm : Tm[wh][u];
    }
    uint2* pe = xg->part[s][wh];
    put_entry(pe + 2 + lane, __float_as_uint(acc), epoch);
    if (lane == 0) {
      put_entry(pe, __float_as_uint(mm), epoch);
      put_entry(pe + 1, __float_as_uint(l), epoch);
    }
  }
  TL_PHASE(tl, 5);
  if (s >= G || wid != 0) {
    TL_END(tl);
    return;
  }

  // 3. workgroup s < G merges query head g*G + s: M = max m_s; w_s = exp(m_s - M); den and num are fma chains
  // over the used splits in order; out = num / den (k_attn_combine)
  const int hh = s;
  const int nsplit = (nb + T - 1) / T;  // used splits
  const __amdgpu_buffer_rsrc_t rp = l2_buffer(&xg->part[0][0][0], sizeof(xg->part));
  constexpr unsigned REC = sizeof(xg->part[0][0]), SREC = sizeof(xg->part[0]);
  // lane d reads acc[d] of every split (s2 >= nsplit: a clamped, unused entry) and lane s2 reads (m, l) of split s2;
  // all of them again until every entry of a used split carries the epoch
  float av[SP], ms = 0.0f, ls = 0.0f;
  const unsigned sl = (unsigned)min(lane, splits - 1);
  bool done = false;
  for (int it = 0; it < spin && !done; it++) {
    bool stale = false;
    poll_fence();
#pragma unroll
    for (int s2 = 0; s2 < SP; s2++) {
      const uint2 e = l2_load_u64(rp, (unsigned)min(s2, splits - 1) * SREC + hh * REC + 8u * (2 + lane));
      av[s2] = __uint_as_float(e.x);
      stale |= s2 < nsplit && e.y != ep_p;
    }
    const uint2 em = l2_load_u64(rp, sl * SREC + hh * REC), el = l2_load_u64(rp, sl * SREC + hh * REC + 8u);
    ms = __uint_as_float(em.x);
    ls = __uint_as_float(el.x);
    stale |= lane < nsplit && (em.y != ep_p || el.y != ep_p);
    done = __ballot(stale) == 0;
    if (!done) __builtin_amdgcn_s_sleep(1);
  }
  if (!done && lane == 0 && !err0) atomicOr(err, 4u);
  if (lane >= nsplit) {
    ms = NEG_INF;
    ls = 0.0f;
  }
  const float M = group_max<64>(ms);
  Cw[0][lane] = lane < nsplit ? dexp(ms - M) : 0.0f;
  Cw[1][lane] = ls;
  wave_lds_sync();
  float den = 0.0f, num = 0.0f;
#pragma unroll
  for (int s2 = 0; s2 < SP; s2++) {
    if (s2 < nsplit) {
      const float ws = Cw[0][s2];
      den = __builtin_fmaf(ws, Cw[1][s2], den);
      num = __builtin_fmaf(ws, av[s2], num);
    }
  }
  att[(g * G + hh) * 64 + lane] = num / den;
  TL_PHASE(tl, 6);
  TL_END(tl);
}

template <int DT, int K, int G, int T, int NP, int SP, bool CMB>
__global__ __launch_bounds__(G * T * 64) void k_attn_block(DMat m, const float* __restrict__ h,
                                                          const float* __restrict__ lnw, float eps,
                                                          const int* __restrict__ st, const float* __restrict__ rope_cur,
                                                          int heads, int max_len, uint16_t* __restrict__ kc,
                                                          uint16_t* __restrict__ vc, float scale, int splits, int pp,
                                                          AbGroup* __restrict__ xg_all,
                                                          const unsigned* __restrict__ step_ctr, unsigned layer,
                                                          unsigned* __restrict__ err, float* __restrict__ att,
                                                          const float* __restrict__ ys, const float* __restrict__ yw,
                                                          float res, float* __restrict__ hc, Tl tl) {
  attn_block_body<DT, K, G, T, NP, SP, CMB>(m, h, lnw, eps, st, rope_cur, heads, max_len, kc, vc, scale, splits, pp,
                                            xg_all, step_ctr, layer, err, att, ys, yw, res, hc, tl);
}

// The attention block of a cached step with its layer's prefetch (cache_pf.h): workgroups past the 8 * splits of
// the attention block decide (the first) or copy (the others); the attention workgroups are those of k_attn_block.
template <int DT, int K, int G, int T, int NP, int SP>
__global__ __launch_bounds__(G * T * 64) void k_attn_block_pf(DMat m, const float* __restrict__ h,
                                                          const float* __restrict__ lnw, float eps,
                                                          const int* __restrict__ st, const float* __restrict__ rope_cur,
                                                          int heads, int max_len, uint16_t* __restrict__ kc,
                                                          uint16_t* __restrict__ vc, float scale, int splits, int pp,
                                                          AbGroup* __restrict__ xg_all,
                                                          const unsigned* __restrict__ step_ctr, unsigned layer,
                                                          unsigned* __restrict__ err, float* __restrict__ att,
                                                          const float* __restrict__ ys, const float* __restrict__ yw,
                                                          float res, float* __restrict__ hc, Tl tl, PfArgs pf) {
  constexpr int NT = G * T * 64;
  const int extra = (int)blockIdx.x - 8 * splits;
  if (extra < 0) {
    attn_block_body<DT, K, G, T, NP, SP, false>(m, h, lnw, eps, st, rope_cur, heads, max_len, kc, vc, scale, splits,
                                                pp, xg_all, step_ctr, layer, err, att, ys, yw, res, hc, tl);
    return;
  }
  const unsigned sctr = __builtin_amdgcn_readfirstlane(
      __builtin_amdgcn_raw_buffer_load_b32(l2_buffer(step_ctr, 4), 0, 0, 0));
  // err[0]: error bits (a launch that finds one set waits for nothing); err[1]: the host's test mask
  // (moert_fault_inject): with bit 16 the copy workgroups wait for an epoch the decide does not write, and with any
  // bit every wait polls at most kInjectSpin times
  const auto ev = __builtin_amdgcn_raw_buffer_load_b64(l2_buffer(err, 8), 0, 0, 0);
  const unsigned err0 = __builtin_amdgcn_readfirstlane(ev[0]), inj = __builtin_amdgcn_readfirstlane(ev[1]);
  const unsigned epoch = sctr * 64u + layer + 1u;
  if (extra == 0) {
    pf_decide<DT, K, NT>(pf, h, epoch);
  } else if (!pf_copy<NT>(pf.c, (inj & 16u) ? kNoEpoch : epoch, extra - 1, err0 ? 0 : inj ? kInjectSpin : kPfSpin) &&
             threadIdx.x == 0 && !err0) {
    atomicOr(err, 16u);
  }
}

// ------------------------------------------------------------------------------------------------------------
namespace {

struct AbShape {
  int G, T, splits, pp, np;
};

// The launch shape of the attention block for these dimensions, or false when the fused path does not apply.
bool ab_shape(const Dims& d, const DMat& qkv, int cus, AbShape* out) {
  // one q/k/v row per wave pass (Q8_0 rows of 1024 or 1536, Q4_0 rows of 1536)
  const bool rows_ok = (qkv.dtype == DT_Q8_0 && (qkv.cols == 1024 || qkv.cols == 1536)) ||
                       (qkv.dtype == DT_Q4_0 && qkv.cols == 1536);
  if (d.kv_heads != 8 || d.head_dim != 64 || d.heads % 8 || !rows_ok || qkv.cols != d.hidden ||
      qkv.rows != (d.heads + 16) * 64)
    return false;
  const int G = d.heads / 8, T = d.tps;
  // the compiled shapes: 2 query heads per KV head with rows of 1024, 3 with rows of 1536
  if (!((G == 2 && qkv.cols == 1024) || (G == 3 && qkv.cols == 1536)) || T < 2 || T > 4 || d.max_len % 64)
    return false;
  const int splits = attn_splits_for(d.max_len, T);
  // every workgroup of a group must be resident at once (they wait for each other): one workgroup per compute
  // unit (the LDS of a workgroup is above half of a compute unit's), at most cus / 8 splits
  if (splits < G || splits > kAbMaxSplits || splits > 32 || 8 * splits > cus) return false;
  const int npair = (G + 2) * 32, pp = (npair + splits - 1) / splits, np = (pp + G * T - 1) / (G * T);
  if (np > 2) return false;
  *out = AbShape{G, T, splits, pp, np};
  return true;
}

}  // namespace

bool attn_block_fits(const Dims& d, const DMat& qkv, int cus) {
  AbShape sh;
  return ab_shape(d, qkv, cus, &sh);
}

bool attn_block_prefetch_fits(const Dims& d, const LayerDev& L, const CacheDev& c) {
  return c.pfx && c.slots >= d.top_k && c.slots <= kCacheMaxSlots && L.router.rows <= 64 && d.top_k <= 8 &&
         L.router.dtype == L.qkv.dtype && L.router.cols == L.qkv.cols;
}

hipError_t launch_attn_block(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int cus, int layer,
                             const AbBufs& x, bool combine, Tl tl, const CacheDev* pfc) {
  AbShape sh;
  if (!ab_shape(d, L.qkv, cus, &sh) || (combine && (d.top_k != 8 || layer < 1))) return hipErrorInvalidValue;
  if (pfc && (combine || !attn_block_prefetch_fits(d, L, *pfc))) return hipErrorInvalidValue;
  const int grid = 8 * sh.splits;
  const float* yw = b.route_w + (size_t)(layer > 0 ? layer - 1 : 0) * d.top_k;
  const PfArgs pf = pfc ? PfArgs{L.router, L.router_bias, L.ln_moe, d.eps, d.top_k, layer, *pfc} : PfArgs{};
#define AB_ARGS                                                                                                    \
  L.qkv, b.h, L.ln_attn, d.eps, b.state, x.rope_cur, d.heads, d.max_len, L.k_cache, L.v_cache, d.attn_mult,         \
      sh.splits, sh.pp, x.groups, x.step_ctr, (unsigned)layer, x.err, b.att, (const float*)x.ys, yw, d.res_mult, b.hc, tl
#define AB_LAUNCH(DD, KK, GG, TT, NN, CC) \
  klaunch(k_attn_block<DD, KK, GG, TT, NN, 32, CC>, grid, GG * TT * 64, 0, s, AB_ARGS)
#define AB_CASE(DD, KK, GG, TT, NN)                                                                                \
  if (L.qkv.dtype == DD && L.qkv.cols == KK && sh.G == GG && sh.T == TT && sh.np == NN) {                         \
    if (pfc)                                                                                                       \
      klaunch(k_attn_block_pf<DD, KK, GG, TT, NN, 32>, grid + 1 + kPfCopyWgs, GG * TT * 64, 0, s, AB_ARGS, pf);   \
    else if (combine)                                                                                              \
      AB_LAUNCH(DD, KK, GG, TT, NN, true);                                                                         \
    else                                                                                                           \
      AB_LAUNCH(DD, KK, GG, TT, NN, false);                                                                        \
    return hipGetLastError();                                                                                      \
  }
#define AB_T(DD, KK, GG) AB_CASE(DD, KK, GG, 2, 1) AB_CASE(DD, KK, GG, 2, 2) AB_CASE(DD, KK, GG, 3, 1) \
                         AB_CASE(DD, KK, GG, 3, 2) AB_CASE(DD, KK, GG, 4, 1) AB_CASE(DD, KK, GG, 4, 2)
  AB_T(DT_Q8_0, 1536, 3) AB_T(DT_Q8_0, 1024, 2) AB_T(DT_Q4_0, 1536, 3)
#undef AB_T
#undef AB_CASE
#undef AB_LAUNCH
#undef AB_ARGS
  return hipErrorInvalidValue;
}

}  // namespace moert

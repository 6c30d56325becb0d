// Every layer of a decode step in one launch: 256 workgroups of 1024 threads (one per compute unit, all resident at
// once), workgroup b on XCD x (its hardware XCC_ID) with index w = b / 8 inside the XCD (the chip dispatches the
// workgroups of a launch round-robin over its 8 XCDs, so the 32 workgroups 8w + r of one residue share an XCD). Per
// layer the workgroups run, with the operations and order of k_attn_block, k_oproj and k_moe_xcd (attn_block.hip,
// kernels.hip, moe_block.hip), so that the results are the same bit for bit:
//   A. the layer input: h' + res * (sum over j < 8 in order of w_j * ys_j) of the previous layer (its h' and its
//      experts' down outputs, by rank, as the previous launch left them), the whole vector in every workgroup; then
//      the rmsnorm (layer 0 reads the embedding row that k_embed left in h);
//   B. attention, KV head g = x: the group's (G + 2) * 32 q/k/v row pairs dealt out over the 32 workgroups, RoPE, the
//      KV append, workgroup s < S (the cache's splits) the partials of split s, workgroups s < G the merge of query
//      head g G + s (k_attn_block's phases 1-3);
//   C. the output projection, rows [x H / 8 + 8 w, + 8) on workgroups w < H / 64: the merged heads gathered from the
//      8 XCDs, h' = h + res * (Wo att);
//   D. every workgroup gathers h' from the 8 XCDs; workgroup w computes the MoE-norm items w and w + 32 (the router
//      dot of expert e, or the sum of squares, over 8-row blocks in moe_norm.h's order) and shares them through its
//      XCD's L2; every workgroup then has the logits, ranks the experts and normalises h';
//   E. the expert of rank x on XCD x, as k_moe_xcd: gate/up pairs, the act vector through the XCD's L2, down rows
//      [w HR, (w + 1) HR) into ys_x.
// After the last layer k_layer_combine combines its experts into h (k_moe_combine's arithmetic) for the head.
//
// Values cross between workgroups as 8-byte entries (value bits, epoch = step_ctr * 64 + layer + 1): through the
// XCD's L2 when both sides share an XCD (plain stores, loads that miss the compute unit's L1), and device-wide when
// they do not (agent-scope atomic stores and loads, which every XCD sees). A consumer polls exactly the entries it
// needs until their epochs match. Every wait is bounded: one that gives up sets a bit of err (2 queries / new K/V
// row, 4 split partials, 8 act vector, 32 the merged heads and 64 h' from the device-wide area, 128 the merged heads
// or h' relayed inside the XCD, or the router items), and the workgroup waits for nothing more in this launch;
// a launch that starts with a bit set waits for nothing. The replaced sequence is gpu_model.rs:338-412 (paths
// relative to rust/moe-rt/src) with the experts of cuda_backend.rs:804-835.
#include "attn_dev.h"
#include "dev_rows.h"
#include "kernels.h"
#include "launch.h"
#include "layers.h"
#include "moe_norm.h"
#include "timeline.h"

namespace moert {

namespace {

constexpr int kPxSpin = 1 << 18;
constexpr int kPxNW = kPxThreads / 64;
constexpr int kPxUpWaves = kPxNW / 2;  // phase E: the first half of the waves gate/up pairs, the second half down rows

// A dword read of a 128-byte line that leaves the line in the XCD's L2 for the next launch; the value is kept only
// so that the read is not dropped.
__device__ __forceinline__ unsigned warm(const void* line) { return *gmem(reinterpret_cast<const unsigned*>(line)); }

}  // namespace

// DT: dtype of every projection; K: hidden (= heads * 64); G: query heads per KV head; T: tiles per split.
template <int DT, int K, int G, int T>
__global__ __launch_bounds__(kPxThreads) void k_layer(PxLayer L, PxLayer Ln, int pf, int l, float eps, float res,
                                                     float scale, int max_len,
                                                     int splits, int pp, const int* __restrict__ st,
                                                     const float* __restrict__ rope_cur, const float* __restrict__ h,
                                                     float* __restrict__ hpp, float* __restrict__ ysp,
                                                     AbGroup* __restrict__ ab_all, MxGroup* __restrict__ mx_all,
                                                     PxXcd* __restrict__ px_all, PxDev* __restrict__ dv,
                                                     const unsigned* __restrict__ step_ctr, unsigned* __restrict__ err,
                                                     int* __restrict__ route_ids, float* __restrict__ route_w, Tl tl) {
  TL_START(tl);
  using Ge = Geo<DT, K>;    // rows of length K (q/k/v, o, gate/up)
  using GD = Geo<DT, 512>;  // down rows
  static_assert(Ge::RPW == 1, "one row of length K per wave and pass");
  constexpr int NW = kPxNW, NT = kPxThreads;
  constexpr int HR = K / 32;                 // rows of the layer input / expert outputs per workgroup
  constexpr int NOW = K / 64;                // workgroups with output-projection rows (8 rows each, per XCD)
  constexpr int TR = 8 % G == 0 ? 64 : 72;   // K tile rows (padding for VShare when G does not divide 8)
  constexpr int KHS = 72;
  constexpr int NPAIR = (G + 2) * 32;
  constexpr int NU = kPxUpWaves, ND = NW - kPxUpWaves;
  constexpr int PW = 512 / 32;               // gate/up pairs per workgroup
  constexpr int NPU = (PW + NU - 1) / NU;    // pairs per gate/up wave
  constexpr int DP = (HR + ND * GD::RPW - 1) / (ND * GD::RPW);  // down passes per down wave
  static_assert(NW >= G * T && NW > 8, "waves for the tiles, the output rows and their gather");
  static_assert((G + 2) * 32 <= 32 * NW && HR <= 64, "one q/k/v row pair per wave");
  constexpr int MA = (512 + ND * 64 - 1) / (ND * 64);  // act values per down thread
  static_assert(NU * NPU * Ge::RPW >= PW && ND * DP * GD::RPW >= HR, "phase E layout");

  __shared__ __align__(16) uint16_t Vt[T][64][64];
  __shared__ __align__(16) uint16_t Kh[T][TR][KHS];
  __shared__ __align__(16) float xs[K];     // normalised layer input (phase B), then the merged heads (phase C)
  __shared__ __align__(16) float hin[K];    // the layer input (residual of the output projection)
  __shared__ __align__(16) float hps[K];    // h' (phases D, E and the next layer's input)
  __shared__ __align__(16) float xm[K];     // normalised h' (phase E)
  __shared__ __align__(16) float as[512];
  __shared__ __align__(16) float Qs[G][64];
  __shared__ __align__(16) float Ps[G][T][64];
  __shared__ float Pv[G][T][64];
  __shared__ float Tm[G][T], Al[G][T], Ts[G][T];
  __shared__ __align__(16) float lg[64];
  __shared__ int part[NW][64];
  __shared__ float rs;
  __shared__ float hp8_s[8];  // the workgroup's output rows of h' (phase C)
  __shared__ int dead_s;

  const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int x = (int)xcc_id() & 7, w = blockIdx.x >> 3;
  const int g = x;
  const int wh = wid % G, wt = wid / G;
  AbGroup* xg = ab_all + g;
  MxGroup* mg = mx_all + x;
  PxXcd* pg = px_all + x;
  const float NEG_INF = __int_as_float(0xff800000);

  // The values earlier launches wrote that every wave needs as scalars (position, step counter, error word and
  // test mask, the previous layer's routing weights) and the step's rope row are the first vector loads; they are
  // read back as scalars only after the layer's bulk loads have been issued (loads complete in issue order, so
  // waiting for them waits for nothing else, and no round trip precedes the bulk loads).
  const unsigned pos_v = __builtin_amdgcn_raw_buffer_load_b32(l2_buffer(st, 4 * ST_WORDS), 4 * ST_POS, 0, 0);
  const unsigned sctr_v = __builtin_amdgcn_raw_buffer_load_b32(l2_buffer(step_ctr, 4), 0, 0, 0);
  const auto err_v = __builtin_amdgcn_raw_buffer_load_b64(l2_buffer(err, 8), 0, 0, 0);
  const float rc_v = *gmem(rope_cur + lane);
  const float yw_v = l > 0 ? *gmem(route_w + (size_t)(l - 1) * 8 + (lane & 7)) : 0.0f;
  __builtin_amdgcn_sched_barrier(0);
  const unsigned tx = threadIdx.x;
  const int s = w;  // this workgroup's split (when s < splits)
  const int t0 = s * T, t = t0 + wt;
  // this wave's q/k/v row pair (one per wave, waves 0 .. pp - 1)
  const int pl = w * pp + wid;
  const bool pok = wid < pp && pl < NPAIR;
  const int plc = pok ? pl : 0;
  const int lh = plc / 32, jp = plc % 32;
  uint16_t* Kc = L.kc + (size_t)g * max_len * 64;
  uint16_t* Vc = L.vc + (size_t)g * max_len * 64;

  // ---- the layer's bulk loads: its input (layer 0: the embedding row; later: the previous layer's h' and its 8
  // expert outputs, left by the previous launch), then the q/k/v pair rows and the split's K/V tiles ----
  // The input is held by the last IW waves, one quad per thread, and the norm runs on the last wave: waves that issue
  // no row or tile loads, so that their waits for the input wait for nothing else (a wait after a load issued under
  // a branch is counted as if the branch had been taken).
  static_assert((K / 4) % 64 == 0 && K / 4 <= NT, "one input quad per thread of the input waves");
  constexpr int IW = K / 256;
  const bool inw = wid >= NW - IW;
  const int q4 = (int)tx - (NW - IW) * 64;  // this thread's quad (input waves)
  float4 h0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), y0[8], wa = h0;
#pragma unroll
  for (int j = 0; j < 8; j++) y0[j] = h0;
  // the norm weights of both halves and the router bias with the input (a load issued after a phase's reduction
  // would put a memory round trip on its critical path)
  constexpr int MQ = (K + NT - 1) / NT;
  float wm[MQ];
#pragma unroll
  for (int m = 0; m < MQ; m++) wm[m] = *gmem(L.ln_moe + min((int)tx + m * NT, K - 1));
  const float bias_v = L.bias ? *gmem(L.bias + min(lane, L.router.rows - 1)) : 0.0f;
  if (inw) {
    wa = gload_f4(reinterpret_cast<const float4*>(L.ln_attn) + q4);
    h0 = gload_f4(reinterpret_cast<const float4*>(l == 0 ? h : hpp) + q4);
    if (l > 0) {
#pragma unroll
      for (int j = 0; j < 8; j++) y0[j] = gload_f4(reinterpret_cast<const float4*>(ysp + j * K) + q4);
    }
  }
  // a compute unit passes requests to its L1 at a fixed rate of bytes: a bare workgroup barrier puts every wave's
  // input loads ahead of any wave's rows and tiles
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  size_t row[2] = {0, 0};
  bool rok[2] = {pok, pok};
  {
    const int gh = lh < G ? g * G + lh : lh == G ? 8 * G + g : 8 * G + 8 + g;
    row[0] = (size_t)gh * 64 + jp;
    row[1] = row[0] + 32;
  }
  Rows<DT, K, 2> rr;
  if (pok) {
    rows_load<DT, K, 2>(rr, L.qkv, row, rok, lane);
    // the wave's rows in before its tiles are requested (vmcnt(0)): the rows come first, and the pair's dot does
    // not wait for the tiles
    __builtin_amdgcn_s_waitcnt(0x0F70);
  }
  const int tc = min(t, max_len / 64 - 1);
  VShare<G> ksh, vsh;
  if (wid < G * T) {
    ksh.load(Kc, tc, lane, wh);
    vsh.load(Vc, tc, lane, wh);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- A. the layer input: h' + res * (sum over j < 8 in order of w_j * ys_j) (k_attn_block's prologue) ----
  float4 hv = h0;
  if (inw) {
    if (l > 0) {
      float wprev[8];
#pragma unroll
      for (int j = 0; j < 8; j++)
        wprev[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(yw_v), j));
      float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        y.x = y.x + wprev[j] * y0[j].x;
        y.y = y.y + wprev[j] * y0[j].y;
        y.z = y.z + wprev[j] * y0[j].z;
        y.w = y.w + wprev[j] * y0[j].w;
      }
      hv = make_float4(hv.x + res * y.x, hv.y + res * y.y, hv.z + res * y.z, hv.w + res * y.w);
    }
    reinterpret_cast<float4*>(hin)[q4] = hv;
    if (wid == NW - 1 && lane == 0) dead_s = __builtin_amdgcn_readfirstlane(err_v[0]) ? 1 : 0;
  }
  __syncthreads();
  // rmsnorm: the canonical sum of squares by the last wave (norm_finish's order)
  if (wid == NW - 1) {
    constexpr int NCH = K / 16;
    float acc = 0.0f;
#pragma unroll
    for (int jj = 0; jj < (NCH + 63) / 64; jj++) {
      const int j = lane + 64 * jj;
      if (j < NCH) {
        const float4* p = reinterpret_cast<const float4*>(hin + 16 * j);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float4 v4 = p[e];
          acc = __builtin_fmaf(v4.x, v4.x, acc);
          acc = __builtin_fmaf(v4.y, v4.y, acc);
          acc = __builtin_fmaf(v4.z, v4.z, acc);
          acc = __builtin_fmaf(v4.w, v4.w, acc);
        }
      }
    }
    const float ss = group_sum<64>(acc);
    if (lane == 0) rs = 1.0f / sqrtf(ss / (float)K + eps);
  }
  __syncthreads();
  if (inw) {
    const float r = rs;
    reinterpret_cast<float4*>(xs)[q4] =
        make_float4(wa.x * (hv.x * r), wa.y * (hv.y * r), wa.z * (hv.z * r), wa.w * (hv.w * r));
  }
  __syncthreads();

  // the scalars (read after phase A: a wave with row or tile loads in flight waits for them at its first read of a
  // loaded value, and none of them may wait before the barriers of phase A)
  const int pos = (int)__builtin_amdgcn_readfirstlane(pos_v);
  const unsigned sctr = __builtin_amdgcn_readfirstlane(sctr_v);
  const unsigned err0 = __builtin_amdgcn_readfirstlane(err_v[0]), inj = __builtin_amdgcn_readfirstlane(err_v[1]);
  const int spin0 = inj ? 16 * kInjectSpin : kPxSpin;
  const int len = pos + 1, nb = (len + 63) / 64;
  const int used = min(T, nb - t0);
  const bool active = wid < G * T && s < splits && wt < used;
  const int nv = active ? min(64, len - t * 64) : 0;
  const int nsplit = (nb + T - 1) / T;
  const float cv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(rc_v), jp));
  const float sv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(rc_v), 32 + jp));
  const unsigned epoch = sctr * 64u + (unsigned)l + 1u;
  const unsigned ep_q = (inj & 2u) ? kNoEpoch : epoch, ep_p = (inj & 4u) ? kNoEpoch : epoch;
  const unsigned ep_a = (inj & 8u) ? kNoEpoch : epoch;

  // a wait that gives up sets `bit` (unless a failure is already recorded) and marks the workgroup dead: its later
  // waits give up at once. With a test mask, the masked waits give up after kInjectSpin polls and every other wait
  // after 16 times that, so that the masked one is always the first to give up (the waits behind it then get their
  // values: a workgroup whose wait gave up goes on and publishes what it computes).
  auto spin_now = [&]() { return dead_s ? 0 : spin0; };
  auto spin_inj = [&](unsigned bit) { return dead_s ? 0 : (inj & bit) ? kInjectSpin : spin0; };
  auto fail = [&](bool ok, unsigned bit) {
    if (!ok && lane == 0) {
      if (!dead_s && !err0) atomicOr(err, bit);
      dead_s = 1;
    }
  };

  {
    TL_PHASE(tl, 2);

    // ---- B. attention of KV head g ----
    if (pok) {
      XReg<DT, K> xr;
      load_x<DT, K>(xr, xs, lane);
      float out[2];
      rows_fma<DT, K, 2>(rr, rok, xr, lane, out);
      if (lane == 0) {
        const float x1 = out[0], x2 = out[1];
        if (lh < G) {
          put_entry(&xg->q[lh][jp], __float_as_uint(x1 * cv - x2 * sv), epoch);
          put_entry(&xg->q[lh][jp + 32], __float_as_uint(x2 * cv + x1 * sv), epoch);
        } else {
          const bool isk = lh == G;
          const uint16_t e1 = f2h(isk ? x1 * cv - x2 * sv : x1), e2 = f2h(isk ? x2 * cv + x1 * sv : x2);
          put_entry(&xg->kv[isk ? 0 : 1][jp], e1, epoch);
          put_entry(&xg->kv[isk ? 0 : 1][jp + 32], e2, epoch);
          uint16_t* crow = (isk ? Kc : Vc) + (size_t)pos * 64;
          *gmem_w(crow + jp) = e1;
          *gmem_w(crow + jp + 32) = e2;
        }
      }
    }
    // the split's tiles into LDS (loaded at the layer's start, in flight while the input and the pairs were formed)
    if (wid < G * T) {
      ksh.template store_h<KHS>(&Kh[wt][0][0], lane, wh, nv);
      vsh.store_ht(&Vt[wt][0][0], lane, wh, nv);
    }
    __syncthreads();
    if (s < splits) {
      bool okw = true;
      if (wid < G * T && wt == 0) {
        const __amdgpu_buffer_rsrc_t rq = l2_buffer(&xg->q[0][0], sizeof(xg->q));
        int idx[1] = {wh * 64 + lane};
        bool use[1] = {true};
        unsigned v[1];
        okw = poll_m<1>([&](int i) { return l2_load_u64(rq, 8u * (unsigned)i); }, idx, use, ep_q, spin_inj(2u), v);
        Qs[wh][lane] = __uint_as_float(v[0]);
      }
      const int tp = pos / 64 - t0;
      if (tp >= 0 && tp < T && wid == tp * G) {
        const __amdgpu_buffer_rsrc_t rk = l2_buffer(&xg->kv[0][0], sizeof(xg->kv));
        int idx[2] = {lane, 64 + lane};
        bool use[2] = {true, true};
        unsigned v[2];
        okw = okw && poll_m<2>([&](int i) { return l2_load_u64(rk, 8u * (unsigned)i); }, idx, use, ep_q,
                               spin_inj(2u), v);
        Kh[tp][pos & 63][lane] = (uint16_t)v[0];
        Vt[tp][lane][VShare<G>::vt_col(pos & 63, lane)] = (uint16_t)v[1];
      }
      fail(okw, 2u);
    }
    __syncthreads();
    // scores and p.v of the split's tiles (k_attn_block phase 2)
    float sc = NEG_INF;
    if (wid < G * T) {
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
      sc = lane < nv ? dt * scale : NEG_INF;
      const float tmax = group_max<64>(sc);
      if (lane == 0) Tm[wh][wt] = tmax;
    }
    __syncthreads();
    float pv = 0.0f;
    if (active) {
      const float tmax = Tm[wh][wt];
      float mprev = NEG_INF;
      for (int u = 0; u < wt; u++) mprev = mprev > Tm[wh][u] ? mprev : Tm[wh][u];
      const float mn = mprev > tmax ? mprev : tmax;
      const float alpha = dexp(mprev - mn);
      const float p = dexp(sc - mn);
      const float tsum = group_sum<64>(p);
      Ps[wh][wt][lane] = p;
      if (lane == 0) {
        Al[wh][wt] = alpha;
        Ts[wh][wt] = tsum;
      }
      wave_lds_sync();
      const uint4* vrow = reinterpret_cast<const uint4*>(&Vt[wt][lane][0]);
      const int sd = (lane ^ (lane >> 3)) & 7;
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
    __syncthreads();
    if (s < splits && wid < G && used > 0) {  // wave wh, wt = 0: the split's partials of head wh
      float mm = NEG_INF, lsum = 0.0f, acc = 0.0f;
      for (int u = 0; u < used; u++) {
        const float a = Al[wh][u];
        lsum = __builtin_fmaf(lsum, a, Ts[wh][u]);
        acc = __builtin_fmaf(acc, a, u == 0 ? pv : Pv[wh][u][lane]);
        mm = mm > Tm[wh][u] ? mm : Tm[wh][u];
      }
      uint2* pe = xg->part[s][wh];
      put_entry(pe + 2 + lane, __float_as_uint(acc), epoch);
      if (lane == 0) {
        put_entry(pe, __float_as_uint(mm), epoch);
        put_entry(pe + 1, __float_as_uint(lsum), epoch);
      }
    }
    // merge of query head g G + s by workgroup s < G, wave 0 (k_attn_block phase 3)
    if (s < G && wid == 0) {
      const __amdgpu_buffer_rsrc_t rp = l2_buffer(&xg->part[0][0][0], sizeof(xg->part));
      constexpr unsigned REC = sizeof(xg->part[0][0]), SREC = sizeof(xg->part[0]);
      float av[32], ms = 0.0f, lsv = 0.0f;
      const unsigned sl = (unsigned)min(lane, splits - 1);
      bool done = false;
      const int sp = spin_inj(4u);
      for (int it = 0; it < sp && !done; it++) {
        bool stale = false;
        poll_fence();
#pragma unroll
        for (int s2 = 0; s2 < 32; s2++) {
          const uint2 e = l2_load_u64(rp, (unsigned)min(s2, splits - 1) * SREC + s * REC + 8u * (2 + lane));
          av[s2] = __uint_as_float(e.x);
          stale |= s2 < nsplit && e.y != ep_p;
        }
        const uint2 em = l2_load_u64(rp, sl * SREC + s * REC), el = l2_load_u64(rp, sl * SREC + s * REC + 8u);
        ms = __uint_as_float(em.x);
        lsv = __uint_as_float(el.x);
        stale |= lane < nsplit && (em.y != ep_p || el.y != ep_p);
        done = __ballot(stale) == 0;
        if (!done) __builtin_amdgcn_s_sleep(1);
      }
      fail(done, 4u);
      if (lane >= nsplit) {
        ms = NEG_INF;
        lsv = 0.0f;
      }
      const float M = group_max<64>(ms);
      // split s2's weight and sum from lane s2 by readlane (no LDS round trips between the FMAs)
      const float wsl = lane < nsplit ? dexp(ms - M) : 0.0f;
      float den = 0.0f, num = 0.0f;
#pragma unroll
      for (int s2 = 0; s2 < 32; s2++) {
        if (s2 < nsplit) {
          const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(wsl), s2));
          const float ls = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(lsv), s2));
          den = __builtin_fmaf(ws, ls, den);
          num = __builtin_fmaf(ws, av[s2], num);
        }
      }
      put_dev(&dv->att[(g * G + s) * 64 + lane], __float_as_uint(num / den), epoch);
    }

    TL_PHASE(tl, 3);
    // ---- C. output projection rows [x K / 8 + 8 w, + 8), workgroups w < NOW ----
    const bool orow = w < NOW && wid < 8;
    const int orw = x * (K / 8) + 8 * w + wid;
    Rows<DT, K, 1> ro;
    unsigned keep0 = 0, keep1 = 0;
    if (wid < 8) {
      // (a workgroup without output rows loads row 0, unused)
      size_t r1[1] = {(size_t)(orow ? orw : 0)};
      bool ok1[1] = {orow};
      rows_load<DT, K, 1>(ro, L.o, r1, ok1, lane);
      // behind the output row: one read of each 128-byte line that the next launch's workgroup of this split loads
      // first (its q/k/v pair rows and output row, slot A; its K/V tiles, slot B), so that they come from the XCD's
      // L2 there (the reads go out while the exchanges of phases C and D leave HBM idle). They are unconditional (a
      // lane without a line reads the head's first one), so that the wait for the output row counts exactly them.
      const PxLayer& N = pf ? Ln : L;
      constexpr int RL = (int)(K * (DT == DT_Q4_0 ? 1 : 2) / 2 / 128);  // lines of a row's payload
      const int pa = w * pp + wid;
      const int ah = min(pa, NPAIR - 1) / 32, aj = min(pa, NPAIR - 1) % 32;
      const int agh = ah < G ? g * G + ah : ah == G ? 8 * G + g : 8 * G + 8 + g;
      const size_t arow0 = (size_t)agh * 64 + aj, orow0 = (size_t)(x * (K / 8) + 8 * w + wid);
      const bool apair = wid < pp && pa < NPAIR;
      const int ar = lane < 3 * RL ? lane / RL : lane - 3 * RL;  // payload lines of rows 0..2, then their scales
      const bool apay = lane < 3 * RL;
      const bool aval = ar <= 1 ? apair : ar == 2 && w < NOW;
      const size_t rsel = ar == 0 ? arow0 : ar == 1 ? arow0 + 32 : orow0;
      const uint8_t* aq = ar == 2 ? N.o.q : N.qkv.q;
      const uint16_t* ad = ar == 2 ? N.o.d : N.qkv.d;
      const uint8_t* la = apay ? aq + rsel * (size_t)(RL * 128) + (size_t)(lane % RL) * 128
                               : reinterpret_cast<const uint8_t*>(ad + rsel * (size_t)(K / 32));
      const int ntl = s < splits ? min(T, max_len / 64 - t0) : 0;
      const int u = wid * 64 + lane;
      const bool bk = u < ntl * 64, bv = !bk && u < 2 * ntl * 64;
      const size_t tbase = ((size_t)g * max_len + (size_t)t0 * 64) * 64;
      const uint8_t* lb = reinterpret_cast<const uint8_t*>(bk ? N.kc + tbase : N.vc + tbase) +
                          (size_t)(bk ? u : bv ? u - ntl * 64 : 0) * 128;
      const uint8_t* l0 = reinterpret_cast<const uint8_t*>(N.kc + (size_t)g * max_len * 64);  // head g's first line
      keep0 = warm(aval ? la : l0);
      keep1 = warm(bk || bv ? lb : l0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the merged heads of the 8 XCDs: wave 8 of workgroup w < 8 relays XCD w's G heads from the device-wide area
    // into this XCD's L2 area, and the output-projection workgroups gather them all from there (one device-wide
    // read of each value per XCD instead of one per workgroup)
    if (w < 8 && wid == 8) {
      int idx[G];
      bool use[G];
#pragma unroll
      for (int m = 0; m < G; m++) {
        idx[m] = w * G * 64 + m * 64 + lane;
        use[m] = true;
      }
      unsigned v[G];
      const bool ok = poll_m<G>([&](int i) { return get_dev(dv->att + i); }, idx, use, epoch, spin_now(), v);
      fail(ok, 32u);
#pragma unroll
      for (int m = 0; m < G; m++) put_entry(&pg->att[idx[m]], v[m], epoch);
    }
    if (w < NOW) {
      // waves 8.. (waves 0..7 have their rows in flight)
      if (wid >= 8) {
        constexpr int FTC = NT - 512, M = (K + FTC - 1) / FTC;
        int idx[M];
        bool use[M];
#pragma unroll
        for (int m = 0; m < M; m++) {
          idx[m] = (int)tx - 512 + m * FTC;
          use[m] = idx[m] < K;
          idx[m] = use[m] ? idx[m] : 0;
        }
        unsigned v[M];
        const __amdgpu_buffer_rsrc_t ra = l2_buffer(pg->att, sizeof(pg->att));
        const bool ok = poll_m<M>([&](int i) { return l2_load_u64(ra, 8u * (unsigned)i); }, idx, use, epoch,
                                  spin_now(), v);
#pragma unroll
        for (int m = 0; m < M; m++)
          if (use[m]) xs[idx[m]] = __uint_as_float(v[m]);
        fail(ok, 128u);
      }
      __syncthreads();
      TL_PHASE(tl, 4);
      if (orow) {
        XReg<DT, K> xr;
        load_x<DT, K>(xr, xs, lane);
        float out[1];
        bool ok1[1] = {true};
        rows_fma<DT, K, 1>(ro, ok1, xr, lane, out);
        if (lane == 0) {
          const float hv = hin[orw] + res * out[0];
          hp8_s[wid] = hv;
          *gmem_w(hpp + orw) = hv;  // for the next launch
        }
      }
      __syncthreads();
      // the workgroup's 8 rows of h' go out device-wide as one 64-byte store (8 lanes), not 8 single entries
      if (wid == 0 && lane < 8) put_dev(&dv->hp[x * (K / 8) + 8 * w + lane], __float_as_uint(hp8_s[lane]), epoch);
      TL_PHASE(tl, 5);
    }

    // ---- D. h' from the 8 XCDs, the router items, ranks ----
    // waves 0 and 1 load the rows of items w and w + 32 (an expert's router row, or none for the sum of squares);
    // waves 2.. gather h', so that their polls do not wait behind those loads
    const int E = L.router.rows;
    const int item = w + 32 * wid;
    const bool iok = wid < 2 && item <= E;
    Col8 cw[3];
    float4 lw0[3], lw1[3];
    if (wid < 2) {
#pragma unroll
      for (int q = 0; q < 3; q++) {
        int c0 = 8 * (lane + 64 * q);
        c0 = c0 < K ? c0 : 0;
        cw[q] = load_col8<DT>(L.router, iok && item < E ? item : 0, c0);
        lw0[q] = gload_f4(L.ln_moe + c0);
        lw1[q] = gload_f4(L.ln_moe + c0 + 4);
      }
    } else {
      // h' rows [x' K / 8, (x' + 1) K / 8) come from XCD x': the last wave of workgroup w < 8 (no output row of
      // its own, so it polls from the end of phase C on) relays XCD w's rows into this XCD's L2 area; waves 2..
      // then gather the whole vector from there
      if (w < 8 && wid == NW - 1) {
        int idx[G];
        bool use[G];
#pragma unroll
        for (int m = 0; m < G; m++) {
          idx[m] = w * G * 64 + m * 64 + lane;
          use[m] = true;
        }
        unsigned v[G];
        const bool ok = poll_m<G>([&](int i) { return get_dev(dv->hp + i); }, idx, use, epoch, spin_now(), v);
        fail(ok, 64u);
#pragma unroll
        for (int m = 0; m < G; m++) put_entry(&pg->hp[idx[m]], v[m], epoch);
      }
      constexpr int FTD = NT - 128, M = (K + FTD - 1) / FTD;
      const int ft = tx - 128;
      int idx[M];
      bool use[M];
#pragma unroll
      for (int m = 0; m < M; m++) {
        idx[m] = ft + m * FTD;
        use[m] = idx[m] < K;
        idx[m] = use[m] ? idx[m] : 0;
      }
      unsigned v[M];
      const __amdgpu_buffer_rsrc_t rh = l2_buffer(pg->hp, sizeof(pg->hp));
      const bool ok = poll_m<M>([&](int i) { return l2_load_u64(rh, 8u * (unsigned)i); }, idx, use, epoch,
                                spin_now(), v);
#pragma unroll
      for (int m = 0; m < M; m++)
        if (use[m]) hps[idx[m]] = __uint_as_float(v[m]);
      fail(ok, 128u);
    }
    __syncthreads();
    TL_PHASE(tl, 6);
    if (iok) {
      // item `item` over the K / 8 blocks: block b in lane b % 64 (blocks added in increasing b), then the lane tree
      float acc = 0.0f;
#pragma unroll
      for (int q = 0; q < 3; q++) {
        const int b = lane + 64 * q, c0 = 8 * b;
        if (c0 < K) {
          const float* hb = hps + c0;
          const float lwv[8] = {lw0[q].x, lw0[q].y, lw0[q].z, lw0[q].w, lw1[q].x, lw1[q].y, lw1[q].z, lw1[q].w};
          float z = 0.0f;
          if (item < E) {
#pragma unroll
            for (int tt = 0; tt < 8; tt++) z = __builtin_fmaf(col8_elem<DT>(cw[q], tt, c0), lwv[tt] * hb[tt], z);
          } else {
#pragma unroll
            for (int tt = 0; tt < 8; tt++) z = __builtin_fmaf(hb[tt], hb[tt], z);
          }
          acc = acc + z;
        }
      }
      const float tot = group_sum<64>(acc);
      if (lane == 0) put_entry(&pg->item[item], __float_as_uint(tot), epoch);
    }
    TL_PHASE(tl, 7);
    {
      bool ok = true;
      if (wid == 0) {
        const __amdgpu_buffer_rsrc_t ri = l2_buffer(pg->item, sizeof(pg->item));
        int idx[1] = {lane <= E ? lane : 0};
        bool use[1] = {lane <= E};
        unsigned v[1];
        ok = poll_m<1>([&](int i) { return l2_load_u64(ri, 8u * (unsigned)i); }, idx, use, epoch, spin_now(), v);
        const float z = __uint_as_float(v[0]);
        const float ssv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_uint(z), E));
        const float r = 1.0f / sqrtf(ssv / (float)K + eps);
        if (lane < E) lg[lane] = L.bias ? z * r + bias_v : z * r;
        if (lane == 0) rs = r;
      }
      fail(ok, 128u);
    }
    __syncthreads();
    TL_PHASE(tl, 8);
    {
      const float r = rs;
#pragma unroll
      for (int m = 0; m < MQ; m++) {
        const int i = tx + m * NT;
        if (i < K) xm[i] = wm[m] * (hps[i] * r);
      }
    }
    int rank;
    {
      // wg_rank for any wave count: wave v counts the keys [v PER, (v + 1) PER) above lane e's key (total-order key,
      // then 63 - e), the counts meet in LDS and are added (an exact integer sum)
      constexpr int PER = (64 + NW - 1) / NW;
      auto key = [&](int e) -> unsigned long long {
        const unsigned long long kv =
            ((unsigned long long)((unsigned)total_key(lg[e & 63]) ^ 0x80000000u) << 6) | (unsigned)(63 - (e & 63));
        return e < E ? kv : 0ull;
      };
      const unsigned long long mine = key(lane);
      int cnt = 0;
#pragma unroll
      for (int u = 0; u < PER; u++) cnt += key(wid * PER + u) > mine;
      part[wid][lane] = cnt;
      __syncthreads();  // (xm and lg are visible after it too)
      rank = 0;
#pragma unroll
      for (int v2 = 0; v2 < NW; v2++) rank += part[v2][lane];
    }
    const bool sel = lane < E && rank < 8;
    TL_PHASE(tl, 9);
    const unsigned long long bx = __ballot(sel && rank == x);
    const int ej = bx ? __ffsll((long long)bx) - 1 : 0;

    // ---- E. the expert of rank x: gate/up pairs, act through the XCD's L2, down rows ----
    const bool up = wid < NU;
    const int dsub = lane % GD::LPR, drw = lane / GD::LPR;
    size_t drow[DP];
    bool dok[DP];
    int dr[DP];
#pragma unroll
    for (int p = 0; p < DP; p++) {
      const int li = ((wid - NU) * DP + p) * GD::RPW + drw;
      dr[p] = w * HR + li;
      dok[p] = !up && li < HR;
      drow[p] = (size_t)ej * K + (dok[p] ? dr[p] : 0);
    }
    // the gate/up requests go out first (a bare workgroup barrier puts them ahead of the down rows, which are needed
    // only after the act vector)
    size_t urow[2 * NPU];
    bool uok[2 * NPU];
    int pi[NPU];
#pragma unroll
    for (int a = 0; a < NPU; a++) {
      const int li = wid * NPU + a;
      pi[a] = w * PW + li;
      const bool v = up && li < PW;
      const size_t r0 = (size_t)ej * 1024 + (v ? pi[a] : 0);
      urow[2 * a] = r0;
      urow[2 * a + 1] = r0 + 512;
      uok[2 * a] = uok[2 * a + 1] = v;
    }
    Rows<DT, K, 2 * NPU> ur;
    if (up) rows_load<DT, K, 2 * NPU, true>(ur, L.gu, urow, uok, lane);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    Rows<DT, 512, DP> dd;
    if (!up) rows_load<DT, 512, DP, true>(dd, L.dn, drow, dok, dsub);
    if (up) {
      XReg<DT, K> xr;
      load_x<DT, K>(xr, xm, lane);
      float out[2 * NPU];
      rows_fma<DT, K, 2 * NPU>(ur, uok, xr, lane, out);
      if (lane == 0) {
#pragma unroll
        for (int a = 0; a < NPU; a++)
          if (uok[2 * a]) put_entry(&mg->act[pi[a]], __float_as_uint(silu_mul(out[2 * a], out[2 * a + 1])), epoch);
      }
    } else {
      // the step's routing record and the weights in rank order for the next layer's input: workgroup 0's last
      // wave, a down wave, after its down rows are requested (no gate/up wave waits for it)
      if (blockIdx.x == 0 && wid == NW - 1) {
        int eid[8];
        ids_by_rank(sel, rank, 8, eid);
        const float lv = lg[lane];
        const float ex = sel ? dexp(lv - lg[eid[0]]) : 0.0f;
        float sum = 0.0f;
#pragma unroll
        for (int r2 = 0; r2 < 8; r2++)
          sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), eid[r2]));
        if (sel) {
          *gmem_w(route_ids + l * 8 + rank) = lane;
          *gmem_w(route_w + l * 8 + rank) = ex / sum;
        }
      }
      const int i = tx - NU * 64;
      const __amdgpu_buffer_rsrc_t ra = l2_buffer(mg->act, sizeof(mg->act));
      int idx[MA];
      bool use[MA];
#pragma unroll
      for (int m = 0; m < MA; m++) {
        idx[m] = i + m * ND * 64;
        use[m] = idx[m] < 512;
        idx[m] = use[m] ? idx[m] : 0;
      }
      unsigned v[MA];
      const bool ok = poll_m<MA>([&](int q) { return l2_load_u64(ra, 8u * (unsigned)q); }, idx, use, ep_a,
                                 spin_inj(8u), v);
#pragma unroll
      for (int m = 0; m < MA; m++)
        if (use[m]) as[idx[m]] = __uint_as_float(v[m]);
      fail(ok, 8u);
    }
    __syncthreads();
    TL_PHASE(tl, 10);
    if (!up) {
      XReg<DT, 512> xa;
      load_x<DT, 512>(xa, as, dsub);
      float dout[DP];
      rows_fma<DT, 512, DP>(dd, dok, xa, dsub, dout);
      if (dsub == 0) {
#pragma unroll
        for (int p = 0; p < DP; p++)
          if (dok[p]) *gmem_w(ysp + (size_t)x * K + dr[p]) = dout[p];
      }
    }
    asm volatile("" ::"v"(keep0), "v"(keep1));
  }

  TL_END(tl);
}

// ------------------------------------------------------------------------------------------------------------
namespace {

struct PxShape {
  int G, T, splits, pp;
};

bool px_shape(const Dims& d, const LayerDev& L, int cus, PxShape* out) {
  const DMat& qkv = L.qkv;
  const bool dt_ok = (qkv.dtype == DT_Q8_0 && (d.hidden == 1024 || d.hidden == 1536)) ||
                     (qkv.dtype == DT_Q4_0 && d.hidden == 1536);
  if (!dt_ok || d.kv_heads != 8 || d.head_dim != 64 || d.heads % 8 || d.heads * 64 != d.hidden ||
      qkv.cols != d.hidden || qkv.rows != (d.heads + 16) * 64 || d.top_k != 8 || d.inter != 512 || d.experts > 63 ||
      d.max_len % 64 || cus < 256)
    return false;
  for (const DMat* m : {&L.o, &L.router, &L.gate_up, &L.down})
    if (m->dtype != qkv.dtype) return false;
  if (L.o.rows != d.hidden || L.o.cols != d.hidden || L.router.cols != d.hidden || L.gate_up.cols != d.hidden ||
      L.down.cols != 512)
    return false;
  const int G = d.heads / 8, T = d.tps;
  if (!((G == 2 && d.hidden == 1024) || (G == 3 && d.hidden == 1536)) || T < 2 || T > 4) return false;
  const int splits = attn_splits_for(d.max_len, T);
  if (splits < G || splits > 32) return false;
  const int pp = ((G + 2) * 32 + 31) / 32;
  *out = PxShape{G, T, splits, pp};
  return true;
}

}  // namespace

bool layers_fit(const Dims& d, const LayerDev& L, int cus) {
  PxShape sh;
  return px_shape(d, L, cus, &sh);
}

// h = h' + res * (sum over j < 8 in order of w_j * ys_j) of the last layer, from the device-wide entries of its
// launch (k_moe_combine's arithmetic): the input of the head.
template <int K>
__global__ __launch_bounds__(256) void k_layer_combine(const float* __restrict__ hpp, const float* __restrict__ ysp,
                                                       const float* __restrict__ wts, float res, float* __restrict__ h,
                                                       Tl tl) {
  TL_START(tl);
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int ic = i < K ? i : K - 1;
  float d[8], wj[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    d[j] = ysp[(size_t)j * K + ic];
    wj[j] = wts[j];
  }
  const float hv = hpp[ic];
  float y = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) y = y + wj[j] * d[j];
  if (i < K) h[i] = hv + res * y;
  TL_END(tl);
}

hipError_t launch_layer(hipStream_t s, const PxLayer& L, const LayerDev& Ld, int layer, const Dims& d,
                        const StepBufs& b, int cus, const AbBufs& x, const PxBufs& p, const PxLayer* next, Tl tl) {
  PxShape sh;
  if (!px_shape(d, Ld, cus, &sh) || layer < 0 || layer > 62) return hipErrorInvalidValue;
#define PX_LAUNCH(DD, KK, GG, TT)                                                                              \
  klaunch(k_layer<DD, KK, GG, TT>, 256, kPxThreads, 0, s, L, next ? *next : L, next ? 1 : 0, layer, d.eps,      \
          d.res_mult, d.attn_mult, d.max_len, sh.splits, sh.pp, b.state, x.rope_cur, b.h, p.hp, x.ys, x.groups, x.moe, \
          p.xcd, p.dev, x.step_ctr, x.err, b.route_ids, b.route_w, tl)
#define PX_CASE(DD, KK, GG, TT)                                                             \
  if (Ld.qkv.dtype == DD && d.hidden == KK && sh.G == GG && sh.T == TT) {                   \
    PX_LAUNCH(DD, KK, GG, TT);                                                              \
    return hipGetLastError();                                                               \
  }
#define PX_T(DD, KK, GG) PX_CASE(DD, KK, GG, 2) PX_CASE(DD, KK, GG, 3) PX_CASE(DD, KK, GG, 4)
  PX_T(DT_Q8_0, 1536, 3) PX_T(DT_Q8_0, 1024, 2) PX_T(DT_Q4_0, 1536, 3)
#undef PX_T
#undef PX_CASE
#undef PX_LAUNCH
  return hipErrorInvalidValue;
}

hipError_t launch_layer_combine(hipStream_t s, const Dims& d, const StepBufs& b, int last_layer, const AbBufs& x,
                                const PxBufs& p, Tl tl) {
  if (d.top_k != 8) return hipErrorInvalidValue;
  const float* wts = b.route_w + (size_t)last_layer * 8;
  switch (d.hidden) {
    case 1024: klaunch(k_layer_combine<1024>, 4, 256, 0, s, (const float*)p.hp, (const float*)x.ys, wts, d.res_mult, b.h, tl); break;
    case 1536: klaunch(k_layer_combine<1536>, 6, 256, 0, s, (const float*)p.hp, (const float*)x.ys, wts, d.res_mult, b.h, tl); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace moert

// MoE half of a decode step in one launch, the routed experts spread over the XCDs: workgroup b runs on XCD x (its
// hardware XCC_ID; the workgroups 8w + r of one residue r share an XCD, w = b / 8) and serves the expert of routing
// rank j = x. Every workgroup computes the rmsnorm and the router from the output projection's MoE-norm partials and
// ranks the experts (as k_route_up does); then
//   1. its gate/up row pairs of expert j (pairs [w * PW, (w + 1) * PW), PW = inter / 32): act = silu(gate . xn) *
//      (up . xn), stored with the launch's epoch into XCD x's L2 area (one 8-byte word per value);
//   2. the expert's whole act vector from that L2, polled until every value carries the epoch, and its down rows
//      [w * RB, (w + 1) * RB) (RB = hidden / 32), loaded right after routing so that they arrive while the act
//      vector is formed: ys[j][r] = down_r . act.
// Waves 0..7 take the gate/up pairs and waves 8..15 the down rows and the act poll (a wave's loads complete in
// issue order, so the polls of a wave that holds down rows in flight return once those rows are in).
// The weighted combine h += res * (sum over j in top-k order of w_j * ys[j]) is done by the next kernel that reads h
// (the attention block of the next layer, or k_moe_combine before the head), with the operations and order of
// k_expert_down's epilogue. Each (row, expert) dot is the canonical chain of k_route_up / k_expert_down, so the
// results are the same bit for bit. Replaces k_route_up + k_expert_down (gemv + route_topk, moe_gate_up, moe_down,
// rust/moe-rt/src/cuda_backend.rs:804-835, hits.rs:67-148; Cpu::experts, cpu.rs:116-150).
// The act poll is bounded; a poll that gives up sets bit 3 of `err` and the kernel still ends.
#include "attn_dev.h"
#include "dev_rows.h"
#include "kernels.h"
#include "launch.h"
#include "moe_norm.h"
#include "timeline.h"

namespace moert {

namespace {
constexpr int kMxSpin = 1 << 18;
constexpr int kMxWaves = 16;
constexpr int kMxUpWaves = 8;  // waves 0..7: gate/up pairs; waves 8..15: down rows

// Wave-level poll of act entry i (one per lane) from the XCD's L2 until every lane's entry carries `epoch`; returns
// the value. Clears *ok when the poll gave up.
__device__ __forceinline__ float mx_poll(__amdgpu_buffer_rsrc_t r, int i, unsigned epoch, int spin, bool* ok) {
  for (int it = 0; it < spin; it++) {
    poll_fence();
    const uint2 e = l2_load_u64(r, 8u * i);
    if (__ballot(e.y != epoch) == 0) return __uint_as_float(e.x);
    __builtin_amdgcn_s_sleep(1);
  }
  *ok = false;
  return 0.0f;
}
}  // namespace

template <int DT, int K, int I, int NP, int DP>
__global__ __launch_bounds__(kMxWaves * 64) void k_moe_xcd(DMat router, const float* __restrict__ bias, DMat gu,
                                                          DMat dn, const float* __restrict__ h,
                                                          const float* __restrict__ lnw, float eps,
                                                          const float* __restrict__ zp, int* __restrict__ ids_out,
                                                          float* __restrict__ w_out, float* __restrict__ ys,
                                                          MxGroup* __restrict__ xg_all,
                                                          const unsigned* __restrict__ step_ctr, unsigned layer,
                                                          unsigned* __restrict__ err, Tl tl) {
  TL_START(tl);
  using G = Geo<DT, K>;   // gate/up rows (length hidden)
  using GD = Geo<DT, I>;  // down rows (length inter)
  constexpr int NW = kMxWaves, NT = NW * 64, P = 2 * NP;
  constexpr int PW = I / kMxWgs;  // gate/up pairs per workgroup
  constexpr int RB = K / kMxWgs;  // down rows per workgroup
  constexpr int NU = kMxUpWaves, ND = NW - kMxUpWaves;
  static_assert(NU * NP * G::RPW >= PW && ND * DP * GD::RPW >= RB, "a workgroup covers its pairs and rows");
  __shared__ float xs[K];
  __shared__ __align__(16) float as[I];
  __shared__ __align__(16) float lg[64];
  __shared__ int part[NW][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int x = (int)xcc_id() & 7, w = blockIdx.x >> 3;
  MxGroup* xg = xg_all + x;
  const int E = router.rows;

  // rmsnorm and router from the MoE-norm partials (k_route_up's prologue): the sum-of-squares partials, this wave's
  // router items and bias, this thread's elements of h and the norm weights
  constexpr int IPW = (64 + NW - 1) / NW;
  constexpr int XP = (K + NT - 1) / NT;
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
  const unsigned epoch = *step_ctr * 64u + layer + 1u;
  // an earlier launch's failure: no wait here (and no further bit); the test mask: a short wait for an epoch no
  // launch writes
  const uint2 errv = *reinterpret_cast<const uint2*>(err);
  const int spin = errv.x ? 0 : errv.y ? kInjectSpin : kMxSpin;
  const unsigned ep_act = (errv.y & 8u) ? kNoEpoch : epoch;
  __builtin_amdgcn_sched_barrier(0);
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
    if (i < K) xs[i] = wv[e] * (hv[e] * r);
  }
  __syncthreads();
  TL_PHASE(tl, 2);
  // routed ids as wave-uniform values; workgroup 0 publishes ids and weights
  const int rank = wg_rank<NW>(lg, E, lane, wave, part);
  const bool sel = lane < E && rank < 8;
  if (blockIdx.x == 0 && wave == 0) {
    int eid[8];
    ids_by_rank(sel, rank, 8, eid);
    route_weights(lg, sel, rank, 8, lane, eid, ids_out, w_out);
  }
  // the expert of rank x (ids_by_rank's entry x, one ballot instead of eight per wave)
  const unsigned long long bx = __ballot(sel && rank == x);
  const int ej = bx ? __ffsll((long long)bx) - 1 : 0;
  TL_PHASE(tl, 3);

  // gate/up waves: their pairs of expert ej; down waves: their down rows of ej, requested right away
  const bool up = wave < NU;
  const int dsub = lane % GD::LPR, drw = lane / GD::LPR;
  size_t drow[DP];
  bool dok[DP];
  int dr[DP];
#pragma unroll
  for (int p = 0; p < DP; p++) {
    const int li = ((wave - NU) * DP + p) * GD::RPW + drw;  // down row of the workgroup (down waves)
    dr[p] = w * RB + li;
    dok[p] = !up && li < RB;
    drow[p] = (size_t)ej * K + (dok[p] ? dr[p] : 0);
  }
  // the gate/up requests go out first (a compute unit passes requests to its L1 at a fixed rate of bytes: a bare
  // workgroup barrier puts them ahead of the down rows, which are needed only after the act vector)
  const int sub = lane % G::LPR, rw = lane / G::LPR;
  size_t row[P];
  bool ok[P];
  int pi[NP];
#pragma unroll
  for (int a = 0; a < NP; a++) {
    const int li = (wave * NP + a) * G::RPW + rw;  // pair of the workgroup
    pi[a] = w * PW + li;
    const bool v = up && li < PW;
    const size_t r0 = (size_t)ej * 2 * I + (v ? pi[a] : 0);
    row[2 * a] = r0;
    row[2 * a + 1] = r0 + I;
    ok[2 * a] = ok[2 * a + 1] = v;
  }
  Rows<DT, K, P> rr;
  if (up) rows_load<DT, K, P>(rr, gu, row, ok, sub);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  Rows<DT, I, DP> dd;
  if (!up) rows_load<DT, I, DP>(dd, dn, drow, dok, dsub);
  if (up) {
    XReg<DT, K> xr;
    load_x<DT, K>(xr, xs, sub);
    float out[P];
    rows_fma<DT, K, P>(rr, ok, xr, sub, out);
    if (sub == 0) {
#pragma unroll
      for (int a = 0; a < NP; a++)
        if (ok[2 * a]) put_entry(&xg->act[pi[a]], __float_as_uint(silu_mul(out[2 * a], out[2 * a + 1])), epoch);
    }
    TL_PHASE(tl, 4);
  } else {
    // the expert's act vector from the L2 (down thread i polls act[i]), then the down rows
    static_assert(I == ND * 64, "one act value per down thread");
    const int i = threadIdx.x - NU * 64;
    bool got = true;
    as[i] = mx_poll(l2_buffer(xg->act, sizeof(xg->act)), i, ep_act, spin, &got);
    if (!got && lane == 0 && !errv.x) atomicOr(err, 8u);
  }
  __syncthreads();
  TL_PHASE(tl, 5);
  if (!up) {
    XReg<DT, I> xa;
    load_x<DT, I>(xa, as, dsub);
    float dout[DP];
    rows_fma<DT, I, DP>(dd, dok, xa, dsub, dout);
    if (dsub == 0) {
#pragma unroll
      for (int p = 0; p < DP; p++)
        if (dok[p]) ys[(size_t)x * K + dr[p]] = dout[p];
    }
  }
  TL_END(tl);
}

// h = h + res * (sum over j < 8, in order, of w_j * ys[j]): the combine of the last layer's experts before the head
// (k_expert_down's epilogue: y = y + w_j * d_j from +0, then h + res * y). One element per thread, its 8 loads at
// once.
template <int K>
__global__ __launch_bounds__(256) void k_moe_combine(float* __restrict__ h, const float* __restrict__ ys,
                                                     const float* __restrict__ wts, float res, Tl tl) {
  TL_START(tl);
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int ic = i < K ? i : K - 1;
  float d[8], wj[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    d[j] = ys[(size_t)j * K + ic];
    wj[j] = wts[j];
  }
  const float hv = h[ic];
  float y = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) y = y + wj[j] * d[j];
  if (i < K) h[i] = hv + res * y;
  TL_END(tl);
}

// ------------------------------------------------------------------------------------------------------------
bool moe_xcd_fits(const Dims& d, const LayerDev& L, int cus) {
  const DMat& gu = L.gate_up;
  return d.top_k == 8 && d.experts <= 64 && d.inter == 512 && (d.hidden == 1024 || d.hidden == 1536) &&
         (gu.dtype == DT_Q8_0 || gu.dtype == DT_Q4_0) && gu.dtype == L.router.dtype && gu.dtype == L.down.dtype &&
         gu.cols == d.hidden && L.down.cols == d.inter && cus >= 8 * kMxWgs;
}

hipError_t launch_moe_xcd(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int cus, int layer,
                          const AbBufs& x, Tl tl) {
  if (!moe_xcd_fits(d, L, cus)) return hipErrorInvalidValue;
  const int grid = 8 * kMxWgs;
#define MX_CASE(DD, KK)                                                                                       \
  if (L.gate_up.dtype == DD && d.hidden == KK) {                                                              \
    constexpr int NU = kMxUpWaves, ND = kMxWaves - kMxUpWaves;                                                \
    constexpr int NP = (512 / kMxWgs + NU * Geo<DD, KK>::RPW - 1) / (NU * Geo<DD, KK>::RPW);                  \
    constexpr int DP = (KK / kMxWgs + ND * Geo<DD, 512>::RPW - 1) / (ND * Geo<DD, 512>::RPW);                 \
    klaunch(k_moe_xcd<DD, KK, 512, NP, DP>, grid, kMxWaves * 64, 0, s, L.router, L.router_bias, L.gate_up,    \
            L.down, b.h, L.ln_moe, d.eps, b.zpart, b.route_ids + layer * 8, b.route_w + layer * 8, x.ys,      \
            x.moe, x.step_ctr, (unsigned)layer, x.err, tl);                                                    \
    return hipGetLastError();                                                                                  \
  }
  MX_CASE(DT_Q8_0, 1536) MX_CASE(DT_Q8_0, 1024) MX_CASE(DT_Q4_0, 1536) MX_CASE(DT_Q4_0, 1024)
#undef MX_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_moe_combine(hipStream_t s, const Dims& d, const StepBufs& b, int layer, const AbBufs& x, Tl tl) {
  if (d.top_k != 8) return hipErrorInvalidValue;
  switch (d.hidden) {
    case 1024:
      klaunch(k_moe_combine<1024>, 4, 256, 0, s, b.h, (const float*)x.ys, b.route_w + layer * 8, d.res_mult, tl);
      break;
    case 1536:
      klaunch(k_moe_combine<1536>, 6, 256, 0, s, b.h, (const float*)x.ys, b.route_w + layer * 8, d.res_mult, tl);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace moert

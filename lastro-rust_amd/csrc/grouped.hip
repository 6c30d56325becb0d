// Multi-position MoE step: m <= 32 token positions through one MoE block with the expert FFNs as a grouped int8
// MFMA GEMM (the multi-position path of Cpu::experts_step, rust/moe-rt/src/cpu.rs:239-296; GPU per-position loops
// cuda_backend.rs:751-917, which this replaces by one grouped pass).
//
// Positions are regrouped per expert in first-appearance order (the reference's list order); every weight row of
// an expert is read once from HBM and used by all of the expert's member positions. The expert GEMMs run on
// v_mfma_i32_16x16x32_i8: one 32-element Q8_0 block is one MFMA K-step, so each block product is an exact int32
// and the block scales are applied afterwards. Activations enter the MFMA as 15-bit codes split in two int8
// planes (v = 256*hi + lo, per 32-element block d = amax/32639), so the products stay exact integers:
//   S_b = 256 * (q . hi)_b + (q . lo)_b,   acc = fmaf((float)S_b, d_w(b) * d_x(b), acc)   for b = 0, 1, ...
// y[p] = y[p] + w * o accumulates the experts in list order, as the reference does.
//
// Kernels (one stream, in order):
//   k_grp_route   grid m:            router + top-k of position p, hi/lo codes of x_p
//   k_grp_up      grid (I/64, U):    grouping (every workgroup), gate/up MFMA of list expert u for its members,
//                                    SwiGLU, hi/lo codes of act; workgroup (0, 0) publishes the plan
//   k_grp_down    grid (H/64, U):    down MFMA of list expert u for its members -> o[member slot]
//   k_grp_combine grid (m, H/256):   y[p] = sum over p's experts in list order of w * o
#include <climits>

#include "dev_rows.h"
#include "grouped.h"
#include "launch.h"
#include "mfma_q8.h"

namespace moert {

constexpr int kRouteThreads = 1024;

// The codes of the m already-normalised inputs x[m, H] (the experts of a multi-position model step, routed by its
// own router): workgroup p.
template <int H>
__global__ __launch_bounds__(256) void k_grp_codes(const float* __restrict__ x, GroupBufs g) {
  constexpr int NB = H / 32;
  const int p = blockIdx.x;
  for (int base = 0; base < NB; base += 256 / 8) {
    const int b = base + (threadIdx.x >> 3), part = threadIdx.x & 7;
    const bool valid = b < NB;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = valid ? x[(size_t)p * H + 32 * b + 4 * part + i] : 0.0f;
    block_codes<H>(v, valid, p, b, part, g.xh, g.xl, g.xd);
  }
}

// ------------------------------------------------------------------------------------------------------------
// Per-position router (canonical dot, optional bias), top-k, and the hi/lo codes of x_p: workgroup p.
template <int DT, int H, bool NORM>
__global__ __launch_bounds__(kRouteThreads) void k_grp_route(DMat router, const float* __restrict__ bias,
                                                             const float* __restrict__ x,
                                                             const float* __restrict__ lnw, float eps, int k,
                                                             GroupBufs g) {
  using G = Geo<DT, H>;
  constexpr int NW = kRouteThreads / 64;
  constexpr int RP = (64 + NW * G::RPW - 1) / (NW * G::RPW);
  constexpr int NB = H / 32;
  __shared__ float xs[H];
  __shared__ __align__(16) float lg[64];
  __shared__ __align__(16) TopkLds tk;
  const int p = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPR, rw = lane / G::LPR;
  const int E = router.rows;
  size_t row[RP];
  bool ok[RP];
#pragma unroll
  for (int q = 0; q < RP; q++) {
    row[q] = (size_t)(q * NW + wave) * G::RPW + rw;
    ok[q] = row[q] < (size_t)E;
  }
  Rows<DT, H, RP> rr;
  rows_load<DT, H, RP>(rr, router, row, ok, sub);
  float bv[RP];
#pragma unroll
  for (int q = 0; q < RP; q++) bv[q] = bias ? bias[ok[q] ? row[q] : 0] : 0.0f;  // clamped, not guarded: one run of loads
  wg_copy<H, kRouteThreads>(x + (size_t)p * H, xs);
  if (NORM) {
    // x is the residual stream: xs = lnw * (x * r), r = 1 / sqrt(mean(x^2) + eps)
    __shared__ float wsum[NW];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < H; i += kRouteThreads) ss = __builtin_fmaf(xs[i], xs[i], ss);
    ss = group_sum<64>(ss);
    if (lane == 0) wsum[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) tot = tot + wsum[w];
    const float r = 1.0f / sqrtf(tot / (float)H + eps);
    for (int i = threadIdx.x; i < H; i += kRouteThreads) xs[i] = lnw[i] * (xs[i] * r);
    __syncthreads();
  }
  XReg<DT, H> xr;
  load_x<DT, H>(xr, xs, sub);
  float out[RP];
  rows_fma<DT, H, RP>(rr, ok, xr, sub, out);
#pragma unroll
  for (int q = 0; q < RP; q++)
    if (ok[q] && sub == 0) lg[row[q]] = bias ? out[q] + bv[q] : out[q];
  // hi/lo codes: 8 lanes per 32-element block, 4 elements per lane
  for (int base = 0; base < NB; base += kRouteThreads / 8) {
    const int b = base + (threadIdx.x >> 3), part = threadIdx.x & 7;
    const bool valid = b < NB;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = valid ? xs[32 * b + 4 * part + i] : 0.0f;
    block_codes<H>(v, valid, p, b, part, g.xh, g.xl, g.xd);
  }
  __syncthreads();
  if (wave == 0) wave_topk(lg, E, k, lane, tk, g.ids + (size_t)p * k, g.w + (size_t)p * k);
}

// ------------------------------------------------------------------------------------------------------------
// Grouping of the m*k (position, expert) entries, computed in LDS by every workgroup of the gate/up kernel:
//   list order   experts sorted by their first entry p*k + j (first appearance, as experts_step builds its list)
//   members      positions routing to the expert, as a bit mask (member index = set bits below the position)
//   slots        member slot = offset of the expert + member index (rows of the act / o buffers)
struct Plan {
  int8_t se[kGrpMaxPos * 8];  // expert of entry p*k + j (< 64)
  int first[64];           // first entry of expert e (INT_MAX when unused)
  unsigned bits[64];       // member positions of expert e
  int uof[64], offe[64];   // list index and first member slot of expert e
  int list[64];            // expert of list index u
  unsigned long long fmask[kGrpMaxPos * 8 / 64];  // entries that are the first entry of their expert
  int nu;
};

template <int NT>
__device__ __forceinline__ void make_plan(const int* __restrict__ ids, int m, int k, Plan& s) {
  constexpr int NWORD = kGrpMaxPos * 8 / 64;
  static_assert(NT >= kGrpMaxPos * 8, "one thread per entry");
  const int t = threadIdx.x, n = m * k;
  const int mine = t < n ? ids[t] : 0;
  if (t < 64) {
    s.first[t] = INT_MAX;
    s.bits[t] = 0u;
  }
  if (t < NWORD) s.fmask[t] = 0ull;
  __syncthreads();
  if (t < n) {
    s.se[t] = (int8_t)mine;
    atomicMin(&s.first[mine], t);
    atomicOr(&s.bits[mine], 1u << (t / k));
  }
  __syncthreads();
  if (t < n && s.first[mine] == t) atomicOr(&s.fmask[t >> 6], 1ull << (t & 63));
  __syncthreads();
  if (t < 64) {
    // lane e: list index of expert e = the first entries below its own (first-appearance order); then the
    // member offsets as an exclusive prefix sum of the member counts in list order
    const bool present = s.bits[t] != 0u;
    const int key = present ? s.first[t] : 0;
    int u = 0, nu = 0;
#pragma unroll
    for (int w = 0; w < NWORD; w++) {
      const unsigned long long word = s.fmask[w];
      nu += __popcll(word);
      const int lo = 64 * w;
      if (key >= lo + 64)
        u += __popcll(word);
      else if (key > lo)
        u += __popcll(word & ((1ull << (key - lo)) - 1ull));
    }
    if (present) {
      s.uof[t] = u;
      s.list[u] = t;
    }
    wave_lds_sync();
    const int cnt = t < nu ? __popc(s.bits[s.list[t]]) : 0;
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d);
      if (t >= d) incl += o;
    }
    if (t < nu) s.offe[s.list[t]] = incl - cnt;
    if (t == 0) s.nu = nu;
  }
  __syncthreads();
}

// The plan in global memory for the down and combine kernels (written once, by one workgroup).
template <int NT>
__device__ __forceinline__ void publish_plan(const Plan& s, const float* __restrict__ w, int m, int k, int* grp) {
  const int t = threadIdx.x, n = m * k;
  if (t == 0) grp[GRP_NU] = s.nu;
  if (t < s.nu) {
    const int e = s.list[t];
    grp[GRP_LIST + t] = e;
    grp[GRP_CNT + t] = __popc(s.bits[e]);
    grp[GRP_OFF + t] = s.offe[e];
    grp[GRP_BITS + t] = (int)s.bits[e];
  }
  for (int i = t; i < n; i += NT) {
    const int p = i / k, e = s.se[i];
    int rank = 0;
    for (int j = 0; j < k; j++) rank += s.uof[s.se[p * k + j]] < s.uof[e];
    grp[GRP_ORD_SLOT + p * 8 + rank] = s.offe[e] + __popc(s.bits[e] & ((1u << p) - 1u));
    grp[GRP_ORD_W + p * 8 + rank] = __float_as_int(w[i]);
  }
}

// ------------------------------------------------------------------------------------------------------------
// Tiled copy of a Q8_0 matrix (TMat layout): thread i writes the 16-byte piece i = (tile, span, lane) and, for
// lanes below 32, the scale of row lane%16 in block 2*span + lane/16.
__global__ __launch_bounds__(256) void k_tile_q8(DMat src, uint8_t* __restrict__ q, uint16_t* __restrict__ d) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const int NP = src.cols / 64, NB = src.cols / 32;
  if (i >= (size_t)src.rows / 16 * NP * 64) return;
  const int l = (int)(i % 64), p = (int)(i / 64 % NP);
  const size_t t = i / 64 / NP, r = 16 * t + (l & 15);
  const uint8_t* sp = src.q + r * src.cols + 64 * p + 8 * (l >> 4);
  const uint2 lo = *reinterpret_cast<const uint2*>(sp), hi = *reinterpret_cast<const uint2*>(sp + 32);
  reinterpret_cast<uint4*>(q)[i] = make_uint4(lo.x, lo.y, hi.x, hi.y);
  if (l < 32) {
    const int b = 2 * p + (l >> 4);
    d[(t * NB + b) * 16 + (l & 15)] = src.d[r * NB + b];
  }
}

hipError_t launch_tile_q8(hipStream_t s, const DMat& src, uint8_t* q, uint16_t* d) {
  if (src.dtype != DT_Q8_0 || src.rows % 16 || src.cols % 64) return hipErrorInvalidValue;
  const size_t n = (size_t)src.rows / 16 * (src.cols / 64) * 64;
  klaunch(k_tile_q8, (unsigned)((n + 255) / 256), 256, 0, s, src, q, d);
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------------------
// Gate/up of list expert u = blockIdx.y for its members, rows [RT t, RT t + RT) of gate and of up (t = blockIdx.x,
// RT = 16 * NT / 128): the first half of the waves computes 16 gate rows each, the second half the same up rows, so
// the members' codes staged in LDS serve every wave. Then act = silu(g)*u and its hi/lo codes (each 32 rows are
// one block of the act vector), written to the members' slots.
constexpr int kGrpUpThreads = 512;

template <int H, int NM, int NT>
__global__ __launch_bounds__(NT) void k_grp_up(int m, int k, int inter, GroupBufs g) {
  constexpr int NB = H / 32;
  constexpr int STR = H + 16;
  constexpr int WH = NT / 128;  // waves per half (gate or up)
  constexpr int RT = 16 * WH;   // gate (and up) rows of the workgroup
  static_assert(RT % 32 == 0, "whole act blocks per workgroup");
  __shared__ Plan plan;
  __shared__ __align__(16) int8_t bh[NM * STR];
  __shared__ __align__(16) int8_t bl[NM * STR];
  __shared__ float dx[NM * NB];
  __shared__ __align__(16) uint16_t sdt[NT / 64][NB * 16];
  __shared__ float gout[2][RT][NM + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int u = blockIdx.y, tile = blockIdx.x;
  make_plan<NT>(g.ids, m, k, plan);
  if (u >= plan.nu) return;
  const int e = plan.list[u], off = plan.offe[e];
  const unsigned bits = plan.bits[e];
  const int ne = __popc(bits);
  // this wave's 16 rows: gate (first half) or up (second half) rows [RT tile + 16 (wave % WH), +16) of expert e
  const size_t t16 = ((size_t)e * 2 * inter + (size_t)(wave / WH) * inter + RT * tile + 16 * (wave % WH)) / 16;
  TileScales<NB> sc;
  fetch_scales<NB>(g.gu, t16, NB, 0, sc);
  Members<H, NM, NT> mb;
  fetch_members<H, NM, NT, false>(g.xh, g.xl, g.xd, bits, 0, ne, mb);
  uint4 a[NB / 2];
  fetch_tile_q8<NB>(g.gu, t16, NB, 0, a);
  store_scales<NB>(sc, sdt[wave]);
  store_members<H, NM, NT>(mb, bh, bl, STR, dx);
  __syncthreads();
  float acc[NM / 16][4];
  mfma_tile<NB, NM>(a, bh, bl, STR, sdt[wave], dx, NB, acc);
  const int grp = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < NM / 16; ct++)
#pragma unroll
    for (int i = 0; i < 4; i++) gout[wave / WH][16 * (wave % WH) + 4 * grp + i][16 * ct + (lane & 15)] = acc[ct][i];
  __syncthreads();
  // act = silu(gate) * up for RT rows (RT/32 blocks) x NM members; 8 lanes per (block, member), 4 rows a lane
  for (int base = 0; base < RT / 32 * NM; base += NT / 8) {
    const int pi = base + (threadIdx.x >> 3), part = threadIdx.x & 7;
    const int bi = pi / NM, j = pi % NM;
    const bool valid = pi < RT / 32 * NM && j < ne;
    float av[4];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = (32 * bi + 4 * part + i) & (RT - 1);
      av[i] = valid ? silu_mul(gout[0][r][j], gout[1][r][j]) : 0.0f;
      const float aa = fabsf(av[i]);
      amax = aa > amax ? aa : amax;
    }
    amax = group_max<8>(amax);
    const float d = amax / 32639.0f;
    uint32_t hw = 0, lw = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int q = d > 0.0f ? (int)__builtin_rintf(av[i] / d) : 0;
      const int h = (q + 128) >> 8;
      hw |= (uint32_t)(uint8_t)(int8_t)h << (8 * i);
      lw |= (uint32_t)(uint8_t)(int8_t)(q - 256 * h) << (8 * i);
    }
    if (valid) {
      const size_t slotv = (size_t)(off + j);
      const int blk = RT / 32 * tile + bi;
      reinterpret_cast<uint32_t*>(g.ah + slotv * inter + 32 * blk)[part] = hw;
      reinterpret_cast<uint32_t*>(g.al + slotv * inter + 32 * blk)[part] = lw;
      if (part == 0) g.ad[slotv * (inter / 32) + blk] = d;
    }
  }
  if (u == 0 && tile == 0) publish_plan<NT>(plan, g.w, m, k, g.grp);
}

// ------------------------------------------------------------------------------------------------------------
// Down of list expert u = blockIdx.y for its members, output rows [64t, 64t+64): o[slot][row].
template <int I, int NM>
__global__ __launch_bounds__(256, NM == 16 ? 2 : 1) void k_grp_down(int hidden, GroupBufs g) {
  constexpr int NB = I / 32;
  constexpr int STR = I + 16;
  __shared__ __align__(16) int8_t bh[NM * STR];
  __shared__ __align__(16) int8_t bl[NM * STR];
  __shared__ float dx[NM * NB];
  __shared__ __align__(16) uint16_t sdt[4][NB * 16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int u = blockIdx.y, tile = blockIdx.x;
  if (u >= g.grp[GRP_NU]) return;
  const int e = g.grp[GRP_LIST + u], ne = g.grp[GRP_CNT + u], off = g.grp[GRP_OFF + u];
  const size_t t16 = ((size_t)e * hidden + 64 * tile + 16 * wave) / 16;  // this wave's 16 output rows
  TileScales<NB> sc;
  fetch_scales<NB>(g.dn, t16, NB, 0, sc);
  Members<I, NM, 256> mb;
  fetch_members<I, NM, 256, true>(g.ah, g.al, g.ad, 0u, off, ne, mb);
  uint4 a[NB / 2];
  fetch_tile_q8<NB>(g.dn, t16, NB, 0, a);
  store_scales<NB>(sc, sdt[wave]);
  store_members<I, NM, 256>(mb, bh, bl, STR, dx);
  __syncthreads();
  float acc[NM / 16][4];
  mfma_tile<NB, NM>(a, bh, bl, STR, sdt[wave], dx, NB, acc);
  const int grp = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < NM / 16; ct++) {
    const int c = 16 * ct + (lane & 15);
    if (c < ne) {
      const int r0 = 64 * tile + 16 * wave + 4 * grp;
      *reinterpret_cast<float4*>(g.o + (size_t)(off + c) * hidden + r0) =
          make_float4(acc[ct][0], acc[ct][1], acc[ct][2], acc[ct][3]);
    }
  }
}

// ------------------------------------------------------------------------------------------------------------
// y[p][r] = sum over p's experts in list order of w * o[slot][r] (the reference's acc[p] += w * o).
__global__ __launch_bounds__(256) void k_grp_combine(int k, int hidden, GroupBufs g, float* __restrict__ y) {
  const int p = blockIdx.x;
  const int r = blockIdx.y * 256 + threadIdx.x;
  int sl[8];
  float wt[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    sl[j] = j < k ? g.grp[GRP_ORD_SLOT + p * 8 + j] : 0;
    wt[j] = j < k ? __int_as_float(g.grp[GRP_ORD_W + p * 8 + j]) : 0.0f;
  }
  if (r >= hidden) return;
  float ov[8];
#pragma unroll
  for (int j = 0; j < 8; j++) ov[j] = j < k ? g.o[(size_t)sl[j] * hidden + r] : 0.0f;
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++)
    if (j < k) {
      const float tw = wt[j] * ov[j];
      acc = acc + tw;
    }
  y[(size_t)p * hidden + r] = acc;
}

// ------------------------------------------------------------------------------------------------------------

hipError_t launch_grouped_block(hipStream_t s, const LayerDev& L, int m, int k, int inter, const float* x,
                                GroupBufs g, float* y, const hipEvent_t* ev) {
  auto arm = [&](int i) {
    if (ev) arm_launch_events(ev[2 * i], ev[2 * i + 1]);
  };
  const int H = L.gate_up.cols, E = L.router.rows;
  if (m < 1 || m > kGrpMaxPos || k < 1 || k > 8 || E > 64 || L.gate_up.dtype != DT_Q8_0 ||
      L.down.dtype != DT_Q8_0 || L.router.dtype != DT_Q8_0 || L.down.cols != inter || inter % 64 || H % 256 ||
      !g.gu.q || !g.dn.q || g.gu.rows != L.gate_up.rows || g.gu.cols != H || g.dn.rows != L.down.rows ||
      g.dn.cols != inter)
    return hipErrorInvalidValue;
  arm(0);
  switch (H) {
    case 1024:
      klaunch(k_grp_route<DT_Q8_0, 1024, false>, m, kRouteThreads, 0, s, L.router, L.router_bias, x, nullptr, 0.0f, k, g);
      break;
    case 1536:
      klaunch(k_grp_route<DT_Q8_0, 1536, false>, m, kRouteThreads, 0, s, L.router, L.router_bias, x, nullptr, 0.0f, k, g);
      break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if ((e = launch_grp_experts(s, H, E, m, k, inter, g, ev)) != hipSuccess) return e;
  arm(3);
  klaunch(k_grp_combine, dim3(m, H / 256), 256, 0, s, k, H, g, y);
  return hipGetLastError();
}

hipError_t launch_grp_codes(hipStream_t s, int K, int m, const float* x, const GroupBufs& g) {
  if (m < 1 || m > kGrpMaxPos) return hipErrorInvalidValue;
  switch (K) {
    case 1024: klaunch(k_grp_codes<1024>, m, 256, 0, s, x, g); break;
    case 1536: klaunch(k_grp_codes<1536>, m, 256, 0, s, x, g); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_grp_route_norm(hipStream_t s, const LayerDev& L, int m, int k, const float* h, const float* lnw,
                                 float eps, const GroupBufs& g) {
  const int H = L.router.cols;
  if (m < 1 || m > kGrpMaxPos || k < 1 || k > 8 || L.router.rows > 64 || L.router.dtype != DT_Q8_0 || !lnw)
    return hipErrorInvalidValue;
  switch (H) {
    case 1024:
      klaunch(k_grp_route<DT_Q8_0, 1024, true>, m, kRouteThreads, 0, s, L.router, L.router_bias, h, lnw, eps, k, g);
      break;
    case 1536:
      klaunch(k_grp_route<DT_Q8_0, 1536, true>, m, kRouteThreads, 0, s, L.router, L.router_bias, h, lnw, eps, k, g);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_grp_experts(hipStream_t s, int H, int E, int m, int k, int inter, const GroupBufs& g,
                              const hipEvent_t* ev) {
  auto arm = [&](int i) {
    if (ev) arm_launch_events(ev[2 * i], ev[2 * i + 1]);
  };
  if (m < 1 || m > kGrpMaxPos || k < 1 || k > 8 || E > 64 || (H != 1024 && H != 1536) || !g.gu.q || !g.dn.q ||
      g.gu.cols != H || g.gu.rows != E * 2 * inter || g.dn.cols != inter || g.dn.rows != E * H)
    return hipErrorInvalidValue;
  hipError_t e;
  const int U = m * k < E ? m * k : E;
  const bool wide = m > 16;
  // u is the slow grid index, so the workgroups of list indices past the step's expert count (which end at once)
  // are dispatched last
  constexpr int NT = kGrpUpThreads, RT = 16 * NT / 128;
  const dim3 gu_grid(inter / RT, U);
  arm(1);
  if (H == 1024) {
    if (wide) klaunch(k_grp_up<1024, 32, NT>, gu_grid, NT, 0, s, m, k, inter, g);
    else klaunch(k_grp_up<1024, 16, NT>, gu_grid, NT, 0, s, m, k, inter, g);
  } else {
    if (wide) klaunch(k_grp_up<1536, 32, NT>, gu_grid, NT, 0, s, m, k, inter, g);
    else klaunch(k_grp_up<1536, 16, NT>, gu_grid, NT, 0, s, m, k, inter, g);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const dim3 dn_grid(H / 64, U);
  arm(2);
  switch (inter) {
#define DOWN_CASE(II)                                                                               \
  case II:                                                                                          \
    if (wide) klaunch(k_grp_down<II, 32>, dn_grid, 256, 0, s, H, g);                            \
    else klaunch(k_grp_down<II, 16>, dn_grid, 256, 0, s, H, g);                                 \
    break;
    DOWN_CASE(128)
    DOWN_CASE(256)
    DOWN_CASE(512)
#undef DOWN_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace moert

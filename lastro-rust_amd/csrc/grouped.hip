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

#include "attn_dev.h"
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
// Gate/up of list expert u = blockIdx.y for its members [NM z, NM z + NM) (z = blockIdx.z; a workgroup past the
// expert's member count ends at once), rows [RT t, RT t + RT) of gate and of up (t = blockIdx.x, RT = 16 * NT /
// 128): the first half of the waves computes 16 gate rows each, the second half the same up rows, so the members'
// codes staged in LDS serve every wave. Then act = silu(g)*u and its hi/lo codes (each 32 rows are one block of the
// act vector), written to the members' slots. Each member's column and act codes depend on that member alone, so
// the cut of the members into groups of NM changes no result.
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
  const int c0 = NM * blockIdx.z;  // this workgroup's first member
  const int e = plan.list[u], off = plan.offe[e] + c0;
  unsigned bits = plan.bits[e];
  if (__popc(bits) <= c0) return;
  for (int i = 0; i < c0; i++) bits &= bits - 1u;  // the members from c0 on
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
  if (u == 0 && tile == 0 && c0 == 0) publish_plan<NT>(plan, g.w, m, k, g.grp);
}

// ------------------------------------------------------------------------------------------------------------
// Down of list expert u = blockIdx.y for its members [NM z, NM z + NM) (z = blockIdx.z; a workgroup past the
// expert's member count ends at once), output rows [64t, 64t+64): o[slot][row].
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
  const int c0 = NM * blockIdx.z;
  if (g.grp[GRP_CNT + u] <= c0) return;
  const int e = g.grp[GRP_LIST + u], ne = g.grp[GRP_CNT + u] - c0, off = g.grp[GRP_OFF + u] + c0;
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
  const int CH = (m + 15) / 16;  // member groups of 16: a step's expert has at most m members
  // u is the slow grid index, so the workgroups of list indices past the step's expert count (which end at once)
  // are dispatched last
  constexpr int NT = kGrpUpThreads, RT = 16 * NT / 128;
  const dim3 gu_grid(inter / RT, U, CH);
  arm(1);
  if (H == 1024) {
    klaunch(k_grp_up<1024, 16, NT>, gu_grid, NT, 0, s, m, k, inter, g);
  } else {
    klaunch(k_grp_up<1536, 16, NT>, gu_grid, NT, 0, s, m, k, inter, g);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const dim3 dn_grid(H / 64, U, CH);
  arm(2);
  switch (inter) {
#define DOWN_CASE(II)                                                                               \
  case II:                                                                                          \
    klaunch(k_grp_down<II, 16>, dn_grid, 256, 0, s, H, g);                                      \
    break;
    DOWN_CASE(128)
    DOWN_CASE(256)
    DOWN_CASE(512)
#undef DOWN_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------------------
// The block as one launch (launch_grp_fused). Workgroup b runs on XCD x = XCC_ID with index w = b / 8 in it (the
// chip deals the workgroups of a launch round-robin over its 8 XCDs; all 256 are resident at once):
//   R. wave slot s = 8 w + wave of the XCD computes the router dots of position s % 16 with experts s / 16 + 16 i
//      (one batch of rows), shared through the XCD's L2; workgroup w < m of each XCD codes input w into the XCD's
//      copy (k_grp_route's codes), raises its flag, ranks the experts of position w (wave_topk) and shares the ids
//      and weights through the XCD's L2; every workgroup gathers them, builds the grouping (make_plan) and reads the
//      XCD's codes into LDS;
//   U. gate/up item q = 2 b + slot (+512 per round) covers act rows [32 blk, +32) of list expert u = q / 16: 32
//      gate and 32 up rows on four waves, every position an MFMA column; silu(g) * u and its hi/lo codes go out
//      device-wide for the expert's members;
//   D. down tile q = 8 b + wave (+2048 per round) covers output rows [16 t, +16) of list expert u = q / (H / 16);
//      the waves of a workgroup span at most two experts per round, whose members' act codes it gathers into LDS;
//      the members' outputs go out device-wide by member slot;
//   C. workgroup b combines rows [b H / 256, +H / 256) of every position from its k slots in list order.
// Every wait is bounded; one that gives up sets a bit of f.err and the workgroup waits for nothing more.
constexpr int kFbThreads = 512;
constexpr int kFbSpin = 1 << 18;

// The hi/lo codes of one 32-element block (block_codes' arithmetic; 8 lanes, 4 elements each, all lanes taking
// part in the maximum).
__device__ __forceinline__ void code_block(const float (&v)[4], uint32_t& hw, uint32_t& lw, float& d) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float a = fabsf(v[i]);
    amax = a > amax ? a : amax;
  }
  amax = group_max<8>(amax);
  d = amax / 32639.0f;
  hw = 0;
  lw = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int q = d > 0.0f ? (int)__builtin_rintf(v[i] / d) : 0;
    const int h = (q + 128) >> 8;
    hw |= (uint32_t)(uint8_t)(int8_t)h << (8 * i);
    lw |= (uint32_t)(uint8_t)(int8_t)(q - 256 * h) << (8 * i);
  }
}

// Wave-level poll of one record of W entries per lane (entry i at src + S i, device-wide) until every used record
// of the wave carries `epoch`; val gets the values (left unset in a lane that does not use its record). Returns
// false when the poll gave up (at once for spin 0).
template <int W, int S>
__device__ __forceinline__ bool poll_rec(const uint2* src, bool use, unsigned epoch, int spin, unsigned (&val)[W]) {
  for (int it = 0; it < spin; it++) {
    poll_fence();
    bool stale = false;
    if (use) {  // one branch around the whole record: its loads still go out together, unused lanes load nothing
#pragma unroll
      for (int i = 0; i < W; i++) {
        const uint2 e = get_dev(src + S * i);
        val[i] = e.x;
        stale |= e.y != epoch;
      }
    }
    if (__ballot(stale) == 0) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

template <int H>
__global__ __launch_bounds__(kFbThreads) void k_grp_fused(DMat router, const float* __restrict__ bias,
                                                          const float* __restrict__ x, int m, int k, unsigned epoch,
                                                          GroupBufs g, FbBufs f, float* __restrict__ y) {
  using GR = Geo<DT_Q8_0, H>;
  static_assert(GR::RPW == 1, "one router row per wave");
  constexpr int NT = kFbThreads, NW = NT / 64, P = kFbPos, I = kFbInter, AW = kFbActW;
  constexpr int NB = H / 32, NBI = I / 32, STR = H + 16, SA = I + 16;
  constexpr int NTILE = H / 16;                // down tiles (16 rows) of an expert
  constexpr int R = H / 256;                   // combined rows per workgroup
  constexpr int LGN = P * 64;                  // logit entries per XCD
  constexpr int RE = (kFbExperts + 15) / 16;   // router rows per wave
  constexpr int XB = 2 * P * STR, AB = 2 * 2 * P * SA;
  static_assert(NB * 8 <= NT && (NB * 8) % 64 == 0, "one pass of whole waves codes an input");
  static_assert(2 * NBI * P == NT, "one thread per act record of two experts");
  __shared__ __align__(16) int8_t big[XB > AB ? XB : AB];  // the input codes (R, U), then two experts' act codes
  __shared__ float xd_s[P * NB];
  __shared__ float ad_s[2 * P * NBI];
  __shared__ __align__(16) float lgs[64];
  __shared__ int ids_s[P * 8];
  __shared__ float w_s[P * 8];
  __shared__ __align__(16) TopkLds tk;
  __shared__ int rk_ids[8];
  __shared__ float rk_w[8];
  __shared__ Plan plan;
  __shared__ __align__(16) uint16_t sdt[NW][NB * 16];
  __shared__ float gout[2][2][32][P + 1];
  __shared__ int dead_s;

  const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int xc = (int)xcc_id() & 7, w = blockIdx.x >> 3, bid = blockIdx.x;
  const int E = router.rows, grp = lane >> 4;
  // f.err[0]: bits of waits that gave up; f.err[1]: a test mask only the host writes (moert_block_fault_inject):
  // a wait whose bit is set looks for an epoch no launch writes, and every wait polls at most kInjectSpin times
  const auto ew = __builtin_amdgcn_raw_buffer_load_b64(l2_buffer(f.err, 8), 0, 0, kL2Policy);
  const unsigned err0 = __builtin_amdgcn_readfirstlane(ew[0]), inj = __builtin_amdgcn_readfirstlane(ew[1]);
  const int spin_max = inj ? kInjectSpin : kFbSpin;
  auto ep = [&](unsigned bit) { return (inj & bit) ? kNoEpoch : epoch; };
  if (threadIdx.x == 0) dead_s = err0 ? 1 : 0;
  auto fail = [&](bool ok, unsigned bit) {
    if (!ok && lane == 0) {
      if (!dead_s && !err0) atomicOr(f.err, bit);
      dead_s = 1;
    }
  };
  int8_t* xh = big;
  int8_t* xl = big + P * STR;

  // ---- R. router dots: wave slot s of the XCD, position s % 16, experts s / 16 + 16 i, one batch of rows; their
  // loads go out first, and workgroup w < m codes input w into the XCD's copy while they are in flight ----
  const int rs = 8 * w + wid, rp = rs % 16, re0 = rs / 16;
  const bool rwave = rp < m;
  size_t rrow[RE];
  bool rok[RE];
#pragma unroll
  for (int i = 0; i < RE; i++) {
    rok[i] = re0 + 16 * i < E;
    rrow[i] = rok[i] ? (size_t)(re0 + 16 * i) : 0;
  }
  Rows<DT_Q8_0, H, RE> rr;
  XReg<DT_Q8_0, H> xr;
  if (rwave) {
    rows_load<DT_Q8_0, H, RE>(rr, router, rrow, rok, lane);
    load_x<DT_Q8_0, H>(xr, x + (size_t)rp * H, lane);
  }
  const bool coder = w < m && (int)threadIdx.x < NB * 8;
  if (coder) {
    const int b = threadIdx.x / 8, part = threadIdx.x % 8;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = x[(size_t)w * H + 32 * b + 4 * part + e];
    uint32_t hw, lw;
    float d;
    code_block(v, hw, lw, d);
    const size_t row = (size_t)xc * P + w;
    reinterpret_cast<uint32_t*>(f.xh + row * H)[8 * b + part] = hw;
    reinterpret_cast<uint32_t*>(f.xl + row * H)[8 * b + part] = lw;
    if (part == 0) f.xd[row * NB + b] = d;
  }
  if (rwave) {
    float out[RE];
    rows_fma<DT_Q8_0, H, RE>(rr, rok, xr, lane, out);
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < RE; i++)
        if (rok[i]) {
          const int e = re0 + 16 * i;
          const float lv = bias ? out[i] + bias[e] : out[i];
          put_entry(&f.lg[xc * LGN + rp * E + e], __float_as_uint(lv), epoch);
        }
    }
  }
  if (coder) wait_mem();
  __syncthreads();
  if (w < m && threadIdx.x == 0) put_entry(&f.xflag[xc * P + w], 0u, epoch);
  // the top-k of position w, once per XCD: wave 0 of workgroup w < m waits for the position's E logits, ranks them
  // (wave_topk) and shares the ids and weights through the XCD's L2
  if (w < m && wid == 0) {
    int idx[1] = {w * E + (lane < E ? lane : 0)};
    bool use[1] = {lane < E};
    unsigned v[1];
    const __amdgpu_buffer_rsrc_t rl = l2_buffer(f.lg + xc * LGN, LGN * 8);
    const bool ok = poll_m<1>([&](int i) { return l2_load_u64(rl, 8u * (unsigned)i); }, idx, use, ep(1u),
                              dead_s ? 0 : spin_max, v);
    lgs[lane] = __uint_as_float(v[0]);
    fail(ok, 1u);
    wave_lds_sync();
    wave_topk(lgs, E, k, lane, tk, rk_ids, rk_w);
    wave_lds_sync();
    if (lane < k) {
      uint2* rk = f.rk + (size_t)(xc * P + w) * 16;
      put_entry(rk + lane, (unsigned)rk_ids[lane], epoch);
      put_entry(rk + 8 + lane, __float_as_uint(rk_w[lane]), epoch);
    }
  }
  // the XCD's input codes: each wave waits for the m flags itself, then loads its share into registers, which
  // reach LDS after the plan (rows past m are never a member)
  constexpr int XC = (P * (H / 16) + NT - 1) / NT, XD = (P * NB + NT - 1) / NT;
  uint4 xhv[XC], xlv[XC];
  float xdv[XD];
  {
    int idx[1] = {lane < m ? lane : 0};
    bool use[1] = {lane < m};
    unsigned v[1];
    const __amdgpu_buffer_rsrc_t rf = l2_buffer(f.xflag + xc * P, P * 8);
    const bool ok = poll_m<1>([&](int i) { return l2_load_u64(rf, 8u * (unsigned)i); }, idx, use, ep(8u),
                              dead_s ? 0 : spin_max, v);
    fail(ok, 8u);
    const __amdgpu_buffer_rsrc_t rh = l2_buffer(f.xh + (size_t)xc * P * H, P * H);
    const __amdgpu_buffer_rsrc_t rlo = l2_buffer(f.xl + (size_t)xc * P * H, P * H);
    const __amdgpu_buffer_rsrc_t rd = l2_buffer(f.xd + (size_t)xc * P * NB, P * NB * 4);
#pragma unroll
    for (int j = 0; j < XC; j++) {
      const int i = (int)threadIdx.x + j * NT;
      if (i < m * (H / 16)) {
        const auto hv = __builtin_amdgcn_raw_buffer_load_b128(rh, 16 * i, 0, kL2Policy);
        const auto lv = __builtin_amdgcn_raw_buffer_load_b128(rlo, 16 * i, 0, kL2Policy);
        xhv[j] = make_uint4(hv[0], hv[1], hv[2], hv[3]);
        xlv[j] = make_uint4(lv[0], lv[1], lv[2], lv[3]);
      }
    }
#pragma unroll
    for (int j = 0; j < XD; j++) {
      const int i = (int)threadIdx.x + j * NT;
      if (i < m * NB) xdv[j] = l2_load_f32(rd, 4u * (unsigned)i);
    }
  }
  {
    // every workgroup: the ids and weights of the m positions (entry 16 p + j: id j, then weight j - 8); an id is
    // clamped below E so that a wait that gave up (stale entries) keeps every index in range
    const int t = threadIdx.x, p = t / 16, j = t % 16;
    int idx[1] = {t < m * 16 ? t : 0};
    bool use[1] = {t < m * 16 && (j & 7) < k};
    unsigned v[1];
    const __amdgpu_buffer_rsrc_t rr = l2_buffer(f.rk + (size_t)xc * P * 16, P * 16 * 8);
    const bool ok = poll_m<1>([&](int i) { return l2_load_u64(rr, 8u * (unsigned)i); }, idx, use, ep(1u),
                              dead_s ? 0 : spin_max, v);
    if (use[0]) {
      if (j < 8)
        ids_s[p * k + j] = (int)min(v[0], (unsigned)(E - 1));
      else
        w_s[p * k + j - 8] = __uint_as_float(v[0]);
    }
    fail(ok, 1u);
  }
  __syncthreads();
  if (bid == 0)
    for (int i = threadIdx.x; i < m * k; i += NT) {
      g.ids[i] = ids_s[i];
      g.w[i] = w_s[i];
    }
  make_plan<NT>(ids_s, m, k, plan);
  if (bid == 0) publish_plan<NT>(plan, w_s, m, k, g.grp);
  const int nu = plan.nu;
#pragma unroll
  for (int j = 0; j < XC; j++) {
    const int i = (int)threadIdx.x + j * NT;
    if (i < m * (H / 16)) {
      const int row = i / (H / 16), c = i % (H / 16);
      *reinterpret_cast<uint4*>(xh + row * STR + 16 * c) = xhv[j];
      *reinterpret_cast<uint4*>(xl + row * STR + 16 * c) = xlv[j];
    }
  }
#pragma unroll
  for (int j = 0; j < XD; j++) {
    const int i = (int)threadIdx.x + j * NT;
    if (i < m * NB) xd_s[i] = xdv[j];
  }
  __syncthreads();

  // ---- U. gate/up items: two per workgroup and round, four waves each ----
  const int sl = wid >> 2, role = wid & 3;  // item slot; rows [16 (role & 1), +16) of gate (role < 2) or up
  for (int r = 0; r < (nu * 16 + 511) / 512; r++) {
    const int q = 2 * bid + sl + 512 * r;
    const bool has = q < nu * 16;
    const int u = has ? q / 16 : 0, blk = q % 16;
    const int e = plan.list[u];
    const size_t t16 = ((size_t)e * 2 * I + (size_t)(role >> 1) * I + 32 * blk + 16 * (role & 1)) / 16;
    TileScales<NB> sc;
    uint4 a[NB / 2];
    if (has) {
      fetch_scales<NB>(g.gu, t16, NB, 0, sc);
      fetch_tile_q8<NB>(g.gu, t16, NB, 0, a);
    }
    if (has) {
      store_scales<NB>(sc, sdt[wid]);
      float acc[1][4];
      mfma_tile<NB, P>(a, xh, xl, STR, sdt[wid], xd_s, NB, acc);
#pragma unroll
      for (int i = 0; i < 4; i++) gout[sl][role >> 1][16 * (role & 1) + 4 * grp + i][lane & 15] = acc[0][i];
    }
    __syncthreads();
    // act = silu(gate) * up of the two items' members: 8 lanes per (item, position), 4 rows a lane
    if (threadIdx.x < 2 * P * 8) {
      const int ss = threadIdx.x / (P * 8), p = (threadIdx.x / 8) % P, part = threadIdx.x & 7;
      const int qq = 2 * bid + ss + 512 * r;
      const bool hq = qq < nu * 16;
      const int uu = hq ? qq / 16 : 0, bb = qq % 16;
      const bool mem = hq && p < m && ((plan.bits[plan.list[uu]] >> p) & 1u);
      float av[4];
#pragma unroll
      for (int i = 0; i < 4; i++)
        av[i] = mem ? silu_mul(gout[ss][0][4 * part + i][p], gout[ss][1][4 * part + i][p]) : 0.0f;
      uint32_t hw, lw;
      float d;
      code_block(av, hw, lw, d);
      if (mem) {
        uint2* ae = f.act + (size_t)(uu * NBI + bb) * AW * P + p;
        put_dev(ae + part * P, hw, epoch);
        put_dev(ae + (8 + part) * P, lw, epoch);
        if (part == 0) put_dev(ae + 16 * P, __float_as_uint(d), epoch);
      }
    }
    __syncthreads();
  }

  // ---- D. down tiles [T b, +T) of the list's nu * (H / 16) (at most two experts, as T <= H / 16); wave w takes
  // tiles w, w + 8, ..., whose weights it fetches before it gathers the experts' act codes into LDS ----
  {
    constexpr int TMAX = (kFbExperts * NTILE + 255) / 256, JD = (TMAX + NW - 1) / NW;  // tiles per wave at most
    const int total = nu * NTILE, T = (total + 255) / 256;
    const int t0 = min(bid * T, total), t1 = min(t0 + T, total);
    const int u0 = min(t0, total - 1) / NTILE, u1 = t1 > t0 ? (t1 - 1) / NTILE : u0;
    constexpr int JP = JD < 2 ? JD : 2;  // tiles fetched ahead of the gather (a third only past 42 experts)
    TileScales<NBI> sc[JD];
    uint4 a[JD][NBI / 2];
    auto fetch = [&](int j) {
      const int dq = t0 + wid + NW * j;
      if (dq < t1) {
        const int e = plan.list[dq / NTILE];
        const size_t t16 = ((size_t)e * H + 16 * (dq % NTILE)) / 16;
        fetch_scales<NBI>(g.dn, t16, NBI, 0, sc[j]);
        fetch_tile_q8<NBI>(g.dn, t16, NBI, 0, a[j]);
      }
    };
#pragma unroll
    for (int j = 0; j < JP; j++) fetch(j);
    int8_t* ahs = big;
    int8_t* als = big + 2 * P * SA;
    {
      // thread (slot, block, position) gathers the 17 entries of one act record; lanes read consecutive positions
      const int s2 = threadIdx.x / (NBI * P), bb = threadIdx.x / P % NBI, p = threadIdx.x % P;
      const int uu = s2 == 0 ? u0 : u1;
      const bool use = t0 < t1 && (s2 == 0 || u1 != u0) && p < m && ((plan.bits[plan.list[uu]] >> p) & 1u);
      const uint2* src = f.act + (size_t)(uu * NBI + bb) * AW * P + p;
      unsigned v[AW];
      const bool ok = poll_rec<AW, P>(src, use, ep(2u), dead_s ? 0 : spin_max, v);
      if (use) {
        int8_t* row_h = ahs + (s2 * P + p) * SA + 32 * bb;
        int8_t* row_l = als + (s2 * P + p) * SA + 32 * bb;
        *reinterpret_cast<uint4*>(row_h) = make_uint4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<uint4*>(row_h + 16) = make_uint4(v[4], v[5], v[6], v[7]);
        *reinterpret_cast<uint4*>(row_l) = make_uint4(v[8], v[9], v[10], v[11]);
        *reinterpret_cast<uint4*>(row_l + 16) = make_uint4(v[12], v[13], v[14], v[15]);
        ad_s[(s2 * P + p) * NBI + bb] = __uint_as_float(v[16]);
      }
      fail(ok, 2u);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < JD; j++) {
      if (j >= JP) fetch(j);
      const int dq = t0 + wid + NW * j;
      if (dq < t1) {
        const int u = dq / NTILE, t = dq % NTILE, s2 = u == u0 ? 0 : 1;
        const int e = plan.list[u];
        store_scales<NBI>(sc[j], sdt[wid]);
        float acc[1][4];
        mfma_tile<NBI, P>(a[j], ahs + s2 * P * SA, als + s2 * P * SA, SA, sdt[wid], ad_s + s2 * P * NBI, NBI, acc);
        const int p = lane & 15;
        const unsigned bits = plan.bits[e];
        if (p < m && ((bits >> p) & 1u)) {
          const int slot = plan.offe[e] + __popc(bits & ((1u << p) - 1u));
#pragma unroll
          for (int i = 0; i < 4; i++)
            put_dev(&f.o[(size_t)slot * H + 16 * t + 4 * grp + i], __float_as_uint(acc[0][i]), epoch);
        }
      }
    }
  }

  // ---- C. rows [R b, +R) of every position: its k member slots in list order ----
  if ((int)threadIdx.x < m * R) {
    const int p = threadIdx.x / R, row = R * bid + (int)threadIdx.x % R;
    int sls[8];
    float wt[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      sls[jj] = 0;
      wt[jj] = 0.0f;
    }
    for (int j0 = 0; j0 < k; j0++) {
      const int e = ids_s[p * k + j0];
      int rank = 0;
      for (int j1 = 0; j1 < k; j1++) rank += plan.uof[ids_s[p * k + j1]] < plan.uof[e];
      const int slot = plan.offe[e] + __popc(plan.bits[e] & ((1u << p) - 1u));
#pragma unroll
      for (int jj = 0; jj < 8; jj++)
        if (jj == rank) {
          sls[jj] = slot;
          wt[jj] = w_s[p * k + j0];
        }
    }
    int idx[8];
    bool use[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      idx[jj] = sls[jj] * H + row;
      use[jj] = jj < k;
    }
    unsigned v[8];
    const bool ok = poll_m<8>([&](int i) { return get_dev(f.o + i); }, idx, use, ep(4u), dead_s ? 0 : spin_max, v);
    float acc = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 8; jj++)
      if (jj < k) {
        const float tw = wt[jj] * __uint_as_float(v[jj]);
        acc = acc + tw;
      }
    y[(size_t)p * H + row] = acc;
    if (!ok) {
      if (!dead_s && !err0) atomicOr(f.err, 4u);
      dead_s = 1;
    }
  }
}

hipError_t launch_grp_fused(hipStream_t s, const LayerDev& L, int m, int k, int inter, const float* x,
                            const GroupBufs& g, const FbBufs& f, unsigned epoch, float* y, int cus) {
  const int H = L.gate_up.cols, E = L.router.rows;
  if (m < 1 || m > kFbPos || k < 1 || k > 8 || E < 1 || E > kFbExperts || inter != kFbInter || cus != 256 ||
      epoch == 0 || L.gate_up.dtype != DT_Q8_0 || L.down.dtype != DT_Q8_0 || L.router.dtype != DT_Q8_0 ||
      L.router.cols != H || L.down.cols != inter || !g.gu.q || !g.dn.q || g.gu.rows != E * 2 * inter ||
      g.gu.cols != H || g.dn.rows != E * H || g.dn.cols != inter || !f.err || !f.lg || !f.xflag || !f.xh || !f.xl ||
      !f.xd || !f.act || !f.o || !f.rk)
    return hipErrorInvalidValue;
  switch (H) {
    case 1024: klaunch(k_grp_fused<1024>, 256, kFbThreads, 0, s, L.router, L.router_bias, x, m, k, epoch, g, f, y); break;
    case 1536: klaunch(k_grp_fused<1536>, 256, kFbThreads, 0, s, L.router, L.router_bias, x, m, k, epoch, g, f, y); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace moert

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
//   k_grp_route   grid m:            router logits + top-k per position, hi/lo codes of x
//   k_grp_up      grid (U, I/32):    grouping, gate/up MFMA of expert u for its members, SwiGLU, hi/lo codes of act
//   k_grp_down    grid (U, H/64):    down MFMA of expert u for its members -> o[member slot]
//   k_grp_combine grid (m, H/256):   y[p] = ordered sum over p's experts of w * o
#include <climits>

#include "dev_rows.h"
#include "grouped.h"
#include "launch.h"

namespace moert {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kRouteThreads = 512;

// ------------------------------------------------------------------------------------------------------------
// Per-position router (canonical dot, optional bias), top-k, and the hi/lo split of x_p.
template <int DT, int H>
__global__ __launch_bounds__(kRouteThreads) void k_grp_route(DMat router, const float* __restrict__ bias,
                                                             const float* __restrict__ x, int k, GroupBufs g) {
  using G = Geo<DT, H>;
  constexpr int NW = kRouteThreads / 64;
  constexpr int RP = (64 + NW * G::RPW - 1) / (NW * G::RPW);
  __shared__ float xs[H];
  __shared__ __align__(16) float lg[64];
  __shared__ float slot[3 * 64];
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
  for (int q = 0; q < RP; q++) bv[q] = (bias && ok[q]) ? bias[row[q]] : 0.0f;
  wg_copy<H, kRouteThreads>(x + (size_t)p * H, xs);
  XReg<DT, H> xr;
  load_x<DT, H>(xr, xs, sub);
  float out[RP];
  rows_fma<DT, H, RP>(rr, ok, xr, sub, out);
#pragma unroll
  for (int q = 0; q < RP; q++)
    if (ok[q] && sub == 0) lg[row[q]] = bias ? out[q] + bv[q] : out[q];
  // hi/lo codes: 8 lanes per 32-element block, 4 elements per lane
  {
    const int t = threadIdx.x, b = t >> 3, part = t & 7;
    const bool valid = b < H / 32;
    float v[4];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[i] = valid ? xs[32 * b + 4 * part + i] : 0.0f;
      float a = fabsf(v[i]);
      amax = a > amax ? a : amax;
    }
    amax = group_max<8>(amax);
    const float d = amax / 32639.0f;
    uint32_t hw = 0, lw = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int q = d > 0.0f ? (int)__builtin_rintf(v[i] / d) : 0;
      int h = (q + 128) >> 8;
      hw |= (uint32_t)(uint8_t)(int8_t)h << (8 * i);
      lw |= (uint32_t)(uint8_t)(int8_t)(q - 256 * h) << (8 * i);
    }
    if (valid) {
      reinterpret_cast<uint32_t*>(g.xh + (size_t)p * H)[8 * b + part] = hw;
      reinterpret_cast<uint32_t*>(g.xl + (size_t)p * H)[8 * b + part] = lw;
      if (part == 0) g.xd[(size_t)p * (H / 32) + b] = d;
    }
  }
  __syncthreads();
  if (wave == 0) wave_topk(lg, E, k, lane, slot, g.ids + (size_t)p * k, g.w + (size_t)p * k);
}

// ------------------------------------------------------------------------------------------------------------
// Grouping of the m*k routed (position, expert) entries, in LDS: experts in first-appearance order (list index u),
// member counts and offsets. Every thread of the workgroup takes part.
struct GroupLds {
  int se[kGrpMaxPos * 8];  // expert of entry i = p*k + j
  int first[64];           // first entry of expert e (INT_MAX if absent)
  int cnt[64];             // entries of expert e
  int list[64];            // expert of list index u
  int uof[64];             // list index of expert e
  int cntu[64];            // member count of list index u
  int offu[64];            // first member slot of list index u
  int nu;
};

template <int NT>
__device__ __forceinline__ void group_entries(const int* __restrict__ ids, int n, GroupLds& s) {
  const int t = threadIdx.x;
  for (int i = t; i < n; i += NT) s.se[i] = ids[i];
  if (t < 64) {
    s.first[t] = INT_MAX;
    s.cnt[t] = 0;
  }
  if (t == 0) s.nu = 0;
  __syncthreads();
  for (int i = t; i < n; i += NT) {
    atomicMin(&s.first[s.se[i]], i);
    atomicAdd(&s.cnt[s.se[i]], 1);
  }
  __syncthreads();
  if (t < 64 && s.cnt[t] > 0) {
    int u = 0;
    for (int e = 0; e < 64; e++) u += (s.cnt[e] > 0 && s.first[e] < s.first[t]) ? 1 : 0;
    s.list[u] = t;
    s.uof[t] = u;
    s.cntu[u] = s.cnt[t];
    atomicAdd(&s.nu, 1);
  }
  __syncthreads();
  if (t < s.nu) {
    int o = 0;
    for (int u = 0; u < t; u++) o += s.cntu[u];
    s.offu[t] = o;
  }
  __syncthreads();
}

// Positions whose top-k holds expert e, in position order (its members): mp[0, count). Wave 0 only, m <= 32.
__device__ __forceinline__ void member_positions(const GroupLds& s, int e, int m, int k, int* mp) {
  const int lane = threadIdx.x & 63;
  bool has = false;
  if (lane < m)
    for (int j = 0; j < k; j++) has |= s.se[lane * k + j] == e;
  const unsigned long long mask = __ballot(has);
  if (has) mp[__popcll(mask & ((1ull << lane) - 1ull))] = lane;
}

// ------------------------------------------------------------------------------------------------------------
// MFMA tile of one wave: 16 weight rows x NM member columns over NB 32-element blocks.
//   a[b]  : this lane's 8 weight codes of block b (row lane%16, elements 8*(lane/16) .. +8)
//   bh/bl : LDS [NM][stride] hi / lo codes of the members
//   sdt   : LDS [NB][16] fp16 scales of the 16 rows, transposed
//   dx    : LDS [NM][NB] activation scales
// acc[ct][i] = output (row 4*(lane/16) + i, column 16*ct + lane%16).
template <int NB, int NM>
__device__ __forceinline__ void mfma_tile(const uint2 (&a)[NB], const int8_t* bh, const int8_t* bl, int stride,
                                          const uint16_t* sdt, const float* dx, float (&acc)[NM / 16][4]) {
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < NM / 16; ct++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[ct][i] = 0.0f;
#pragma unroll
  for (int b = 0; b < NB; b++) {
    const long av = (long)(((unsigned long long)a[b].y << 32) | a[b].x);
    const uint2 s4 = *reinterpret_cast<const uint2*>(sdt + b * 16 + 4 * grp);
    const float dw[4] = {h2f((uint16_t)(s4.x & 0xffff)), h2f((uint16_t)(s4.x >> 16)), h2f((uint16_t)(s4.y & 0xffff)),
                         h2f((uint16_t)(s4.y >> 16))};
#pragma unroll
    for (int ct = 0; ct < NM / 16; ct++) {
      const int c = 16 * ct + col;
      const uint2 h2 = *reinterpret_cast<const uint2*>(bh + (size_t)c * stride + 32 * b + 8 * grp);
      const uint2 l2 = *reinterpret_cast<const uint2*>(bl + (size_t)c * stride + 32 * b + 8 * grp);
      const long hv = (long)(((unsigned long long)h2.y << 32) | h2.x);
      const long lv = (long)(((unsigned long long)l2.y << 32) | l2.x);
      const v4i z = {0, 0, 0, 0};
      const v4i sh = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, hv, z, 0, 0, 0);
      const v4i sl = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, lv, z, 0, 0, 0);
      const float dxc = dx[c * NB + b];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int S = 256 * sh[i] + sl[i];
        acc[ct][i] = __builtin_fmaf((float)S, dw[i] * dxc, acc[ct][i]);
      }
    }
  }
}

// Loads the 8-byte A-operand pieces of NB blocks of one weight row (Q8_0 payload plane) and stages the row's fp16
// scales into LDS transposed ([b][row-in-tile]).
template <int NB>
__device__ __forceinline__ void load_rows_q8(const DMat& m, size_t row, int r16, uint2 (&a)[NB], uint16_t* sdt) {
  const int grp = (threadIdx.x & 63) >> 4;
  const uint8_t* base = m.q + row * (size_t)m.cols + 8 * grp;
#pragma unroll
  for (int b = 0; b < NB; b++) a[b] = *reinterpret_cast<const uint2*>(base + 32 * b);
  const uint16_t* sc = m.d + row * (size_t)(m.cols / 32);
  for (int b = grp; b < NB; b += 4) sdt[b * 16 + r16] = sc[b];
}

// Member activations into LDS: rows [0, ne) of hi/lo (row length K, padded stride) and their block scales.
template <int K, int NM, int NT>
__device__ __forceinline__ void load_members(const int8_t* __restrict__ srch, const int8_t* __restrict__ srcl,
                                             const float* __restrict__ srcd, const int* rows, int ne, int8_t* bh,
                                             int8_t* bl, int stride, float* dx) {
  constexpr int C16 = K / 16;  // 16-byte chunks per row
  for (int i = threadIdx.x; i < NM * C16; i += NT) {
    const int c = i / C16, j = i % C16;
    uint4 vh = {0, 0, 0, 0}, vl = {0, 0, 0, 0};
    if (c < ne) {
      const size_t r = (size_t)rows[c];
      vh = reinterpret_cast<const uint4*>(srch + r * K)[j];
      vl = reinterpret_cast<const uint4*>(srcl + r * K)[j];
    }
    *reinterpret_cast<uint4*>(bh + (size_t)c * stride + 16 * j) = vh;
    *reinterpret_cast<uint4*>(bl + (size_t)c * stride + 16 * j) = vl;
  }
  for (int i = threadIdx.x; i < NM * (K / 32); i += NT) {
    const int c = i / (K / 32), b = i % (K / 32);
    dx[i] = c < ne ? srcd[(size_t)rows[c] * (K / 32) + b] : 0.0f;
  }
}

// ------------------------------------------------------------------------------------------------------------
// Gate/up of list expert u = blockIdx.x for its members, rows [32t, 32t+32) of gate and of up (t = blockIdx.y):
// wave w computes 16 rows (w & 1) of gate (w < 2) or up (w >= 2). Then act = silu(g)*u and its hi/lo codes (the
// 32 rows are one block of the act vector). Workgroup (0, 0) also publishes the grouping for the later kernels.
template <int H, int NM>
__global__ __launch_bounds__(256) void k_grp_up(DMat gu, int m, int k, int inter, GroupBufs g) {
  constexpr int NB = H / 32;
  constexpr int STR = H + 16;
  __shared__ GroupLds s;
  __shared__ int mp[kGrpMaxPos];
  __shared__ __align__(16) int8_t bh[NM * STR];
  __shared__ __align__(16) int8_t bl[NM * STR];
  __shared__ float dx[NM * NB];
  __shared__ __align__(16) uint16_t sdt[4][NB * 16];
  __shared__ float gout[2][32][NM + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = m * k;
  group_entries<256>(g.ids, n, s);
  const int u = blockIdx.x, tile = blockIdx.y;
  if (u >= s.nu) return;
  const int e = s.list[u], ne = s.cntu[u];
  const int r16 = lane & 15;
  const size_t row = (size_t)e * 2 * inter + (size_t)(wave >> 1) * inter + 32 * tile + 16 * (wave & 1) + r16;
  uint2 a[NB];
  load_rows_q8<NB>(gu, row, r16, a, sdt[wave]);
  if (wave == 0) member_positions(s, e, m, k, mp);
  __syncthreads();
  load_members<H, NM, 256>(g.xh, g.xl, g.xd, mp, ne, bh, bl, STR, dx);
  __syncthreads();
  float acc[NM / 16][4];
  mfma_tile<NB, NM>(a, bh, bl, STR, sdt[wave], dx, acc);
  const int grp = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < NM / 16; ct++)
#pragma unroll
    for (int i = 0; i < 4; i++) gout[wave >> 1][16 * (wave & 1) + 4 * grp + i][16 * ct + (lane & 15)] = acc[ct][i];
  __syncthreads();
  // act = silu(gate) * up for 32 rows x NM members; 8 lanes per member, 4 rows per lane
  for (int base = 0; base < NM; base += 32) {
    const int j = base + (threadIdx.x >> 3), part = threadIdx.x & 7;
    const bool valid = j < ne;
    float av[4];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = 4 * part + i;
      av[i] = valid ? silu_mul(gout[0][r][j < NM ? j : 0], gout[1][r][j < NM ? j : 0]) : 0.0f;
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
      const size_t slot = (size_t)(s.offu[u] + j);
      reinterpret_cast<uint32_t*>(g.ah + slot * inter + 32 * tile)[part] = hw;
      reinterpret_cast<uint32_t*>(g.al + slot * inter + 32 * tile)[part] = lw;
      if (part == 0) g.ad[slot * (inter / 32) + tile] = d;
    }
  }
  if (u == 0 && tile == 0) {
    // grouping for k_grp_down / k_grp_combine: list, counts, offsets, and the member slot of every entry
    const int t = threadIdx.x;
    if (t == 0) g.grp[GRP_NU] = s.nu;
    if (t < 64) {
      g.grp[GRP_LIST + t] = t < s.nu ? s.list[t] : 0;
      g.grp[GRP_CNT + t] = t < s.nu ? s.cntu[t] : 0;
      g.grp[GRP_OFF + t] = t < s.nu ? s.offu[t] : 0;
      g.grp[GRP_UOF + t] = s.cnt[t] > 0 ? s.uof[t] : 0;
    }
    for (int i = t; i < n; i += 256) {
      const int ee = s.se[i], p = i / k;
      int before = 0;  // earlier positions that also route to ee
      for (int q = 0; q < p; q++)
        for (int jj = 0; jj < k; jj++) before += s.se[q * k + jj] == ee;
      g.grp[GRP_SLOT + i] = s.offu[s.uof[ee]] + before;
    }
  }
}

// ------------------------------------------------------------------------------------------------------------
// Down of list expert u = blockIdx.x for its members, output rows [64t, 64t+64): o[slot][row].
template <int I, int NM>
__global__ __launch_bounds__(256) void k_grp_down(DMat dn, int hidden, GroupBufs g) {
  constexpr int NB = I / 32;
  constexpr int STR = I + 16;
  __shared__ int slots[kGrpMaxPos];
  __shared__ __align__(16) int8_t bh[NM * STR];
  __shared__ __align__(16) int8_t bl[NM * STR];
  __shared__ float dx[NM * NB];
  __shared__ __align__(16) uint16_t sdt[4][NB * 16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int u = blockIdx.x, tile = blockIdx.y;
  if (u >= g.grp[GRP_NU]) return;
  const int e = g.grp[GRP_LIST + u], ne = g.grp[GRP_CNT + u], off = g.grp[GRP_OFF + u];
  const int r16 = lane & 15;
  const int r = 64 * tile + 16 * wave + r16;
  uint2 a[NB];
  load_rows_q8<NB>(dn, (size_t)e * hidden + r, r16, a, sdt[wave]);
  if (threadIdx.x < kGrpMaxPos) slots[threadIdx.x] = off + threadIdx.x;
  __syncthreads();
  load_members<I, NM, 256>(g.ah, g.al, g.ad, slots, ne, bh, bl, STR, dx);
  __syncthreads();
  float acc[NM / 16][4];
  mfma_tile<NB, NM>(a, bh, bl, STR, sdt[wave], dx, acc);
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
  __shared__ int ord_slot[8];
  __shared__ float ord_w[8];
  const int p = blockIdx.x, t = threadIdx.x;
  if (t == 0) {
    int us[8], sl[8];
    float ws[8];
    for (int j = 0; j < k; j++) {
      us[j] = g.grp[GRP_UOF + g.ids[p * k + j]];
      sl[j] = g.grp[GRP_SLOT + p * k + j];
      ws[j] = g.w[p * k + j];
    }
    for (int j = 0; j < k; j++) {  // rank by list index (distinct)
      int rank = 0;
      for (int q = 0; q < k; q++) rank += us[q] < us[j];
      ord_slot[rank] = sl[j];
      ord_w[rank] = ws[j];
    }
  }
  __syncthreads();
  const int r = blockIdx.y * 256 + t;
  if (r >= hidden) return;
  float acc = 0.0f;
  for (int j = 0; j < k; j++) {
    const float tw = ord_w[j] * g.o[(size_t)ord_slot[j] * hidden + r];
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
      L.down.dtype != DT_Q8_0 || L.router.dtype != DT_Q8_0 || L.down.cols != inter || inter % 32 || H % 256)
    return hipErrorInvalidValue;
  const int U = m * k < E ? m * k : E;
  const bool wide = m > 16;
  arm(0);
  switch (H) {
    case 1024: klaunch(k_grp_route<DT_Q8_0, 1024>, m, kRouteThreads, 0, s, L.router, L.router_bias, x, k, g); break;
    case 1536: klaunch(k_grp_route<DT_Q8_0, 1536>, m, kRouteThreads, 0, s, L.router, L.router_bias, x, k, g); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 gu_grid(U, inter / 32);
  arm(1);
  if (H == 1024) {
    if (wide) klaunch(k_grp_up<1024, 32>, gu_grid, 256, 0, s, L.gate_up, m, k, inter, g);
    else klaunch(k_grp_up<1024, 16>, gu_grid, 256, 0, s, L.gate_up, m, k, inter, g);
  } else {
    if (wide) klaunch(k_grp_up<1536, 32>, gu_grid, 256, 0, s, L.gate_up, m, k, inter, g);
    else klaunch(k_grp_up<1536, 16>, gu_grid, 256, 0, s, L.gate_up, m, k, inter, g);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const dim3 dn_grid(U, H / 64);
  arm(2);
  switch (inter) {
#define DOWN_CASE(II)                                                                               \
  case II:                                                                                          \
    if (wide) klaunch(k_grp_down<II, 32>, dn_grid, 256, 0, s, L.down, H, g);                        \
    else klaunch(k_grp_down<II, 16>, dn_grid, 256, 0, s, L.down, H, g);                             \
    break;
    DOWN_CASE(128)
    DOWN_CASE(256)
    DOWN_CASE(512)
#undef DOWN_CASE
    default: return hipErrorInvalidValue;
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  arm(3);
  klaunch(k_grp_combine, dim3(m, H / 256), 256, 0, s, k, H, g, y);
  return hipGetLastError();
}

}  // namespace moert

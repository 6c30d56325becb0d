// Oracle: CPU restatement of the reference decode path — test infrastructure only (tests/, smoke(), and
// bench.py's cpu_baseline leg). See oracle.h for the canonical evaluation order it defines.
//
// Reference files followed (paths relative to the reference root):
//   rust/moe-rt/src/model.rs:63-73     inv_freq / rope_cos_sin        -> orc_rope_cos_sin
//   rust/moe-rt/src/model.rs:134-158   embedding, rmsnorm, rope       -> orc_rmsnorm, orc_rope
//   rust/moe-rt/src/model.rs:181-243   CpuSession::step               -> orc_session_step
//   rust/moe-rt/src/block.rs:56-62     HostLayer::forward_cpu         -> orc_moe_block
//   rust/moe-rt/src/block.rs:81-89     Routing::from_logits           -> orc_route
//   rust/moe-rt/src/cpu.rs:30-62       dot (AVX2 FMA accumulation)    -> dot_t (canonical order, FMA)
//   rust/moe-rt/src/cpu.rs:65-68       swiglu                         -> orc_swiglu
//   rust/moe-rt/src/cpu.rs:108-150     Cpu::gemv, Cpu::experts        -> orc_gemv, experts()
//   rust/moe-rt/src/cpu.rs:239-296     Cpu::experts_step              -> orc_experts_step
//   rust/moe-rt/src/pool.rs:96-199     Pool::run (atomic task counter) -> Pool
//   rust/moe-rt/src/gpu.rs:205-292     attn_split / attn_combine      -> orc_attention
//   rust/moe-rt/src/bin/m1b-gulosa.rs:22-24  argmax (last index wins) -> orc_argmax
#include "oracle.h"
#include "pool.h"

#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace {

using orc::Pool;

// Rows per pool task (rust/moe-rt/src/cpu.rs:10).
constexpr int kRowsPerTask = 16;
constexpr int kLanes = 64;
constexpr int kTile = 64;  // attention positions per tile (ATTN_BN, rust/moe-rt/src/gpu_model.rs:19)

inline float bits_f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t f_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

inline float h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  uint32_t e = (h >> 10) & 31, m = h & 1023;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-8f;  // m * 2^-24, exact
    return sign ? -v : v;
  }
  if (e == 31) return bits_f(sign | 0x7f800000u | (m << 13));
  return bits_f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

// f32 -> fp16, round to nearest even.
inline uint16_t f2h(float f) {
  uint32_t x = f_bits(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return sign | 0x7c00 | (ax > 0x7f800000u ? 0x200 : 0);
  if (ax >= 0x477ff000u) return sign | 0x7c00;  // >= 65520 rounds to infinity
  if (ax < 0x38800000u) {                        // below 2^-14: subnormal half
    float r = std::rint(bits_f(ax) * 16777216.0f);  // exact scaling by 2^24, then RNE to an integer
    return sign | (uint16_t)r;
  }
  uint32_t h = (((ax >> 23) - 127 + 15) << 10) | ((ax & 0x7fffffu) >> 13);
  uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return sign | (uint16_t)h;
}

int chunk_elems(int dtype) { return dtype == MOERT_Q8_0 ? 16 : dtype == MOERT_Q4_0 ? 32 : 4; }

size_t row_bytes(int dtype, int cols) {
  if (dtype == MOERT_Q8_0) return (size_t)cols / 32 * 34;
  if (dtype == MOERT_Q4_0) return (size_t)cols / 32 * 18;
  return (size_t)cols * 4;
}

// Dequantise one row into natural order.
void dequant_row(const void* w, int dtype, int cols, size_t row, float* out) {
  const uint8_t* p = (const uint8_t*)w + row * row_bytes(dtype, cols);
  if (dtype == MOERT_F32) {
    std::memcpy(out, p, (size_t)cols * 4);
    return;
  }
  for (int b = 0; b < cols / 32; b++) {
    if (dtype == MOERT_Q8_0) {
      const uint8_t* blk = p + (size_t)b * 34;
      float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
      for (int i = 0; i < 32; i++) out[b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
    } else {
      const uint8_t* blk = p + (size_t)b * 18;
      float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
      for (int i = 0; i < 16; i++) {
        out[b * 32 + i] = (float)((int)(blk[2 + i] & 15) - 8) * d;
        out[b * 32 + 16 + i] = (float)((int)(blk[2 + i] >> 4) - 8) * d;
      }
    }
  }
}

// Lane-transposed layout of a length-K vector for chunk size C: groups of 64 chunks, [e][lane] inside a
// group. Element i of chunk j sits at ((j/64)*C + i)*64 + j%64.
void to_lanes(const float* x, int K, int C, float* t) {
  int nch = K / C;
  for (int j = 0; j < nch; j++) {
    int g = j / kLanes, l = j % kLanes;
    for (int e = 0; e < C; e++) t[((size_t)g * C + e) * kLanes + l] = x[(size_t)j * C + e];
  }
}
size_t lanes_len(int K, int C) { return (size_t)((K / C + kLanes - 1) / kLanes) * C * kLanes; }

// Canonical dot of two lane-transposed vectors.
float dot_t(const float* wt, const float* xt, int K, int C) {
  float acc[kLanes];
  for (int l = 0; l < kLanes; l++) acc[l] = 0.0f;
  int nch = K / C, ng = (nch + kLanes - 1) / kLanes;
  for (int g = 0; g < ng; g++) {
    int nl = nch - g * kLanes < kLanes ? nch - g * kLanes : kLanes;
    for (int e = 0; e < C; e++) {
      const float* a = wt + ((size_t)g * C + e) * kLanes;
      const float* b = xt + ((size_t)g * C + e) * kLanes;
      for (int l = 0; l < nl; l++) acc[l] = std::fmaf(a[l], b[l], acc[l]);
    }
  }
  for (int s = 1; s < kLanes; s *= 2)
    for (int l = 0; l < kLanes; l += 2 * s) acc[l] = acc[l] + acc[l + s];
  return acc[0];
}

// Dequantise one row straight into the lane-transposed layout of to_lanes.
void dequant_row_lanes(const void* w, int dtype, int cols, size_t row, float* t) {
  const uint8_t* p = (const uint8_t*)w + row * row_bytes(dtype, cols);
  int C = chunk_elems(dtype), nch = cols / C;
  for (int j = 0; j < nch; j++) {
    float* o = t + (size_t)(j / kLanes) * C * kLanes + (j % kLanes);
    if (dtype == MOERT_F32) {
      const float* src = (const float*)p + (size_t)j * 4;
      for (int e = 0; e < 4; e++) o[e * kLanes] = src[e];
    } else if (dtype == MOERT_Q8_0) {
      const uint8_t* blk = p + (size_t)(j / 2) * 34;
      float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
      const int8_t* q = (const int8_t*)blk + 2 + (j % 2) * 16;
      for (int e = 0; e < 16; e++) o[e * kLanes] = (float)q[e] * d;
    } else {
      const uint8_t* blk = p + (size_t)j * 18;
      float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
      for (int e = 0; e < 16; e++) {
        o[e * kLanes] = (float)((int)(blk[2 + e] & 15) - 8) * d;
        o[(16 + e) * kLanes] = (float)((int)(blk[2 + e] >> 4) - 8) * d;
      }
    }
  }
}

// A row dotter: x transposed once, rows dequantised into a per-thread buffer.
struct Dotter {
  const void* w;
  int dtype, cols, C;
  std::vector<float> xt;
  Dotter(const void* w_, int dtype_, int cols_, const float* x) : w(w_), dtype(dtype_), cols(cols_) {
    C = chunk_elems(dtype);
    xt.assign(lanes_len(cols, C), 0.0f);
    to_lanes(x, cols, C, xt.data());
  }
  float operator()(size_t row, std::vector<float>& nat, std::vector<float>& wt) const {
    (void)nat;
    wt.resize(xt.size());
    dequant_row_lanes(w, dtype, cols, row, wt.data());
    return dot_t(wt.data(), xt.data(), cols, C);
  }
};

// y[r] = f(r) in 16-row tasks (Cpu::fill_rows, rust/moe-rt/src/cpu.rs:93-105).
void fill_rows(Pool& pool, float* y, size_t rows, const std::function<float(size_t, std::vector<float>&, std::vector<float>&)>& f) {
  size_t tasks = (rows + kRowsPerTask - 1) / kRowsPerTask;
  pool.run(tasks, [&](size_t t) {
    thread_local std::vector<float> nat, wt;
    size_t r0 = t * kRowsPerTask, r1 = r0 + kRowsPerTask < rows ? r0 + kRowsPerTask : rows;
    for (size_t r = r0; r < r1; r++) y[r] = f(r, nat, wt);
  });
}

void gemv(Pool& pool, const void* w, int dtype, int rows, int cols, const float* x, float* y) {
  Dotter d(w, dtype, cols, x);
  fill_rows(pool, y, rows, [&](size_t r, std::vector<float>& nat, std::vector<float>& wt) { return d(r, nat, wt); });
}

inline float silu_mul(float g, float u) { return (g / (1.0f + orc_exp(-g))) * u; }

// Cpu::experts (rust/moe-rt/src/cpu.rs:116-150): gate_up rows of the k experts, SwiGLU, then per output row the
// weighted sum over experts in top-k order.
void experts(Pool& pool, int hidden, int inter, const moert_tensor* gate_up, const moert_tensor* down, const float* x,
             const int* ids, const float* weights, int k, float* y) {
  std::vector<float> a((size_t)k * inter);
  Dotter dg(gate_up->data, gate_up->dtype, hidden, x);
  size_t per = (size_t)(inter + kRowsPerTask - 1) / kRowsPerTask;
  pool.run((size_t)k * per, [&](size_t t) {
    thread_local std::vector<float> nat, wt;
    size_t j = t / per, c = t % per;
    size_t base = (size_t)ids[j] * 2 * inter;
    int r0 = (int)(c * kRowsPerTask), r1 = r0 + kRowsPerTask < inter ? r0 + kRowsPerTask : inter;
    for (int r = r0; r < r1; r++) {
      float g = dg(base + r, nat, wt);
      float u = dg(base + inter + r, nat, wt);
      a[j * inter + r] = silu_mul(g, u);
    }
  });
  int C = chunk_elems(down->dtype);
  std::vector<std::vector<float>> at(k);
  for (int j = 0; j < k; j++) {
    at[j].assign(lanes_len(inter, C), 0.0f);
    to_lanes(&a[(size_t)j * inter], inter, C, at[j].data());
  }
  fill_rows(pool, y, hidden, [&](size_t r, std::vector<float>& nat, std::vector<float>& wt) {
    float acc = 0.0f;
    nat.resize(inter);
    wt.resize(at[0].size());
    for (int j = 0; j < k; j++) {
      dequant_row_lanes(down->data, down->dtype, inter, (size_t)ids[j] * hidden + r, wt.data());
      float t = weights[j] * dot_t(wt.data(), at[j].data(), inter, C);
      acc = acc + t;
    }
    return acc;
  });
}


// fp16 -> f32 for every code, built once.
const float* h2f_table() {
  static std::vector<float> t = [] {
    std::vector<float> v(65536);
    for (uint32_t i = 0; i < 65536; i++) v[i] = h2f((uint16_t)i);
    return v;
  }();
  return t.data();
}

// Split-KV decode attention (rust/moe-rt/src/gpu.rs:205-292) in the canonical order:
//   tiles of 64 positions; split s covers tiles [s*tps, s*tps + tps) of the nb = ceil(len/64) valid ones (tps =
//   tiles per split, fixed for a cache), used = ceil(nb/tps) splits non-empty. In a split, per tile:
//     s_i = (fmaf chain over dims 0..d-1 of q*k_i) * scale for valid positions, -inf otherwise;
//     m' = max(m, max_i s_i); alpha = exp(m - m'); p_i = exp(s_i - m'); ts = pairwise tree of the 64 p_i;
//     l = fmaf(l, alpha, ts); pv_c = fmaf chain over valid i of p_i * v_ic; acc_c = fmaf(acc_c, alpha, pv_c).
//   Combine over blocks s = 0..used-1 in order: M = max m_s; w = exp(m_s - M); den = fmaf(w, l_s, den);
//   num_c = fmaf(w, acc_sc, num_c); out_c = num_c / den.
// The loops run across independent positions (scores) or dims (p.v) innermost, each chain in its own order.
void attention(Pool* pool, const float* q, const uint16_t* k_cache, const uint16_t* v_cache, int heads, int kv_heads,
               int d, int max_len, int len, float scale, int tps, float* out) {
  const float* H2F = h2f_table();
  int G = heads / kv_heads;
  int nb = (len + kTile - 1) / kTile;
  int per = tps;
  int used = (nb + per - 1) / per;
  auto one_head = [&](size_t hh) {
    int h = (int)hh, g = h / G;
    const uint16_t* K = k_cache + (size_t)g * max_len * d;
    const uint16_t* V = v_cache + (size_t)g * max_len * d;
    const float* qh = q + (size_t)h * d;
    std::vector<float> ms(used), ls(used), accs((size_t)used * d), kt((size_t)d * kTile), vt((size_t)kTile * d);
    float sc[kTile], p[kTile], tree[kTile];
    std::vector<float> pv(d);
    for (int s = 0; s < used; s++) {
      float m = -INFINITY, l = 0.0f;
      float* acc = &accs[(size_t)s * d];
      for (int c = 0; c < d; c++) acc[c] = 0.0f;
      int t1 = (s + 1) * per < nb ? (s + 1) * per : nb;
      for (int t = s * per; t < t1; t++) {
        int nv = len - t * kTile < kTile ? len - t * kTile : kTile;
        for (int i = 0; i < nv; i++)
          for (int c = 0; c < d; c++) {
            kt[(size_t)c * kTile + i] = H2F[K[(size_t)(t * kTile + i) * d + c]];
            vt[(size_t)i * d + c] = H2F[V[(size_t)(t * kTile + i) * d + c]];
          }
        float dt[kTile];
        for (int i = 0; i < kTile; i++) dt[i] = 0.0f;
        for (int c = 0; c < d; c++) {
          const float* kr = &kt[(size_t)c * kTile];
          for (int i = 0; i < nv; i++) dt[i] = std::fmaf(qh[c], kr[i], dt[i]);
        }
        float tmax = -INFINITY;
        for (int i = 0; i < kTile; i++) {
          sc[i] = i < nv ? dt[i] * scale : -INFINITY;
          tmax = sc[i] > tmax ? sc[i] : tmax;
        }
        float mn = m > tmax ? m : tmax;
        float alpha = orc_exp(m - mn);
        for (int i = 0; i < kTile; i++) p[i] = orc_exp(sc[i] - mn);
        for (int i = 0; i < kTile; i++) tree[i] = p[i];
        for (int st = 1; st < kTile; st *= 2)
          for (int i = 0; i < kTile; i += 2 * st) tree[i] = tree[i] + tree[i + st];
        l = std::fmaf(l, alpha, tree[0]);
        for (int c = 0; c < d; c++) pv[c] = 0.0f;
        for (int i = 0; i < nv; i++) {
          const float* vr = &vt[(size_t)i * d];
          for (int c = 0; c < d; c++) pv[c] = std::fmaf(p[i], vr[c], pv[c]);
        }
        for (int c = 0; c < d; c++) acc[c] = std::fmaf(acc[c], alpha, pv[c]);
        m = mn;
      }
      ms[s] = m;
      ls[s] = l;
    }
    float M = -INFINITY;
    for (int s = 0; s < used; s++) M = ms[s] > M ? ms[s] : M;
    float den = 0.0f;
    std::vector<float> num(d, 0.0f);
    for (int s = 0; s < used; s++) {
      float w = orc_exp(ms[s] - M);
      den = std::fmaf(w, ls[s], den);
      for (int c = 0; c < d; c++) num[c] = std::fmaf(w, accs[(size_t)s * d + c], num[c]);
    }
    for (int c = 0; c < d; c++) out[(size_t)h * d + c] = num[c] / den;
  };
  if (pool)
    pool->run((size_t)heads, one_head);
  else
    for (int h = 0; h < heads; h++) one_head((size_t)h);
}

}  // namespace

extern "C" {

// exp(x) by Cody-Waite range reduction (x = n ln2 + r, ln2 split in a 15-bit head and a tail) and the degree-7
// Taylor polynomial of e^r on |r| <= ln2/2 (truncation error < 1e-8 relative), in Horner form with FMA; the
// result is 2p * 2^(n-1), both factors exact. Below -86.5 the result is 0 (no subnormal results), above 89 it
// is +inf.
float orc_exp(float x) {
  if (x != x) return x;
  if (x > 89.0f) return INFINITY;
  if (x < -86.5f) return 0.0f;
  float n = std::rint(x * 1.44269504088896341f);
  float r = std::fmaf(-n, 0.693145751953125f, x);
  r = std::fmaf(-n, 1.42860682030941723212e-6f, r);
  float p = 1.98412698412698413e-4f;
  p = std::fmaf(p, r, 1.38888888888888889e-3f);
  p = std::fmaf(p, r, 8.33333333333333333e-3f);
  p = std::fmaf(p, r, 4.16666666666666667e-2f);
  p = std::fmaf(p, r, 1.66666666666666667e-1f);
  p = std::fmaf(p, r, 0.5f);
  p = std::fmaf(p, r, 1.0f);
  p = std::fmaf(p, r, 1.0f);
  int ni = (int)n;
  return (p * 2.0f) * bits_f((uint32_t)(ni - 1 + 127) << 23);
}

void orc_exp_n(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = orc_exp(x[i]);
}
void orc_h2f_n(const uint16_t* h, float* f, size_t n) {
  for (size_t i = 0; i < n; i++) f[i] = h2f(h[i]);
}
void orc_f2h_n(const float* f, uint16_t* h, size_t n) {
  for (size_t i = 0; i < n; i++) h[i] = f2h(f[i]);
}

void orc_dequant(const void* w, int dtype, size_t n, float* out) {
  if (dtype == MOERT_F32) {
    std::memcpy(out, w, n * 4);
    return;
  }
  dequant_row(w, dtype, (int)n, 0, out);
}

float orc_dot(const void* w, int dtype, int cols, size_t row, const float* x) {
  Dotter d(w, dtype, cols, x);
  std::vector<float> nat, wt;
  return d(row, nat, wt);
}

void orc_gemv(const void* w, int dtype, int rows, int cols, const float* x, float* y, int threads) {
  Pool pool(threads);
  gemv(pool, w, dtype, rows, cols, x, y);
}

// rust/moe-rt/src/model.rs:141-145: ms = sum(x^2)/n, r = 1/sqrt(ms + eps), out = w * (x * r). The sum of
// squares uses the canonical order with 16-element chunks (element i in chunk i/16, lane (i/16) % 64).
void orc_rmsnorm(const float* x, const float* w, int n, float eps, float* out) {
  float acc[kLanes];
  for (int l = 0; l < kLanes; l++) acc[l] = 0.0f;
  for (int i = 0; i < n; i++) acc[(i / 16) % kLanes] = std::fmaf(x[i], x[i], acc[(i / 16) % kLanes]);
  for (int s = 1; s < kLanes; s *= 2)
    for (int l = 0; l < kLanes; l += 2 * s) acc[l] = acc[l] + acc[l + s];
  float ss = acc[0];
  float ms = ss / (float)n;
  float r = 1.0f / std::sqrt(ms + eps);
  for (int i = 0; i < n; i++) out[i] = w[i] * (x[i] * r);
}

// rust/moe-rt/src/model.rs:63-73: inv_freq[j] = 1/theta^(2j/d) in f32; cs = [cos(pos*f); sin(pos*f)].
void orc_rope_cos_sin(float theta, int head_dim, int pos, float* cs) {
  int half = head_dim / 2;
  for (int j = 0; j < half; j++) {
    float f = 1.0f / std::pow(theta, (float)(2 * j) / (float)head_dim);
    float a = (float)pos * f;
    cs[j] = std::cos(a);
    cs[half + j] = std::sin(a);
  }
}

// rust/moe-rt/src/model.rs:148-158: rotate_half on the two halves of each head.
void orc_rope(float* x, int n, int head_dim, const float* cs) {
  int half = head_dim / 2;
  for (int h = 0; h < n / head_dim; h++) {
    float* p = x + (size_t)h * head_dim;
    for (int j = 0; j < half; j++) {
      float x1 = p[j], x2 = p[j + half];
      p[j] = x1 * cs[j] - x2 * cs[half + j];
      p[j + half] = x2 * cs[j] + x1 * cs[half + j];
    }
  }
}

// rust/moe-rt/src/block.rs:81-89: order by total_cmp descending, ties to the lower index; truncate to k;
// w_i = exp(l_i - l_top) / sum (sum left to right).
void orc_route(const float* logits, const float* bias, int n, int k, int* ids, float* weights) {
  std::vector<float> l(logits, logits + n);
  if (bias)
    for (int i = 0; i < n; i++) l[i] = l[i] + bias[i];
  auto key = [&](int i) {
    int32_t s = (int32_t)f_bits(l[i]);
    return s >= 0 ? s : (s ^ 0x7fffffff);
  };
  std::vector<int> order(n);
  for (int i = 0; i < n; i++) order[i] = i;
  // insertion sort: stable, so equal keys keep increasing index order
  for (int i = 1; i < n; i++) {
    int v = order[i], j = i - 1;
    while (j >= 0 && key(order[j]) < key(v)) {
      order[j + 1] = order[j];
      j--;
    }
    order[j + 1] = v;
  }
  float top = l[order[0]];
  std::vector<float> ex(k);
  float sum = 0.0f;
  for (int j = 0; j < k; j++) {
    ex[j] = orc_exp(l[order[j]] - top);
    sum = sum + ex[j];
  }
  for (int j = 0; j < k; j++) {
    ids[j] = order[j];
    weights[j] = ex[j] / sum;
  }
}

// The MoE half's rmsnorm and router from partial sums over blocks of 8 rows (the engine's producer/consumer split,
// lastro-rust_amd/csrc/moe_norm.h), rmsnorm model.rs:141-145 + router block.rs:56-62 with r factored out of the dots:
//   per block b: z[e][b] = fmaf chain over t of W[e][8b+t] * (lnw[8b+t] * h[8b+t]); ss[b] = fmaf chain of h^2;
//   per item: block b in lane b % 64, lanes add their blocks in increasing b from +0, then the 64-lane pairwise tree;
//   r = 1/sqrtf(ss/H + eps); xn = lnw * (h * r); logits[e] = z[e] * r (+ bias[e]).
void orc_moe_norm_route(const float* h, const float* lnw, const moert_tensor* router, const float* bias, int H, int E,
                        float eps, float* xn, float* logits) {
  const int nb = H / 8;
  std::vector<float> w((size_t)E * H);
  for (int e = 0; e < E; e++) dequant_row(router->data, router->dtype, H, (size_t)e, &w[(size_t)e * H]);
  auto reduce = [&](const std::function<float(int)>& part) {
    float acc[kLanes];
    for (int l = 0; l < kLanes; l++) acc[l] = 0.0f;
    for (int b = 0; b < nb; b++) acc[b % kLanes] = acc[b % kLanes] + part(b);
    for (int st = 1; st < kLanes; st *= 2)
      for (int l = 0; l < kLanes; l += 2 * st) acc[l] = acc[l] + acc[l + st];
    return acc[0];
  };
  const float ss = reduce([&](int b) {
    float a = 0.0f;
    for (int t = 0; t < 8; t++) a = std::fmaf(h[8 * b + t], h[8 * b + t], a);
    return a;
  });
  const float r = 1.0f / std::sqrt(ss / (float)H + eps);
  for (int i = 0; i < H; i++) xn[i] = lnw[i] * (h[i] * r);
  for (int e = 0; e < E; e++) {
    const float* we = &w[(size_t)e * H];
    const float z = reduce([&](int b) {
      float a = 0.0f;
      for (int t = 0; t < 8; t++) a = std::fmaf(we[8 * b + t], lnw[8 * b + t] * h[8 * b + t], a);
      return a;
    });
    logits[e] = bias ? z * r + bias[e] : z * r;
  }
}

void orc_swiglu(const float* h, int inter, float* a) {
  for (int j = 0; j < inter; j++) a[j] = silu_mul(h[j], h[inter + j]);
}

// max_by(total_cmp) keeps the last of equal maxima (rust/moe-rt/src/bin/m1b-gulosa.rs:22-24).
int orc_argmax(const float* v, int n) {
  if (n <= 0) return 0;
  auto key = [&](int i) {
    int32_t s = (int32_t)f_bits(v[i]);
    return s >= 0 ? s : (s ^ 0x7fffffff);
  };
  int best = 0;
  for (int i = 1; i < n; i++)
    if (key(i) >= key(best)) best = i;
  return best;
}

void orc_moe_block(int hidden, int inter, int n_experts, int k, const moert_tensor* router, const float* bias,
                   const moert_tensor* gate_up, const moert_tensor* down, const float* x, float* y, int* ids,
                   float* weights, int threads) {
  Pool pool(threads);
  std::vector<float> logits(n_experts);
  gemv(pool, router->data, router->dtype, n_experts, hidden, x, logits.data());
  orc_route(logits.data(), bias, n_experts, k, ids, weights);
  experts(pool, hidden, inter, gate_up, down, x, ids, weights, k, y);
}

void orc_attention(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, int heads, int kv_heads,
                   int d, int max_len, int len, float scale, int tiles_per_split, float* out) {
  attention(nullptr, q, k_cache, v_cache, heads, kv_heads, d, max_len, len, scale, tiles_per_split, out);
}

int orc_tiles_per_split(int max_len, int attn_splits) {
  int nbmax = (max_len + kTile - 1) / kTile;
  return (nbmax + attn_splits - 1) / attn_splits;
}

// Cpu::experts_step (rust/moe-rt/src/cpu.rs:239-296): positions grouped per expert in first-appearance order,
// each weight row read once for its members; per position, experts are summed in that list order.
void orc_experts_step(int hidden, int inter, int m, int k, const moert_tensor* gate_up, const moert_tensor* down,
                      const float* x, const int* ids, const float* weights, float* y, int threads) {
  Pool pool(threads);
  std::vector<int> list;                                  // experts in first-appearance order
  std::vector<std::vector<std::pair<int, float>>> members;  // (position, weight)
  for (int p = 0; p < m; p++)
    for (int j = 0; j < k; j++) {
      int e = ids[p * k + j];
      size_t idx = 0;
      while (idx < list.size() && list[idx] != e) idx++;
      if (idx == list.size()) {
        list.push_back(e);
        members.emplace_back();
      }
      members[idx].push_back({p, weights[p * k + j]});
    }
  size_t ne = list.size();
  std::vector<size_t> off(ne);
  size_t tot = 0;
  for (size_t e = 0; e < ne; e++) {
    off[e] = tot;
    tot += members[e].size();
  }
  std::vector<float> a(tot * inter);
  int Cg = chunk_elems(gate_up->dtype), Cd = chunk_elems(down->dtype);
  std::vector<std::vector<float>> xt((size_t)m);
  for (int p = 0; p < m; p++) {
    xt[p].assign(lanes_len(hidden, Cg), 0.0f);
    to_lanes(x + (size_t)p * hidden, hidden, Cg, xt[p].data());
  }
  size_t per = (size_t)(inter + kRowsPerTask - 1) / kRowsPerTask;
  pool.run(ne * per, [&](size_t t) {
    thread_local std::vector<float> nat, wg, wu;
    size_t e = t / per, c = t % per;
    nat.resize(hidden);
    wg.resize(xt[0].size());
    wu.resize(xt[0].size());
    size_t base = (size_t)list[e] * 2 * inter;
    int r0 = (int)(c * kRowsPerTask), r1 = r0 + kRowsPerTask < inter ? r0 + kRowsPerTask : inter;
    for (int r = r0; r < r1; r++) {
      dequant_row_lanes(gate_up->data, gate_up->dtype, hidden, base + r, wg.data());
      dequant_row_lanes(gate_up->data, gate_up->dtype, hidden, base + inter + r, wu.data());
      for (size_t j = 0; j < members[e].size(); j++) {
        const float* xp = xt[members[e][j].first].data();
        a[(off[e] + j) * inter + r] = silu_mul(dot_t(wg.data(), xp, hidden, Cg), dot_t(wu.data(), xp, hidden, Cg));
      }
    }
  });
  std::vector<std::vector<float>> at(tot);
  for (size_t i = 0; i < tot; i++) {
    at[i].assign(lanes_len(inter, Cd), 0.0f);
    to_lanes(&a[i * inter], inter, Cd, at[i].data());
  }
  size_t tasks = (size_t)(hidden + kRowsPerTask - 1) / kRowsPerTask;
  pool.run(tasks, [&](size_t t) {
    thread_local std::vector<float> nat, wt, acc;
    nat.resize(inter);
    wt.resize(lanes_len(inter, Cd));
    acc.assign(m, 0.0f);
    int r0 = (int)(t * kRowsPerTask), r1 = r0 + kRowsPerTask < hidden ? r0 + kRowsPerTask : hidden;
    for (int r = r0; r < r1; r++) {
      for (int p = 0; p < m; p++) acc[p] = 0.0f;
      for (size_t e = 0; e < ne; e++) {
        dequant_row_lanes(down->data, down->dtype, inter, (size_t)list[e] * hidden + r, wt.data());
        for (size_t j = 0; j < members[e].size(); j++) {
          float o = dot_t(wt.data(), at[off[e] + j].data(), inter, Cd);
          int p = members[e][j].first;
          float tw = members[e][j].second * o;
          acc[p] = acc[p] + tw;
        }
      }
      for (int p = 0; p < m; p++) y[(size_t)p * hidden + r] = acc[p];
    }
  });
}

// ------------------------------------------------------------------------------------------------------------
// Grouped (multi-position) expert step in the integer order of the MFMA path. Same structure as Cpu::experts_step
// (rust/moe-rt/src/cpu.rs:239-296): experts in first-appearance order, each weight row used by all positions that
// route to it, y[p] = y[p] + w * o summed in list order. The arithmetic differs from the f32 path only in that
// each activation vector is first split into 15-bit integer codes per 32-element block (orc_quant_hilo), so that
// every block product is an exact integer:
//   S_b = 256 * sum(q * hi) + sum(q * lo),   acc = fmaf((float)S_b, d_w(b) * d_x(b), acc) over blocks b in order.

void orc_quant_hilo(const float* x, int n, int8_t* hi, int8_t* lo, float* d) {
  for (int b = 0; b < n / 32; b++) {
    const float* xb = x + (size_t)b * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
      float a = std::fabs(xb[i]);
      amax = a > amax ? a : amax;
    }
    const float s = amax / 32639.0f;
    d[b] = s;
    for (int i = 0; i < 32; i++) {
      int v = s > 0.0f ? (int)std::rint(xb[i] / s) : 0;
      int h = (v + 128) >> 8;  // floor((v + 128) / 256)
      hi[b * 32 + i] = (int8_t)h;
      lo[b * 32 + i] = (int8_t)(v - 256 * h);
    }
  }
}

namespace {

// Integer codes and fp16 scale of block b of a Q8_0 / Q4_0 row (natural element order).
void block_codes(const void* w, int dtype, int cols, size_t row, int b, int8_t* q, float* d) {
  const uint8_t* p = (const uint8_t*)w + row * row_bytes(dtype, cols);
  if (dtype == MOERT_Q8_0) {
    const uint8_t* blk = p + (size_t)b * 34;
    *d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int i = 0; i < 32; i++) q[i] = (int8_t)blk[2 + i];
  } else {
    const uint8_t* blk = p + (size_t)b * 18;
    *d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int i = 0; i < 16; i++) {
      q[i] = (int8_t)((int)(blk[2 + i] & 15) - 8);
      q[16 + i] = (int8_t)((int)(blk[2 + i] >> 4) - 8);
    }
  }
}

float dot_hilo(const void* w, int dtype, int cols, size_t row, const int8_t* hi, const int8_t* lo, const float* dx) {
  float acc = 0.0f;
  int8_t q[32];
  for (int b = 0; b < cols / 32; b++) {
    float dw;
    block_codes(w, dtype, cols, row, b, q, &dw);
    int32_t sh = 0, sl = 0;
    for (int i = 0; i < 32; i++) {
      sh += (int32_t)q[i] * hi[b * 32 + i];
      sl += (int32_t)q[i] * lo[b * 32 + i];
    }
    const int32_t S = 256 * sh + sl;
    acc = std::fmaf((float)S, dw * dx[b], acc);
  }
  return acc;
}

}  // namespace

float orc_dot_hilo(const void* w, int dtype, int cols, size_t row, const int8_t* hi, const int8_t* lo,
                   const float* dx) {
  return dot_hilo(w, dtype, cols, row, hi, lo, dx);
}

void orc_experts_grouped(int hidden, int inter, int m, int k, const moert_tensor* gate_up, const moert_tensor* down,
                         const float* x, const int* ids, const float* weights, float* y, int threads) {
  Pool pool(threads);
  std::vector<int> list;                                  // experts in first-appearance order
  std::vector<std::vector<std::pair<int, float>>> members;  // (position, weight), position order
  for (int p = 0; p < m; p++)
    for (int j = 0; j < k; j++) {
      int e = ids[p * k + j];
      size_t idx = 0;
      while (idx < list.size() && list[idx] != e) idx++;
      if (idx == list.size()) {
        list.push_back(e);
        members.emplace_back();
      }
      members[idx].push_back({p, weights[p * k + j]});
    }
  const size_t ne = list.size();
  std::vector<size_t> off(ne);
  size_t tot = 0;
  for (size_t e = 0; e < ne; e++) {
    off[e] = tot;
    tot += members[e].size();
  }
  const int HB = hidden / 32, IB = inter / 32;
  std::vector<int8_t> xh((size_t)m * hidden), xl((size_t)m * hidden);
  std::vector<float> xd((size_t)m * HB);
  for (int p = 0; p < m; p++)
    orc_quant_hilo(x + (size_t)p * hidden, hidden, &xh[(size_t)p * hidden], &xl[(size_t)p * hidden], &xd[(size_t)p * HB]);
  std::vector<float> a(tot * inter);
  size_t per = (size_t)(inter + kRowsPerTask - 1) / kRowsPerTask;
  pool.run(ne * per, [&](size_t t) {
    size_t e = t / per, c = t % per;
    size_t base = (size_t)list[e] * 2 * inter;
    int r0 = (int)(c * kRowsPerTask), r1 = r0 + kRowsPerTask < inter ? r0 + kRowsPerTask : inter;
    for (int r = r0; r < r1; r++)
      for (size_t j = 0; j < members[e].size(); j++) {
        size_t p = (size_t)members[e][j].first;
        float g = dot_hilo(gate_up->data, gate_up->dtype, hidden, base + r, &xh[p * hidden], &xl[p * hidden], &xd[p * HB]);
        float u = dot_hilo(gate_up->data, gate_up->dtype, hidden, base + inter + r, &xh[p * hidden], &xl[p * hidden],
                           &xd[p * HB]);
        a[(off[e] + j) * inter + r] = (g / (1.0f + orc_exp(-g))) * u;
      }
  });
  std::vector<int8_t> ah(tot * inter), al(tot * inter);
  std::vector<float> ad(tot * IB);
  for (size_t i = 0; i < tot; i++) orc_quant_hilo(&a[i * inter], inter, &ah[i * inter], &al[i * inter], &ad[i * IB]);
  size_t tasks = (size_t)(hidden + kRowsPerTask - 1) / kRowsPerTask;
  pool.run(tasks, [&](size_t t) {
    thread_local std::vector<float> acc;
    acc.assign(m, 0.0f);
    int r0 = (int)(t * kRowsPerTask), r1 = r0 + kRowsPerTask < hidden ? r0 + kRowsPerTask : hidden;
    for (int r = r0; r < r1; r++) {
      for (int p = 0; p < m; p++) acc[p] = 0.0f;
      for (size_t e = 0; e < ne; e++)
        for (size_t j = 0; j < members[e].size(); j++) {
          size_t i = off[e] + j;
          float o = dot_hilo(down->data, down->dtype, inter, (size_t)list[e] * hidden + r, &ah[i * inter],
                             &al[i * inter], &ad[i * IB]);
          int p = members[e][j].first;
          float tw = members[e][j].second * o;
          acc[p] = acc[p] + tw;
        }
      for (int p = 0; p < m; p++) y[(size_t)p * hidden + r] = acc[p];
    }
  });
}

void orc_moe_block_batched(int hidden, int inter, int experts, int k, const moert_tensor* router, const float* bias,
                           const moert_tensor* gate_up, const moert_tensor* down, int m, const float* x, float* y,
                           int* ids, float* weights, int threads) {
  std::vector<float> logits(experts);
  for (int p = 0; p < m; p++) {
    orc_gemv(router->data, router->dtype, experts, hidden, x + (size_t)p * hidden, logits.data(), 1);
    orc_route(logits.data(), bias, experts, k, ids + (size_t)p * k, weights + (size_t)p * k);
  }
  orc_experts_grouped(hidden, inter, m, k, gate_up, down, x, ids, weights, y, threads);
}

// ------------------------------------------------------------------------------------------------------------
// LRU expert cache replay (the LruSync rule of ExpertCache, rust/moe-rt/src/cache.rs:249-354, as stated by
// reference_lru in rust/moe-rt/tests/model.rs:380-412): one clock tick per (step, layer); every requested key that
// is resident is touched first (pinned for the tick); then, in top-k order, a resident key is a hit, and a missing
// key takes the first free slot, else the slot with the oldest last use among those not used in this tick (lowest
// index on ties), else goes to the CPU. out = {hits, copies, cpu}.
struct orc_lru {
  int layers, experts, slots;
  std::vector<int> skey;                // key held by each slot, -1 when free
  std::vector<unsigned long long> last; // clock of each slot's last use
  std::vector<int> where;               // slot of each key, -1 when not in the pool
  unsigned long long clock = 0, hits = 0, copies = 0, cpu = 0;

  // One tick over the keys of one layer step (or one prefetch): requested keys already in the pool are touched
  // first; then each missing key takes the first free slot, else the least recently used slot not touched at this
  // tick (lowest index on ties), else it is left out (served by the CPU). Counted in hits / copies / cpu only when
  // `counted` (a decode step's request, not a prefetch).
  void tick(int layer, const int* ids, int n, bool counted, int* copied) {
    clock++;
    for (int j = 0; j < n; j++) {
      const int sl = where[(size_t)layer * experts + ids[j]];
      if (sl >= 0) last[sl] = clock;
    }
    int nc = 0;
    for (int j = 0; j < n; j++) {
      const int key = layer * experts + ids[j];
      if (where[key] >= 0) {
        if (counted) hits++;
        continue;
      }
      int v = -1;
      for (int i = 0; i < slots && v < 0; i++)
        if (skey[i] < 0) v = i;
      if (v < 0)
        for (int i = 0; i < slots; i++)
          if (last[i] < clock && (v < 0 || last[i] < last[v])) v = i;
      if (v < 0) {
        if (counted) cpu++;
        continue;
      }
      if (skey[v] >= 0) where[skey[v]] = -1;
      skey[v] = key;
      last[v] = clock;
      where[key] = v;
      nc++;
      if (counted) copies++;
    }
    if (copied) *copied = nc;
  }
};

orc_lru* orc_lru_create(int layers, int experts, int slots) {
  if (layers < 1 || experts < 1 || slots < 1) return nullptr;
  orc_lru* c = new orc_lru;
  c->layers = layers;
  c->experts = experts;
  c->slots = slots;
  c->skey.assign(slots, -1);
  c->last.assign(slots, 0);
  c->where.assign((size_t)layers * experts, -1);
  return c;
}

void orc_lru_destroy(orc_lru* c) { delete c; }

void orc_lru_step_layer(orc_lru* c, int layer, const int* ids, int k) { c->tick(layer, ids, k, true, nullptr); }

int orc_lru_prefetch(orc_lru* c, int layer, const int* ids, int n) {
  int copied = 0;
  c->tick(layer, ids, n, false, &copied);
  return copied;
}

// ExpertCache::fill (rust/moe-rt/src/cache.rs:212-227): in key order, every key not in the pool takes the first free
// slot, stamped with the current clock (copy_on_compute, rust/moe-rt/src/cache/core.rs:366-377); stops when no slot
// is free. The clock does not advance and nothing is counted.
int orc_lru_fill(orc_lru* c) {
  int copied = 0;
  for (int key = 0; key < c->layers * c->experts; key++) {
    if (c->where[key] >= 0) continue;
    int v = -1;
    for (int i = 0; i < c->slots && v < 0; i++)
      if (c->skey[i] < 0) v = i;
    if (v < 0) break;
    c->skey[v] = key;
    c->last[v] = c->clock;
    c->where[key] = v;
    copied++;
  }
  return copied;
}

void orc_lru_stats(const orc_lru* c, unsigned long long* out) {
  out[0] = c->hits;
  out[1] = c->copies;
  out[2] = c->cpu;
}

void orc_lru_slots(const orc_lru* c, int* keys) {
  for (int i = 0; i < c->slots; i++) keys[i] = c->skey[i];
}

void orc_lru_replay(const int* routes, int steps, int layers, int k, int experts, int slots,
                    unsigned long long* out) {
  orc_lru* c = orc_lru_create(layers, experts, slots);
  for (int st = 0; st < steps; st++)
    for (int l = 0; l < layers; l++) orc_lru_step_layer(c, l, routes + ((size_t)st * layers + l) * k, k);
  orc_lru_stats(c, out);
  orc_lru_destroy(c);
}

struct orc_session {
  moert_config cfg;
  moert_model_weights w;
  std::vector<moert_layer_weights> layers;
  int max_len, tps, pos;
  Pool* pool;
  std::vector<std::vector<uint16_t>> kc, vc;  // per layer [kv_heads, max_len, d]
};

int orc_session_create(const moert_config* cfg, const moert_model_weights* w, int max_len, int attn_splits,
                       int threads, orc_session** out) {
  if (!cfg || !w || !out || max_len <= 0 || attn_splits <= 0 || cfg->heads % cfg->kv_heads != 0) return MOERT_E_CONFIG;
  orc_session* s = new orc_session;
  s->cfg = *cfg;
  s->w = *w;
  s->layers.assign(w->layers, w->layers + cfg->layers);
  s->w.layers = s->layers.data();
  s->max_len = max_len;
  s->tps = orc_tiles_per_split(max_len, attn_splits);
  s->pos = 0;
  s->pool = new Pool(threads);
  size_t kv = (size_t)cfg->kv_heads * max_len * cfg->head_dim;
  s->kc.assign(cfg->layers, std::vector<uint16_t>(kv, 0));
  s->vc.assign(cfg->layers, std::vector<uint16_t>(kv, 0));
  *out = s;
  return MOERT_OK;
}

void orc_session_destroy(orc_session* s) {
  if (!s) return;
  delete s->pool;
  delete s;
}

void orc_session_set_pos(orc_session* s, int pos) { s->pos = pos; }
int orc_session_pos(orc_session* s) { return s->pos; }

int orc_session_kv_prefill(orc_session* s, int layer, const uint16_t* k, const uint16_t* v, int n) {
  const moert_config& c = s->cfg;
  if (layer < 0 || layer >= c.layers || n < 0 || n > s->max_len) return MOERT_E_RANGE;
  for (int g = 0; g < c.kv_heads; g++)
    for (int p = 0; p < n; p++)
      for (int i = 0; i < c.head_dim; i++) {
        size_t src = ((size_t)g * n + p) * c.head_dim + i, dst = ((size_t)g * s->max_len + p) * c.head_dim + i;
        s->kc[layer][dst] = k[src];
        s->vc[layer][dst] = v[src];
      }
  return MOERT_OK;
}

int orc_session_read_kv(orc_session* s, int layer, uint16_t* k, uint16_t* v, int n) {
  const moert_config& c = s->cfg;
  if (layer < 0 || layer >= c.layers || n < 0 || n > s->max_len) return MOERT_E_RANGE;
  for (int g = 0; g < c.kv_heads; g++)
    for (int p = 0; p < n; p++)
      for (int i = 0; i < c.head_dim; i++) {
        size_t dst = ((size_t)g * n + p) * c.head_dim + i, src = ((size_t)g * s->max_len + p) * c.head_dim + i;
        k[dst] = s->kc[layer][src];
        v[dst] = s->vc[layer][src];
      }
  return MOERT_OK;
}

// rust/moe-rt/src/model.rs:181-243, with the fp16 KV cache and split-KV attention of the build.
int orc_session_step(orc_session* s, int token, float* logits, int* route_ids, float* route_weights, float* hidden) {
  const moert_config& c = s->cfg;
  if (s->pos >= s->max_len) return MOERT_E_FULL;
  if (token < 0 || token >= c.vocab) return MOERT_E_RANGE;
  Pool& pool = *s->pool;
  int H = c.hidden, d = c.head_dim, qd = c.heads * d, kvd = c.kv_heads * d, I = c.inter, k = c.top_k;
  std::vector<float> cs(d), x(H), xn(H), q(qd), kk(kvd), vv(kvd), att(qd), o(H), rl(c.experts), y(H);
  std::vector<int> ids(k);
  std::vector<float> wts(k);
  orc_rope_cos_sin(c.rope_theta, d, s->pos, cs.data());
  dequant_row(s->w.embed.data, s->w.embed.dtype, H, (size_t)token, x.data());
  for (int i = 0; i < H; i++) x[i] = x[i] * c.embedding_multiplier;
  for (int l = 0; l < c.layers; l++) {
    const moert_layer_weights& L = s->layers[l];
    orc_rmsnorm(x.data(), L.ln_attn, H, c.eps, xn.data());
    gemv(pool, L.q.data, L.q.dtype, qd, H, xn.data(), q.data());
    gemv(pool, L.k.data, L.k.dtype, kvd, H, xn.data(), kk.data());
    gemv(pool, L.v.data, L.v.dtype, kvd, H, xn.data(), vv.data());
    orc_rope(q.data(), qd, d, cs.data());
    orc_rope(kk.data(), kvd, d, cs.data());
    for (int g = 0; g < c.kv_heads; g++)
      for (int i = 0; i < d; i++) {
        size_t dst = ((size_t)g * s->max_len + s->pos) * d + i;
        s->kc[l][dst] = f2h(kk[g * d + i]);
        s->vc[l][dst] = f2h(vv[g * d + i]);
      }
    attention(s->pool, q.data(), s->kc[l].data(), s->vc[l].data(), c.heads, c.kv_heads, d, s->max_len, s->pos + 1,
              c.attention_multiplier, s->tps, att.data());
    gemv(pool, L.o.data, L.o.dtype, H, qd, att.data(), o.data());
    for (int i = 0; i < H; i++) x[i] = x[i] + c.residual_multiplier * o[i];
    orc_moe_norm_route(x.data(), L.ln_moe, &L.router, L.router_bias, H, c.experts, c.eps, xn.data(), rl.data());
    orc_route(rl.data(), nullptr, c.experts, k, ids.data(), wts.data());
    experts(pool, H, I, &L.gate_up, &L.down, xn.data(), ids.data(), wts.data(), k, y.data());
    for (int i = 0; i < H; i++) x[i] = x[i] + c.residual_multiplier * y[i];
    if (route_ids)
      for (int j = 0; j < k; j++) route_ids[l * k + j] = ids[j];
    if (route_weights)
      for (int j = 0; j < k; j++) route_weights[l * k + j] = wts[j];
  }
  if (hidden) std::memcpy(hidden, x.data(), (size_t)H * 4);
  if (logits) {
    orc_rmsnorm(x.data(), s->w.norm, H, c.eps, xn.data());
    gemv(pool, s->w.embed.data, s->w.embed.dtype, c.vocab, H, xn.data(), logits);
    for (int v = 0; v < c.vocab; v++) logits[v] = logits[v] / c.logits_scaling;
  }
  s->pos++;
  return MOERT_OK;
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------------------
// The grouped mode of the engine's multi-position step (moert_batched_mode 1): n <= 32 consecutive positions through
// every layer with each weight GEMM on 15-bit activation codes (the block prefill of rust/moe-rt/src/cuda_dense.rs:
// 236-288 and motor/leitura.rs:79-85, with the arithmetic of rust/moe-rt/src/cpu.rs:239-296 for the experts). Per
// layer and position p, in this order:
//   1. xn = rmsnorm(h_p, ln_attn) in the 256-thread order of norm_codes_256 below, then its codes (orc_quant_hilo);
//   2. each q/k/v row: dot_hilo_quarters (the row's blocks cut into four quarters, each an fmaf chain over its
//      blocks of (float)S_b * (d_w * d_x), the quarters added in order); rows (j, j + 32) of a head rotated as RoPE
//      at position p (x1 c - x2 s, x2 c + x1 s); K and V rounded to fp16 into the cache;
//   3. split-KV attention over the first pos0 + p + 1 positions (the decode order);
//   4. the codes of the attention output, then h_p += res * dot_hilo_quarters(o row, codes);
//   5. xn = rmsnorm(h_p, ln_moe) in the 1024-thread order of norm_1024 below; router logits = canonical dot (+ bias),
//      Routing::from_logits; the experts of all n positions grouped (orc_experts_grouped: codes of xn, exact block
//      products, first-appearance list order); h_p += res * y_p.
// Then the final norm, tied head and logits_scaling of the last position, in the decode order.
namespace {

// Sum of squares over h[0, H) as 256 threads hold it: thread t the elements 1024 j + 4 t + i (j, then i, in
// increasing order, those below H), each an fmaf chain from +0; the 64 sums of a wave through the pairwise lane
// tree; the 4 wave sums added in order.
float ss_256(const float* h, int H) {
  float wsum[4];
  for (int w = 0; w < 4; w++) {
    float lane[kLanes];
    for (int l = 0; l < kLanes; l++) {
      const int t = 64 * w + l;
      float ss = 0.0f;
      for (int j = 0; j < (H + 1023) / 1024; j++)
        for (int i = 0; i < 4; i++) {
          const int e = 1024 * j + 4 * t + i;
          const float v = e < H ? h[e] : 0.0f;
          ss = std::fmaf(v, v, ss);
        }
      lane[l] = ss;
    }
    for (int st = 1; st < kLanes; st *= 2)
      for (int l = 0; l < kLanes; l += 2 * st) lane[l] = lane[l] + lane[l + st];
    wsum[w] = lane[0];
  }
  return ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
}

// The same over 1024 threads (16 waves): thread t the elements t, t + 1024, ..., the 16 wave sums added in order
// from +0.
float ss_1024(const float* h, int H) {
  float tot = 0.0f;
  for (int w = 0; w < 16; w++) {
    float lane[kLanes];
    for (int l = 0; l < kLanes; l++) {
      float ss = 0.0f;
      for (int e = 64 * w + l; e < H; e += 1024) ss = std::fmaf(h[e], h[e], ss);
      lane[l] = ss;
    }
    for (int st = 1; st < kLanes; st *= 2)
      for (int l = 0; l < kLanes; l += 2 * st) lane[l] = lane[l] + lane[l + st];
    tot = tot + lane[0];
  }
  return tot;
}

void norm_with(const float* h, const float* lnw, int H, float eps, float ss, float* xn) {
  const float r = 1.0f / std::sqrt(ss / (float)H + eps);
  for (int i = 0; i < H; i++) xn[i] = lnw[i] * (h[i] * r);
}

float dot_hilo_quarters(const void* w, int dtype, int cols, size_t row, const int8_t* hi, const int8_t* lo,
                        const float* dx) {
  const int NB = cols / 32, NBW = NB / 4;
  int8_t q[32];
  float part[4];
  for (int kq = 0; kq < 4; kq++) {
    float acc = 0.0f;
    for (int b = kq * NBW; b < (kq + 1) * NBW; b++) {
      float dw;
      block_codes(w, dtype, cols, row, b, q, &dw);
      int32_t sh = 0, sl = 0;
      for (int i = 0; i < 32; i++) {
        sh += (int32_t)q[i] * hi[b * 32 + i];
        sl += (int32_t)q[i] * lo[b * 32 + i];
      }
      const int32_t S = 256 * sh + sl;
      acc = std::fmaf((float)S, dw * dx[b], acc);
    }
    part[kq] = acc;
  }
  return ((part[0] + part[1]) + part[2]) + part[3];
}

}  // namespace

extern "C" {

float orc_dot_hilo_quarters(const void* w, int dtype, int cols, size_t row, const int8_t* hi, const int8_t* lo,
                            const float* dx) {
  return dot_hilo_quarters(w, dtype, cols, row, hi, lo, dx);
}

void orc_rmsnorm_threads(const float* h, const float* lnw, int H, float eps, int threads, float* xn) {
  norm_with(h, lnw, H, eps, threads == 1024 ? ss_1024(h, H) : ss_256(h, H), xn);
}

int orc_session_step_grouped(orc_session* s, const int* tokens, int n, float* logits, int* route_ids,
                             float* route_weights, float* hidden) {
  const moert_config& c = s->cfg;
  if (n < 1 || n > 32) return MOERT_E_CONFIG;
  if (s->pos + n > s->max_len) return MOERT_E_FULL;
  for (int p = 0; p < n; p++)
    if (tokens[p] < 0 || tokens[p] >= c.vocab) return MOERT_E_RANGE;
  if (c.head_dim != 64 || (c.hidden % 128) || ((c.heads * 64) % 128)) return MOERT_E_CONFIG;
  Pool& pool = *s->pool;
  const int H = c.hidden, d = c.head_dim, qd = c.heads * d, k = c.top_k, E = c.experts, pos0 = s->pos;
  const int HB = H / 32, QB = qd / 32;
  std::vector<float> h((size_t)n * H), xn((size_t)n * H), q((size_t)n * qd), att((size_t)n * qd), cs(d), lg(E),
      y((size_t)n * H);
  std::vector<int8_t> xh((size_t)n * std::max(H, qd)), xl((size_t)n * std::max(H, qd));
  std::vector<float> xd((size_t)n * std::max(HB, QB));
  std::vector<int> ids((size_t)n * k);
  std::vector<float> wts((size_t)n * k);
  for (int p = 0; p < n; p++) {
    dequant_row(s->w.embed.data, s->w.embed.dtype, H, (size_t)tokens[p], &h[(size_t)p * H]);
    for (int i = 0; i < H; i++) h[(size_t)p * H + i] = h[(size_t)p * H + i] * c.embedding_multiplier;
  }
  const int nh = c.heads + 2 * c.kv_heads;
  for (int l = 0; l < c.layers; l++) {
    const moert_layer_weights& L = s->layers[l];
    // 1. norm codes of every position
    for (int p = 0; p < n; p++) {
      float* xp = &xn[(size_t)p * H];
      norm_with(&h[(size_t)p * H], L.ln_attn, H, c.eps, ss_256(&h[(size_t)p * H], H), xp);
      orc_quant_hilo(xp, H, &xh[(size_t)p * H], &xl[(size_t)p * H], &xd[(size_t)p * HB]);
    }
    // 2. q/k/v with RoPE and the KV append, one task per (head, position)
    pool.run((size_t)nh * n, [&](size_t t) {
      const int head = (int)(t / n), p = (int)(t % n), pos = pos0 + p;
      const moert_tensor& W = head < c.heads ? L.q : head < c.heads + c.kv_heads ? L.k : L.v;
      const int hr = head < c.heads ? head : head < c.heads + c.kv_heads ? head - c.heads : head - c.heads - c.kv_heads;
      float rc[64];
      orc_rope_cos_sin(c.rope_theta, d, pos, rc);
      const int8_t* ph = &xh[(size_t)p * H];
      const int8_t* pl = &xl[(size_t)p * H];
      const float* pd = &xd[(size_t)p * HB];
      for (int jp = 0; jp < 32; jp++) {
        const float x1 = dot_hilo_quarters(W.data, W.dtype, H, (size_t)hr * 64 + jp, ph, pl, pd);
        const float x2 = dot_hilo_quarters(W.data, W.dtype, H, (size_t)hr * 64 + jp + 32, ph, pl, pd);
        const float co = rc[jp], sn = rc[32 + jp];
        if (head < c.heads) {
          float* qv = &q[(size_t)p * qd + head * 64];
          qv[jp] = x1 * co - x2 * sn;
          qv[jp + 32] = x2 * co + x1 * sn;
        } else if (head < c.heads + c.kv_heads) {
          uint16_t* kp = &s->kc[l][((size_t)hr * s->max_len + pos) * 64];
          kp[jp] = f2h(x1 * co - x2 * sn);
          kp[jp + 32] = f2h(x2 * co + x1 * sn);
        } else {
          uint16_t* vp = &s->vc[l][((size_t)hr * s->max_len + pos) * 64];
          vp[jp] = f2h(x1);
          vp[jp + 32] = f2h(x2);
        }
      }
    });
    // 3. attention of every position over its causal length
    for (int p = 0; p < n; p++)
      attention(s->pool, &q[(size_t)p * qd], s->kc[l].data(), s->vc[l].data(), c.heads, c.kv_heads, d, s->max_len,
                pos0 + p + 1, c.attention_multiplier, s->tps, &att[(size_t)p * qd]);
    // 4. output projection on the attention output's codes, residual
    for (int p = 0; p < n; p++)
      orc_quant_hilo(&att[(size_t)p * qd], qd, &xh[(size_t)p * qd], &xl[(size_t)p * qd], &xd[(size_t)p * QB]);
    pool.run((size_t)n * ((H + 15) / 16), [&](size_t t) {
      const int p = (int)(t % n), r0 = (int)(t / n) * 16;
      for (int r = r0; r < r0 + 16 && r < H; r++) {
        const float o = dot_hilo_quarters(L.o.data, L.o.dtype, qd, (size_t)r, &xh[(size_t)p * qd],
                                          &xl[(size_t)p * qd], &xd[(size_t)p * QB]);
        float& hv = h[(size_t)p * H + r];
        hv = hv + c.residual_multiplier * o;
      }
    });
    // 5. router of each position on its own rmsnorm, then the experts of all positions grouped
    for (int p = 0; p < n; p++) {
      float* xp = &xn[(size_t)p * H];
      norm_with(&h[(size_t)p * H], L.ln_moe, H, c.eps, ss_1024(&h[(size_t)p * H], H), xp);
      for (int e = 0; e < E; e++) lg[e] = orc_dot(L.router.data, L.router.dtype, H, (size_t)e, xp);
      orc_route(lg.data(), L.router_bias, E, k, &ids[(size_t)p * k], &wts[(size_t)p * k]);
    }
    orc_experts_grouped(H, c.inter, n, k, &L.gate_up, &L.down, xn.data(), ids.data(), wts.data(), y.data(),
                        pool.threads());
    for (size_t i = 0; i < (size_t)n * H; i++) h[i] = h[i] + c.residual_multiplier * y[i];
    for (int p = 0; p < n; p++)
      for (int j = 0; j < k; j++) {
        if (route_ids) route_ids[((size_t)p * c.layers + l) * k + j] = ids[(size_t)p * k + j];
        if (route_weights) route_weights[((size_t)p * c.layers + l) * k + j] = wts[(size_t)p * k + j];
      }
  }
  const float* last = &h[(size_t)(n - 1) * H];
  if (hidden) std::memcpy(hidden, last, (size_t)H * 4);
  if (logits) {
    orc_rmsnorm(last, s->w.norm, H, c.eps, xn.data());
    gemv(pool, s->w.embed.data, s->w.embed.dtype, c.vocab, H, xn.data(), logits);
    for (int v = 0; v < c.vocab; v++) logits[v] = logits[v] / c.logits_scaling;
  }
  s->pos += n;
  return MOERT_OK;
}

}  // extern "C"

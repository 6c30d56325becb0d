// CPU port of the reference's CPU decode path, timed as bench.py's CPU baseline. Test infrastructure, like the
// rest of oracle/: nothing in the product links or calls it.
//
// oracle.cpp fixes the canonical evaluation order that the GPU kernels share (its results are compared bit for
// bit). This file instead keeps the reference's own arithmetic shape, so that its speed is that of the reference CPU
// path on the same weights (paths relative to rust/moe-rt/src):
//   cpu.rs:30-52     dot_avx2: four 8-lane accumulators, 32 elements per iteration, horizontal sum
//                    (acc0 + acc1) + (acc2 + acc3), then the 128-bit halves, movehl, shuffle; the BF16 shift that
//                    widens a weight is replaced by the block dequantisation q * d of the Q8_0 / Q4_0 formats
//   cpu.rs:17-27     dot_scalar for what is left after the 32-element steps (f32 rows only)
//   cpu.rs:65-68     swiglu with libm expf
//   cpu.rs:93-150    fill_rows / gemv / experts: 16-row tasks on the pool, two dispatches per MoE layer
//   model.rs:141-158 rmsnorm (sequential sum of squares), rotate_half rope
//   model.rs:181-243 CpuSession::step: f32 KV cache [position][kv * d] per layer, attention per query head on the
//                    calling thread (scores, maximum, exp, sum, weighted V rows), residuals, tied head / scaling
//   block.rs:56-89   forward_cpu: router gemv, Routing::from_logits (stable sort by total order, ties to the lower
//                    index; softmax over the k)
//   pool.rs:96-199   Pool (pool.h)
// Its results agree with the oracle's within float rounding (tests/test_cpu_port.py), not bit for bit.
#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "oracle.h"
#include "pool.h"

namespace {

constexpr size_t kRowsPerTask = 16;  // cpu.rs:10

float h2f_port(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = s;
    } else {  // subnormal: normalise
      int k = -1;
      uint32_t mm = m;
      do {
        k++;
        mm <<= 1;
      } while (!(mm & 1024u));
      u = s | ((uint32_t)(127 - 15 - k) << 23) | ((mm & 1023u) << 13);
    }
  } else if (e == 31) {
    u = s | 0x7f800000u | (m << 13);
  } else {
    u = s | ((e + 127 - 15) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

size_t row_bytes(int dtype, int cols) {
  if (dtype == MOERT_Q8_0) return (size_t)cols / 32 * 34;
  if (dtype == MOERT_Q4_0) return (size_t)cols / 32 * 18;
  return (size_t)cols * 4;
}

// The horizontal sum of dot_avx2.
inline float hsum(const __m256 acc[4]) {
  __m256 s = _mm256_add_ps(_mm256_add_ps(acc[0], acc[1]), _mm256_add_ps(acc[2], acc[3]));
  __m128 t = _mm_add_ps(_mm256_castps256_ps128(s), _mm256_extractf128_ps(s, 1));
  t = _mm_add_ps(t, _mm_movehl_ps(t, t));
  t = _mm_add_ss(t, _mm_shuffle_ps(t, t, 1));
  return _mm_cvtss_f32(t);
}

// Row `row` of a [rows, n] matrix against x: dot_avx2's accumulation, 32 elements (one quantisation block) per step.
float dot_row(const void* w, int dtype, int n, size_t row, const float* x) {
  const uint8_t* p = (const uint8_t*)w + row * row_bytes(dtype, n);
  __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
  if (dtype == MOERT_F32) {
    const float* r = (const float*)p;
    int i = 0;
    for (; i + 32 <= n; i += 32)
      for (int j = 0; j < 4; j++)
        acc[j] = _mm256_fmadd_ps(_mm256_loadu_ps(r + i + 8 * j), _mm256_loadu_ps(x + i + 8 * j), acc[j]);
    // dot_scalar on the tail: four accumulators over groups of 4, then the remainder
    float a4[4] = {0, 0, 0, 0}, tail = 0.0f;
    int t = i;
    for (; t + 4 <= n; t += 4)
      for (int j = 0; j < 4; j++) a4[j] += r[t + j] * x[t + j];
    for (; t < n; t++) tail += r[t] * x[t];
    return hsum(acc) + (a4[0] + a4[1] + a4[2] + a4[3] + tail);
  }
  const int nb = n / 32;
  if (dtype == MOERT_Q8_0) {
    for (int b = 0; b < nb; b++) {
      const uint8_t* blk = p + (size_t)b * 34;
      const __m256 d = _mm256_set1_ps(h2f_port((uint16_t)(blk[0] | (blk[1] << 8))));
      for (int j = 0; j < 4; j++) {
        const __m128i raw = _mm_loadl_epi64((const __m128i*)(blk + 2 + 8 * j));
        const __m256 wf = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(raw)), d);
        acc[j] = _mm256_fmadd_ps(wf, _mm256_loadu_ps(x + 32 * b + 8 * j), acc[j]);
      }
    }
  } else {  // Q4_0: elements 0..15 in the low nibbles of the 16 bytes, 16..31 in the high ones
    const __m128i lo4 = _mm_set1_epi8(15), eight = _mm_set1_epi8(8);
    for (int b = 0; b < nb; b++) {
      const uint8_t* blk = p + (size_t)b * 18;
      const __m256 d = _mm256_set1_ps(h2f_port((uint16_t)(blk[0] | (blk[1] << 8))));
      const __m128i q = _mm_loadu_si128((const __m128i*)(blk + 2));
      const __m128i lo = _mm_sub_epi8(_mm_and_si128(q, lo4), eight);
      const __m128i hi = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(q, 4), lo4), eight);
      const __m128i parts[4] = {lo, _mm_srli_si128(lo, 8), hi, _mm_srli_si128(hi, 8)};
      for (int j = 0; j < 4; j++) {
        const __m256 wf = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(parts[j])), d);
        acc[j] = _mm256_fmadd_ps(wf, _mm256_loadu_ps(x + 32 * b + 8 * j), acc[j]);
      }
    }
  }
  return hsum(acc);
}

// Cpu::fill_rows: y[r] = f(r) in 16-row tasks.
template <class F>
void fill_rows(orc::Pool& pool, float* y, size_t rows, const F& f) {
  const size_t tasks = (rows + kRowsPerTask - 1) / kRowsPerTask;
  pool.run(tasks, [&](size_t t) {
    const size_t r0 = t * kRowsPerTask, r1 = std::min(rows, r0 + kRowsPerTask);
    for (size_t r = r0; r < r1; r++) y[r] = f(r);
  });
}

void gemv(orc::Pool& pool, const moert_tensor& w, int rows, int cols, const float* x, float* y) {
  fill_rows(pool, y, (size_t)rows, [&](size_t r) { return dot_row(w.data, w.dtype, cols, r, x); });
}

std::vector<float> rmsnorm(const std::vector<float>& x, const float* w, float eps) {
  float ss = 0.0f;
  for (float v : x) ss += v * v;
  const float ms = ss / (float)x.size();
  const float r = 1.0f / std::sqrt(ms + eps);
  std::vector<float> out(x.size());
  for (size_t i = 0; i < x.size(); i++) out[i] = w[i] * (x[i] * r);
  return out;
}

void rope(std::vector<float>& x, int d, const std::vector<float>& cs) {
  const int half = d / 2;
  for (size_t h0 = 0; h0 + d <= x.size(); h0 += d)
    for (int j = 0; j < half; j++) {
      const float x1 = x[h0 + j], x2 = x[h0 + j + half];
      x[h0 + j] = x1 * cs[j] - x2 * cs[half + j];
      x[h0 + j + half] = x2 * cs[j] + x1 * cs[half + j];
    }
}

// total_cmp's key: the IEEE total order as a signed integer.
inline int32_t total_key(float f) {
  int32_t i;
  std::memcpy(&i, &f, 4);
  return i ^ (int32_t)((uint32_t)(i >> 31) >> 1);
}

}  // namespace

struct port_session {
  moert_config c;
  moert_model_weights w;
  std::vector<moert_layer_weights> layers;
  int max_len = 0, pos = 0;
  std::vector<std::vector<float>> kc, vc;  // [layer][max_len * kv * d]
  orc::Pool* pool = nullptr;
  ~port_session() { delete pool; }
};

extern "C" {

int port_session_create(const moert_config* cfg, const moert_model_weights* w, int max_len, int threads,
                        port_session** out) {
  if (!cfg || !w || !out || max_len < 1 || threads < 1 || cfg->heads % cfg->kv_heads) return -2;
  auto* s = new port_session;
  s->c = *cfg;
  s->layers.assign(w->layers, w->layers + cfg->layers);
  s->w = *w;
  s->w.layers = s->layers.data();
  s->max_len = max_len;
  const size_t kvd = (size_t)cfg->kv_heads * cfg->head_dim;
  s->kc.assign(cfg->layers, std::vector<float>((size_t)max_len * kvd, 0.0f));
  s->vc.assign(cfg->layers, std::vector<float>((size_t)max_len * kvd, 0.0f));
  s->pool = new orc::Pool(threads);
  *out = s;
  return 0;
}

void port_session_destroy(port_session* s) { delete s; }

void port_session_set_pos(port_session* s, int pos) { s->pos = pos; }

// Positions [0, n) of layer `layer` from fp16 rows in the engine's layout [kv_heads][n][head_dim].
int port_session_kv_prefill(port_session* s, int layer, const uint16_t* k, const uint16_t* v, int n) {
  const moert_config& c = s->c;
  if (layer < 0 || layer >= c.layers || n < 0 || n > s->max_len) return -2;
  const int d = c.head_dim, kvd = c.kv_heads * d;
  for (int g = 0; g < c.kv_heads; g++)
    for (int p = 0; p < n; p++)
      for (int i = 0; i < d; i++) {
        const size_t src = ((size_t)g * n + p) * d + i, dst = (size_t)p * kvd + g * d + i;
        s->kc[layer][dst] = h2f_port(k[src]);
        s->vc[layer][dst] = h2f_port(v[src]);
      }
  return 0;
}

// CpuSession::step (model.rs:181-243) at the session's position; logits [vocab] (may be null), routes [layers][k].
int port_session_step(port_session* s, int token, float* logits, int* route_ids, float* route_weights) {
  const moert_config& c = s->c;
  if (token < 0 || token >= c.vocab || s->pos >= s->max_len) return -2;
  orc::Pool& pool = *s->pool;
  const int H = c.hidden, I = c.inter, d = c.head_dim, E = c.experts, K = c.top_k;
  const int qd = c.heads * d, kvd = c.kv_heads * d, group = c.heads / c.kv_heads;
  std::vector<float> cs(d);
  orc_rope_cos_sin(c.rope_theta, d, s->pos, cs.data());
  // embedding row times the multiplier
  std::vector<float> x(H), row(H);
  orc_dequant((const uint8_t*)s->w.embed.data + (size_t)token * row_bytes(s->w.embed.dtype, H), s->w.embed.dtype,
              (size_t)H, row.data());
  for (int i = 0; i < H; i++) x[i] = row[i] * c.embedding_multiplier;
  std::vector<float> q(qd), k(kvd), v(kvd), att(qd), o(H), lg(E), y(H), hgu, a;
  std::vector<float> scores;
  const int len = s->pos + 1;
  for (int l = 0; l < c.layers; l++) {
    const moert_layer_weights& L = s->layers[l];
    std::vector<float> xn = rmsnorm(x, L.ln_attn, c.eps);
    gemv(pool, L.q, qd, H, xn.data(), q.data());
    gemv(pool, L.k, kvd, H, xn.data(), k.data());
    gemv(pool, L.v, kvd, H, xn.data(), v.data());
    rope(q, d, cs);
    rope(k, d, cs);
    std::memcpy(&s->kc[l][(size_t)s->pos * kvd], k.data(), (size_t)kvd * 4);
    std::memcpy(&s->vc[l][(size_t)s->pos * kvd], v.data(), (size_t)kvd * 4);
    const float* kc = s->kc[l].data();
    const float* vc = s->vc[l].data();
    scores.resize(len);
    std::fill(att.begin(), att.end(), 0.0f);
    for (int hq = 0; hq < c.heads; hq++) {
      const int kvh = hq / group;
      const float* qh = &q[(size_t)hq * d];
      float mx = -INFINITY;
      for (int p = 0; p < len; p++) {
        const float* kr = kc + (size_t)p * kvd + kvh * d;
        float dt = 0.0f;
        for (int i = 0; i < d; i++) dt += qh[i] * kr[i];
        scores[p] = dt * c.attention_multiplier;
        mx = std::max(mx, scores[p]);
      }
      float sum = 0.0f;
      for (int p = 0; p < len; p++) {
        scores[p] = std::exp(scores[p] - mx);
        sum += scores[p];
      }
      float* out = &att[(size_t)hq * d];
      for (int p = 0; p < len; p++) {
        const float* vr = vc + (size_t)p * kvd + kvh * d;
        const float wgt = scores[p] / sum;
        for (int i = 0; i < d; i++) out[i] += wgt * vr[i];
      }
    }
    gemv(pool, L.o, H, qd, att.data(), o.data());
    for (int i = 0; i < H; i++) x[i] += c.residual_multiplier * o[i];
    xn = rmsnorm(x, L.ln_moe, c.eps);
    // forward_cpu: router, Routing::from_logits, Cpu::experts
    gemv(pool, L.router, E, H, xn.data(), lg.data());
    if (L.router_bias)
      for (int e = 0; e < E; e++) lg[e] += L.router_bias[e];
    std::vector<int> order(E);
    for (int e = 0; e < E; e++) order[e] = e;
    std::stable_sort(order.begin(), order.end(),
                     [&](int a2, int b2) { return total_key(lg[a2]) > total_key(lg[b2]); });
    const float top = lg[order[0]];
    float ex[64], esum = 0.0f;
    for (int j = 0; j < K; j++) {
      ex[j] = std::exp(lg[order[j]] - top);
      esum += ex[j];
    }
    float wts[64];
    for (int j = 0; j < K; j++) wts[j] = ex[j] / esum;
    // dispatch 1: the 2I gate/up rows of each routed expert
    hgu.assign((size_t)K * 2 * I, 0.0f);
    const size_t per = (2 * (size_t)I + kRowsPerTask - 1) / kRowsPerTask;
    const size_t gu_rows = 2 * (size_t)I;
    pool.run((size_t)K * per, [&](size_t t) {
      const size_t j = t / per, ch = t % per;
      const size_t r0 = ch * kRowsPerTask, r1 = std::min(gu_rows, r0 + kRowsPerTask);
      const size_t base = (size_t)order[j] * gu_rows;
      for (size_t r = r0; r < r1; r++) hgu[j * gu_rows + r] = dot_row(L.gate_up.data, L.gate_up.dtype, H, base + r, xn.data());
    });
    a.assign((size_t)K * I, 0.0f);
    for (int j = 0; j < K; j++)
      for (int i = 0; i < I; i++) {
        const float g = hgu[(size_t)j * 2 * I + i], u = hgu[(size_t)j * 2 * I + I + i];
        a[(size_t)j * I + i] = g / (1.0f + std::exp(-g)) * u;
      }
    // dispatch 2: each output row sums the experts in top-k order
    fill_rows(pool, y.data(), (size_t)H, [&](size_t r) {
      float acc = 0.0f;
      for (int j = 0; j < K; j++)
        acc += wts[j] * dot_row(L.down.data, L.down.dtype, I, (size_t)order[j] * H + r, &a[(size_t)j * I]);
      return acc;
    });
    for (int i = 0; i < H; i++) x[i] += c.residual_multiplier * y[i];
    for (int j = 0; j < K; j++) {
      if (route_ids) route_ids[l * K + j] = order[j];
      if (route_weights) route_weights[l * K + j] = wts[j];
    }
  }
  if (logits) {
    std::vector<float> xn = rmsnorm(x, s->w.norm, c.eps);
    gemv(pool, s->w.embed, c.vocab, H, xn.data(), logits);
    for (int t = 0; t < c.vocab; t++) logits[t] /= c.logits_scaling;
  }
  s->pos++;
  return 0;
}

// One row's dot in the port's order, for its pin against float64.
float port_dot(const void* w, int dtype, int cols, size_t row, const float* x) { return dot_row(w, dtype, cols, row, x); }

}  // extern "C"

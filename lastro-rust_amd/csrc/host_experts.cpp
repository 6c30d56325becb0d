// Host expert FFN of the hybrid (host_experts.h).
#include "host_experts.h"

#include <math.h>

#include "../../include/moert.h"
#include "host_utils.h"

namespace moert {

namespace {

typedef float f8 __attribute__((vector_size(32)));

// sum of the 8 lanes
inline float hsum(f8 v) {
  return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

// row . x for row `row` of a matrix of `cols` columns stored as a payload plane q and a scale plane d: per 32-element
// block, the block's weights (codes, exact in f32) times x in 8 lanes, then times the block scale
template <int DT>
float row_dot_t(const uint8_t* q, const uint16_t* d, int cols, size_t row, const float* x) {
  f8 acc = {0, 0, 0, 0, 0, 0, 0, 0};
  if (DT == MOERT_F32) {
    const float* wr = (const float*)q + row * cols;
    for (int i = 0; i < cols; i += 8) {
      f8 a, b;
      __builtin_memcpy(&a, wr + i, 32);
      __builtin_memcpy(&b, x + i, 32);
      acc += a * b;
    }
    return hsum(acc);
  }
  const int nb = cols / 32;
  const uint16_t* s = d + row * (size_t)nb;
  const uint8_t* p = DT == MOERT_Q8_0 ? q + row * (size_t)cols : q + row * (size_t)(cols / 2);
  for (int b = 0; b < nb; b++) {
    float wv[32];
    if (DT == MOERT_Q8_0) {
      const int8_t* c = (const int8_t*)p + 32 * b;
      for (int j = 0; j < 32; j++) wv[j] = (float)c[j];
    } else {
      const uint8_t* c = p + 16 * b;
      for (int j = 0; j < 16; j++) {
        wv[j] = (float)((c[j] & 15) - 8);
        wv[j + 16] = (float)((c[j] >> 4) - 8);
      }
    }
    f8 blk = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < 32; j += 8) {
      f8 a, xv;
      __builtin_memcpy(&a, wv + j, 32);
      __builtin_memcpy(&xv, x + 32 * b + j, 32);
      blk += a * xv;
    }
    const float sc = host_h2f(s[b]);
    acc += blk * sc;
  }
  return hsum(acc);
}

// the same compiled for AVX2 + FMA, chosen at run time when the host has them
template <int DT>
__attribute__((target("avx2,fma"))) float row_dot_avx2(const uint8_t* q, const uint16_t* d, int cols, size_t row,
                                                         const float* x) {
  return row_dot_t<DT>(q, d, cols, row, x);
}

float row_dot(const uint8_t* q, const uint16_t* d, int dtype, int cols, size_t row, const float* x) {
  static const bool avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
  switch (dtype) {
    case MOERT_F32:
      return avx2 ? row_dot_avx2<MOERT_F32>(q, d, cols, row, x) : row_dot_t<MOERT_F32>(q, d, cols, row, x);
    case MOERT_Q8_0:
      return avx2 ? row_dot_avx2<MOERT_Q8_0>(q, d, cols, row, x) : row_dot_t<MOERT_Q8_0>(q, d, cols, row, x);
    default:
      return avx2 ? row_dot_avx2<MOERT_Q4_0>(q, d, cols, row, x) : row_dot_t<MOERT_Q4_0>(q, d, cols, row, x);
  }
}

}  // namespace

void host_experts_layer(const HostRecordGeo& g, const uint8_t* const* recs, const float* w, int n, const float* x,
                        float* act, float* y, int threads) {
  if (n <= 0) return;
  const size_t I = (size_t)g.inter, H = (size_t)g.hidden;
  // gate and up rows of every expert: item t = e * I + i
  parallel_for_n((size_t)n * I, 32, threads, [&](size_t a, size_t b) {
    for (size_t t = a; t < b; t++) {
      const size_t e = t / I, i = t % I;
      const uint8_t* gq = recs[e];
      const uint16_t* gd = (const uint16_t*)(recs[e] + g.gu_q);
      const float gv = row_dot(gq, gd, g.dtype, g.hidden, i, x);
      const float uv = row_dot(gq, gd, g.dtype, g.hidden, I + i, x);
      act[t] = gv / (1.0f + expf(-gv)) * uv;
    }
  });
  // down rows: y[r] += w[e] * (down_r . act[e]) in expert order
  parallel_for_n(H, 64, threads, [&](size_t a, size_t b) {
    for (size_t r = a; r < b; r++) {
      float acc = y[r];
      for (int e = 0; e < n; e++) {
        const uint8_t* dq = recs[e] + g.gu_q + g.gu_d;
        const uint16_t* dd = (const uint16_t*)(dq + g.dn_q);
        acc += w[e] * row_dot(dq, dd, g.dtype, g.inter, r, act + (size_t)e * I);
      }
      y[r] = acc;
    }
  });
}

}  // namespace moert

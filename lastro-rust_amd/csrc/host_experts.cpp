// Host expert FFN of the hybrid (host_experts.h).
#include "host_experts.h"

#include <math.h>

#include "../../include/moert.h"
#include "host_utils.h"

namespace moert {

namespace {

// row . x for row `row` of a matrix of `cols` columns stored as a payload plane q and a scale plane d
float row_dot(const uint8_t* q, const uint16_t* d, int dtype, int cols, size_t row, const float* x) {
  float sum = 0.0f;
  if (dtype == MOERT_F32) {
    const float* w = (const float*)q + row * cols;
    for (int i = 0; i < cols; i++) sum += w[i] * x[i];
    return sum;
  }
  const int nb = cols / 32;
  const uint16_t* s = d + row * (size_t)nb;
  if (dtype == MOERT_Q8_0) {
    const int8_t* p = (const int8_t*)q + row * (size_t)cols;
    for (int b = 0; b < nb; b++) {
      float sb = 0.0f;
      for (int j = 0; j < 32; j++) sb += (float)p[32 * b + j] * x[32 * b + j];
      sum += host_h2f(s[b]) * sb;
    }
    return sum;
  }
  const uint8_t* p = q + row * (size_t)(cols / 2);
  for (int b = 0; b < nb; b++) {
    float sb = 0.0f;
    for (int j = 0; j < 16; j++) {
      const int v = p[16 * b + j];
      sb += (float)((v & 15) - 8) * x[32 * b + j] + (float)((v >> 4) - 8) * x[32 * b + j + 16];
    }
    sum += host_h2f(s[b]) * sb;
  }
  return sum;
}

}  // namespace

void host_expert_ffn(const uint8_t* rec, int dtype, int hidden, int inter, size_t gu_q, size_t gu_d, size_t dn_q,
                     const float* x, float w, float* act, float* y, int threads) {
  const uint8_t* gq = rec;
  const uint16_t* gd = (const uint16_t*)(rec + gu_q);
  const uint8_t* dq = rec + gu_q + gu_d;
  const uint16_t* dd = (const uint16_t*)(rec + gu_q + gu_d + dn_q);
  parallel_for_n((size_t)inter, 64, threads, [&](size_t a, size_t b) {
    for (size_t i = a; i < b; i++) {
      const float g = row_dot(gq, gd, dtype, hidden, i, x);
      const float u = row_dot(gq, gd, dtype, hidden, (size_t)inter + i, x);
      act[i] = g / (1.0f + expf(-g)) * u;
    }
  });
  parallel_for_n((size_t)hidden, 128, threads, [&](size_t a, size_t b) {
    for (size_t r = a; r < b; r++) y[r] += w * row_dot(dq, dd, dtype, inter, r, act);
  });
}

}  // namespace moert

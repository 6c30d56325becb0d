// Multi-position step of the whole model (prefill.hip): device buffers and launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "grouped.h"
#include "kernels.h"

namespace moert {

constexpr int kPfMaxPos = 32;  // positions per step (the reference's block limit, cuda_backend.rs:272-274)

// Device buffers of one multi-position step, sized for kPfMaxPos positions.
struct PfBufs {
  int* toks;     // [m] tokens of the positions
  int* pos0;     // [1] first position of the step (the length every attention length is counted from)
  float* h;      // [m, H] residual streams
  float* q;      // [m, heads*d] queries
  float* att;    // [m, heads*d] attention outputs
  float* part;   // [m, heads, splits, 2 + d] split-KV partials
  float* zpart;  // [m, kNormItems] MoE-norm partials of each position (moe_norm.h)
  float* xn;     // [m, H] rmsnorm of h before the experts
  int* ids;      // [m, k] routed experts, top-k order
  float* w;      // [m, k] routing weights
  float* act;    // [m, k, I] SwiGLU activations
  float* o;      // [m, k, H] expert outputs
};

hipError_t launch_embed_b(hipStream_t s, const DMat& emb, const Dims& d, const PfBufs& p, int nv);
// One layer for positions pos0 .. pos0 + nv - 1 (*lenp == pos0 on the device), rope: the [max_len, 64] table; the
// per-row FMA kernels, whose results equal nv decode steps bit for bit.
hipError_t launch_layer_b(hipStream_t s, const LayerDev& L, const Dims& d, const PfBufs& p, const int* lenp, int pos0,
                          int nv, const float* rope);
// The same layer in grouped mode: q/k/v, output projection and experts through the int8 MFMA kernels of grouped.h,
// g holding the layer's tiled matrices. On entry g's codes are those of rmsnorm(h, L.ln_attn) (launch_norm_codes or
// the previous layer's combine); with next_lnw the layer leaves the codes of rmsnorm(h, next_lnw) for the next one.
hipError_t launch_layer_grouped(hipStream_t s, const LayerDev& L, const Dims& d, const PfBufs& p, const int* lenp,
                                int pos0, int nv, const float* rope, const GroupBufs& g, const float* next_lnw);

}  // namespace moert

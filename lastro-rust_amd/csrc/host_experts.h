// Experts computed on the host (the host-CPU hybrid): the SwiGLU FFN of a layer's host-served experts, from their
// records in the pinned host store, added with their routing weights into y in top-k order. Replaces
// HostExperts::compute for a layer's missed experts (rust/moe-rt/src/cpu.rs:116-148: gate and up rows dotted with
// the normalised input, silu(g) * u, down rows dotted with that, weighted sum in top-k order).
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace moert {

// Record layout [gate/up payload | gate/up scales | down payload | down scales] (gu_q, gu_d, dn_q bytes, the rest),
// rows of GGML blocks split into payload and fp16 scale planes; dtype MOERT_F32 / Q8_0 / Q4_0.
struct HostRecordGeo {
  int dtype, hidden, inter;
  size_t gu_q, gu_d, dn_q;
};

// For the n experts recs[0..n) (in top-k order) with weights w: act[e][i] = silu(gate_i . x) * (up_i . x), then
// y[r] += w[e] * (down_r . act[e]) for e = 0 .. n-1 in order. act is scratch of n * inter floats. Two parallel
// passes over `threads` threads (rows of every expert, then output rows).
void host_experts_layer(const HostRecordGeo& g, const uint8_t* const* recs, const float* w, int n, const float* x,
                        float* act, float* y, int threads);

}  // namespace moert

// Experts computed on the host (the host-CPU hybrid): one expert's SwiGLU FFN from its record in the pinned host
// store, added with its routing weight into y. Replaces HostExperts::compute for a layer's missed experts
// (rust/moe-rt/src/cpu.rs:116-148: gate and up rows dotted with the normalised input, silu(g) * u, down rows dotted
// with that, weighted sum in top-k order).
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace moert {

// Record layout [gate/up payload | gate/up scales | down payload | down scales] (gu_q, gu_d, dn_q bytes, the rest),
// rows of GGML blocks split into payload and fp16 scale planes; dtype MOERT_F32 / Q8_0 / Q4_0.
// y[r] += w * (down_r . act) with act[i] = silu(gate_i . x) * (up_i . x); act is scratch of `inter` floats.
void host_expert_ffn(const uint8_t* rec, int dtype, int hidden, int inter, size_t gu_q, size_t gu_d, size_t dn_q,
                     const float* x, float w, float* act, float* y, int threads);

}  // namespace moert

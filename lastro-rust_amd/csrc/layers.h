// Every layer of a decode step in one launch (layers.hip): per-layer parameters and the exchange areas.
#pragma once
#include "kernels.h"

namespace moert {

constexpr int kPxThreads = 1024;

// One layer's weights and cache as the launch reads them (a device array of these, built at create).
struct PxLayer {
  DMat qkv, o, router, gu, dn;
  const float* ln_attn;
  const float* ln_moe;
  const float* bias;  // router bias or null
  uint16_t* kc;
  uint16_t* vc;
};

// Exchange area of one XCD's workgroups (entries: value bits, epoch): the MoE-norm items (router dots of the
// experts, then the sum of squares), and the XCD's copies of the device-wide merged heads and h'.
struct PxXcd {
  uint2 item[64];
  uint2 att[2048];  // the merged heads of every XCD, relayed from the device-wide area
  uint2 hp[2048];   // h', relayed from the device-wide area
};

// Device-wide exchange area: the merged attention heads and the post-attention residual h'.
struct PxDev {
  uint2 att[2048];
  uint2 hp[2048];
};

struct PxBufs {
  PxXcd* xcd;  // [8]
  PxDev* dev;
  float* hp;   // [hidden] h' as plain values, for the next layer's launch (its expert outputs go to AbBufs::ys)
};

// Whether a layer of a model of these dimensions (shaped like L) runs as one launch: Q8_0 (hidden 1024 or 1536) or
// Q4_0 (hidden 1536) projections, 8 KV heads of 64 with 2 (1024) or 3 (1536) query heads each, 2..4 (G = 2) or 2..3
// (G = 3) tiles per split and at most 32 splits, top-8 of at most 63 experts with ffn 512, 256 compute units.
bool layers_fit(const Dims& d, const LayerDev& L, int cus);
// One layer as one launch: layer 0 reads the embedding row from b.h; a later layer reads the previous launch's h'
// (p.hp), expert outputs (x.ys) and routing weights (b.route_w); its own routing goes to b.route_ids / b.route_w.
// With `next` (the following layer), the launch's last phase also reads the next launch's q/k/v and output rows and
// K/V tiles once, into the XCDs' L2s.
hipError_t launch_layer(hipStream_t s, const PxLayer& L, const LayerDev& Ld, int layer, const Dims& d,
                        const StepBufs& b, int cus, const AbBufs& x, const PxBufs& p, const PxLayer* next,
                        Tl tl = {});
// The last layer's experts combined into b.h for the head.
hipError_t launch_layer_combine(hipStream_t s, const Dims& d, const StepBufs& b, int last_layer, const AbBufs& x,
                                const PxBufs& p, Tl tl = {});

}  // namespace moert

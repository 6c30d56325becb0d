// Launchers of the decode-step kernels (kernels.hip). All take device pointers and enqueue on `s`.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dev_math.h"
#include "timeline.h"

namespace moert {

// Device sequence state, one int each: position of the token being decoded, first position whose token the
// greedy argmax may write (positions before it are forced prompt tokens), last argmax.
enum { ST_POS = 0, ST_FIXED = 1, ST_ARGMAX = 2, ST_WORDS = 4 };

struct LayerDev {
  const float* ln_attn;
  const float* ln_moe;
  DMat qkv;           // [heads*d + 2*kv*d, H]: q rows, then k rows, then v rows
  DMat o;             // [H, heads*d]
  DMat router;        // [E, H]
  const float* router_bias;  // [E] or null
  DMat gate_up;       // [E*2I, H]
  DMat down;          // [E*H, I]
  uint16_t* k_cache;  // [kv, max_len, d] fp16
  uint16_t* v_cache;
};

struct Dims {
  int hidden, inter, heads, kv_heads, head_dim, vocab, experts, top_k, max_len, tps;  // tps: attention tiles per split
  float eps, emb_mult, res_mult, attn_mult, logits_scaling;
};

// Scratch buffers of one decode step (device).
struct StepBufs {
  float* h;          // [H] residual stream
  float* hc;         // [H] residual stream with the previous layer's experts combined (attention block -> o-proj)
  float* q;          // [heads*d]
  float* att;        // [heads*d]
  float* part;       // [heads, splits, 2 + d] split-KV partials
  float* zpart;      // [65, 256] MoE-norm partials of the current layer (moe_norm.h)
  float* act;        // [k, I] SwiGLU activations
  int* route_ids;    // [layers, k]
  float* route_w;    // [layers, k]
  float* logits;     // [V]
  int2* best;        // [head blocks] per-block argmax
  int* seq;          // [max_len] token of each position
  int* argmax_hist;  // [max_len] argmax produced at each position
  int* state;        // [ST_WORDS]
  const float* rope; // [max_len, d]: cos of the d/2 frequencies, then sin
};

// Exchange area of the attention block kernel (attn_block.hip) for one KV head, used only by the workgroups that
// run on the XCD of that head. Every entry is an 8-byte word (value bits, epoch of the launch that wrote it), written
// and read whole, so a reader knows a value is the current launch's by its epoch alone: the head group's queries
// after RoPE, the new K and V rows (fp16 bits), and the partials (m, l, acc[64]) of every split and query head.
constexpr int kAbMaxSplits = 64;
struct AbGroup {
  uint2 q[4][64];
  uint2 kv[2][64];
  uint2 part[kAbMaxSplits][4][66];
};
// Exchange area of the MoE kernel spread over the XCDs (moe_block.hip) for one XCD: the act vector of the XCD's
// expert, each value with the epoch of the launch that stored it.
constexpr int kMxWgs = 32;  // workgroups per XCD
struct MxGroup {
  uint2 act[512];  // (value bits, epoch of the launch that wrote it), written and read as one 8-byte word
};
struct AbBufs {
  AbGroup* groups;     // [8]
  MxGroup* moe;        // [8]
  float* ys;           // [8][hidden]: down output of the expert of each routing rank (k_moe_xcd)
  unsigned* step_ctr;  // decode steps started (k_embed adds one); a launch's epoch is step_ctr * 64 + layer + 1
  float* rope_cur;     // [64]: the rope row (cos, then sin) of the step's position (k_embed copies it)
  // err[0]: bits 1, 2: a wait for values of a KV head's workgroups (queries and K/V row, partials) gave up; bit 3: a
  // wait for the act values of an XCD's expert gave up. A launch that finds a bit set at its start waits for nothing
  // (its waits give up at once and set no further bit), so a failure costs at most one launch of bounded waits.
  // err[1]: a test mask that only the host writes (moert_fault_inject): a wait whose bit is set there looks for an
  // epoch no launch writes (kNoEpoch), and every wait of a launch that sees a nonzero mask polls at most kInjectSpin
  // times, so the failure path runs with every kernel still ending normally.
  unsigned* err;
};
constexpr unsigned kNoEpoch = 0xffffffffu;  // stored by no launch: epochs stay below 2^32 - 64 (the host clears the
                                            // exchange areas and the step counter before that)
constexpr int kInjectSpin = 256;

// tl: the launch's timeline record (measurement build; null otherwise). step_ctr (may be null): incremented once.
// rope_cur (may be null): receives the 64-float rope row of the step's position (head_dim 64).
hipError_t launch_embed(hipStream_t s, const DMat& emb, const Dims& d, const StepBufs& b, unsigned* step_ctr,
                        float* rope_cur = nullptr, Tl tl = {});
hipError_t launch_qkv(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, Tl tl = {});
hipError_t launch_attn_split(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, Tl tl = {});
hipError_t launch_attn_combine(hipStream_t s, const Dims& d, const StepBufs& b, Tl tl = {});
// The attention block (q/k/v + RoPE + KV append, split-KV attention, merge) in one launch, or false / an error when
// its shape does not apply: 8 KV heads of dim 64 with 2 query heads each and q/k/v rows of 1024 (Q8_0) or 3 query
// heads each and rows of 1536 (Q8_0 or Q4_0), 2-4 tiles
// per split, at most min(32, cus / 8) splits (cus: compute units of the device), layer < 63.
bool attn_block_fits(const Dims& d, const DMat& qkv, int cus);
// combine: the previous layer's experts are in x.ys (k_moe_xcd); the block forms h + res * sum_j w_j ys[j] (weights
// of layer - 1) as its input and workgroup 0 writes it to b.hc, the output projection's input.
// pfc (a cached model, not with combine): the same launch also predicts the layer's experts from h and copies the
// predicted misses into the pool (one decide and 64 copy workgroups after the attention workgroups, cache_pf.h);
// attn_block_prefetch_fits says whether the layer allows it (router of at most 64 rows in the q/k/v rows' format,
// top_k <= 8, top_k <= slots <= 4096).
struct CacheDev;
bool attn_block_prefetch_fits(const Dims& d, const LayerDev& L, const CacheDev& c);
hipError_t launch_attn_block(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int cus, int layer,
                             const AbBufs& x, bool combine, Tl tl = {}, const CacheDev* pfc = nullptr);
// The MoE half with the 8 routed experts spread over the 8 XCDs (router + gate/up + down in one launch, the down
// outputs left in x.ys for the next reader of h), or false / an error when it does not apply: top-8 routing, ffn
// 512, hidden 1024 or 1536, Q8_0 or Q4_0 experts and router, 256 compute units.
bool moe_xcd_fits(const Dims& d, const LayerDev& L, int cus);
hipError_t launch_moe_xcd(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int cus, int layer,
                          const AbBufs& x, Tl tl = {});
// h += res * sum_j w_j ys[j] for the last layer (before the head).
hipError_t launch_moe_combine(hipStream_t s, const Dims& d, const StepBufs& b, int layer, const AbBufs& x,
                              Tl tl = {});
// Both attention kernels for ny consecutive positions of a multi-position step: position y has its query at
// q + y * heads * 64, attends to *lenp + len_add + y cached positions and writes att + y * heads * 64 (part holds
// ny * heads * splits * 66 floats).
hipError_t launch_attn_batched(hipStream_t s, const LayerDev& L, const Dims& d, const int* lenp, int len_add, int ny,
                               const float* q, float* part, float* att);
// Output projection + residual; the epilogue writes the MoE-norm partials of the new h into b.zpart. from_hc: the
// residual input is b.hc (the attention block's combined h) instead of b.h; the result goes to b.h either way.
hipError_t launch_oproj(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, Tl tl = {},
                        bool from_hc = false);
// Router + gate/up of the routed experts (every workgroup ranks the experts, workgroup 0 publishes the routing).
// partials: the rmsnorm of h and the router logits from the MoE-norm partials that launch_oproj wrote (decode
// step); otherwise h is the normalised block input and the router's dots are computed in full.
hipError_t launch_route_up(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                           bool partials, Tl tl = {});
// accumulate: h += res * y (decode step); otherwise y is written to b.logits (standalone MoE block output).
hipError_t launch_expert_down(hipStream_t s, const LayerDev& L, const Dims& d, const StepBufs& b, int layer,
                              bool accumulate, Tl tl = {});
hipError_t launch_head(hipStream_t s, const DMat& head, const float* norm, const Dims& d, const StepBufs& b,
                       Tl tl = {});
hipError_t launch_head_argmax(hipStream_t s, const DMat& head, const Dims& d, const StepBufs& b, Tl tl = {});
int head_blocks(const DMat& head);

// The next kernel launched on this thread records its dispatch start/end into these events (hipExtLaunchKernelGGL).
void arm_launch_events(hipEvent_t start, hipEvent_t stop);

// Unit kernels.
hipError_t launch_gemv(hipStream_t s, const DMat& w, const float* x, float* y);
hipError_t launch_dequant(hipStream_t s, const DMat& w, float* out);
hipError_t launch_rmsnorm(hipStream_t s, const float* x, const float* w, int n, float eps, float* out);
hipError_t launch_rope(hipStream_t s, float* x, int heads, int head_dim, const float* cs);
hipError_t launch_topk(hipStream_t s, const float* logits, const float* bias, int n, int k, int* ids, float* w);
hipError_t launch_argmax(hipStream_t s, const float* v, int n, int2* best, int* cnt, int* out);
hipError_t launch_exp(hipStream_t s, const float* x, float* y, int n);
hipError_t launch_copy(hipStream_t s, const void* src, void* dst, size_t bytes);
// Streaming read of `bytes` (multiple of 16) into read_probe_blocks(bytes) * 256 words of out.
hipError_t launch_read(hipStream_t s, const void* src, size_t bytes, unsigned* out);
int read_probe_blocks(size_t bytes);
hipError_t launch_attn_unit(hipStream_t s, const float* q, const uint16_t* kc, const uint16_t* vc, int heads,
                            int kv_heads, int max_len, const int* len_dev, float scale, int tps, float* part,
                            float* out);
// Splits of a cache of max_len positions with tps 64-position tiles per split.
int attn_splits_for(int max_len, int tps);

}  // namespace moert

// Multi-position MoE step (grouped int8 MFMA expert GEMM): device buffers and launcher (grouped.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace moert {

constexpr int kGrpMaxPos = 32;  // positions per grouped step (the reference caps a step at 32, cuda_backend.rs:272-274)

// Offsets (in ints) of the step plan published by the gate/up kernel: number of distinct experts, then per list
// index u (first-appearance order) the expert, its member count, its first member slot and its member positions as
// a bit mask; then per position p its k member slots and routing weights (as float bits) in list order.
enum { GRP_NU = 0, GRP_LIST = 1, GRP_CNT = 65, GRP_OFF = 129, GRP_BITS = 193, GRP_ORD_SLOT = 257,
       GRP_ORD_W = GRP_ORD_SLOT + kGrpMaxPos * 8, GRP_WORDS = GRP_ORD_W + kGrpMaxPos * 8 };

// A Q8_0 matrix (rows % 16 == 0, cols % 64 == 0) in the tiled layout of the grouped MFMA kernels. Payload: per
// 16-row tile t and 64-column span p, one 1 KB piece in which lane l holds 16 bytes: elements 8*(l/16) .. +8 of
// row 16t + l%16 in block 2p, then the same elements of block 2p + 1 (the A operands of two MFMA K-steps, so a
// wave's load is 1 KB of consecutive bytes). Scales: per tile t and block b the 16 rows' fp16 scales [t][b][16].
struct TMat {
  const uint8_t* q;
  const uint16_t* d;
  int rows, cols;
};

// Device buffers of one grouped step, sized for kGrpMaxPos positions, hidden H, inter I and top-k <= 8.
struct GroupBufs {
  int* ids;      // [m, k] routed experts, top-k order
  float* w;      // [m, k] routing weights
  int8_t* xh;    // [m, H] hi codes of the block inputs
  int8_t* xl;    // [m, H] lo codes
  float* xd;     // [m, H/32] their block scales
  int* grp;      // [GRP_WORDS] the step plan (see GRP_*)
  int8_t* ah;    // [m*k, I] hi codes of the SwiGLU activations, by member slot
  int8_t* al;    // [m*k, I]
  float* ad;     // [m*k, I/32]
  float* o;      // [m*k, H] down outputs by member slot
  TMat gu, dn;   // gate_up [E*2I, H] and down [E*H, I] of the block in the tiled layout
  TMat qkv, oproj;  // the layer's q/k/v [(heads + 2 kv_heads) * 64, H] and output [H, heads * 64] projections, tiled
};

// Exchange buffers of the one-launch block (launch_grp_fused), zeroed at allocation. Entries are (value bits,
// epoch) 8-byte words; the input codes are plain bytes published by a per-position epoch flag.
constexpr int kFbPos = 16;         // positions per one-launch block step
constexpr int kFbExperts = 48;     // routed experts at most
constexpr int kFbInter = 512;      // ffn width of the one-launch block
constexpr int kFbActW = 17;        // act entries per (expert, 32-row block, position): 8 hi words, 8 lo words, scale
struct FbBufs {
  unsigned* err;  // [2] bits of the waits that gave up (1 router logits, 2 act vectors, 4 expert outputs, 8 codes),
                  // then the test mask of waits made to give up (moert_block_fault_inject)
  uint2* lg;      // [8][kFbPos * 64] router logits (position, expert) of each XCD
  uint2* xflag;   // [8][kFbPos] one flag per (XCD, position) over the XCD's copy of the input codes
  int8_t* xh;     // [8][kFbPos][hidden] hi codes of the inputs, one copy per XCD
  int8_t* xl;     // [8][kFbPos][hidden] lo codes
  float* xd;      // [8][kFbPos][hidden / 32] their block scales
  uint2* act;     // [kFbExperts][kFbInter / 32][kFbActW][kFbPos] act codes by list index, device-wide
  uint2* o;       // [kFbPos * 8][hidden] expert outputs by member slot, device-wide
  uint2* rk;      // [8][kFbPos][16] per XCD: the top-k ids (8), then weights (8), of each position
};

// y[m, H] = the MoE block of launch_grouped_block as one launch of 256 workgroups of 512 threads, all resident (one
// per compute unit, 8 XCDs): each XCD codes and ranks the m positions once and shares the codes, router logits and
// top-k through its L2; the gate/up items and down tiles of all routed experts are dealt over the 256 workgroups,
// with the m positions as MFMA columns and the act vectors device-wide; the expert outputs go out device-wide and
// workgroup b combines rows [b H / 256, +H / 256). Same arithmetic and order as the four
// kernels, bit for bit. m <= 16, k <= 8, E <= 48, ffn 512, Q8_0, 256 compute units; `epoch` >= 1 differs from the
// previous launch's on these buffers.
hipError_t launch_grp_fused(hipStream_t s, const LayerDev& L, int m, int k, int inter, const float* x,
                            const GroupBufs& g, const FbBufs& f, unsigned epoch, float* y, int cus);

// Tiled copy (TMat layout) of the Q8_0 matrix src into q [rows*cols] and d [rows*cols/32].
hipError_t launch_tile_q8(hipStream_t s, const DMat& src, uint8_t* q, uint16_t* d);

// y[m, H] = MoE block of the m rows of x (already normalised), router + top-k per row, experts grouped.
// Q8_0 router, gate_up and down; E <= 64, k <= 8, m <= kGrpMaxPos. With `ev` (8 events), the four kernels
// (route, up, down, combine) record their dispatch start/end into ev[2i], ev[2i+1].
hipError_t launch_grouped_block(hipStream_t s, const LayerDev& L, int m, int k, int inter, const float* x,
                                GroupBufs g, float* y, const hipEvent_t* ev = nullptr);
// Pieces of a layer of the multi-position step in grouped mode (every projection an int8 MFMA GEMM), on m <= 32
// positions; the activation codes live in g.xh / g.xl / g.xd between kernels.
//   launch_norm_codes     codes of rmsnorm(h[p], lnw) (H 1024 or 1536)
//   launch_gd_qkv         q/k/v of the coded rows through g.qkv, RoPE at positions pos0 + p, q [m, heads*64] in f32,
//                         K and V into the fp16 cache rows pos0 + p
//   launch_grp_codes      codes of x[m, K] (the attention outputs)
//   launch_gd_oproj       h += res * (g.oproj times the coded rows)
//   launch_grp_route_norm router of rmsnorm(h[p], lnw) (+ bias), top-k into g.ids / g.w, codes of the normalised row
//   launch_grp_experts    gate/up and down of the routed experts (tiled g.gu / g.dn) into g.o by member slot; with
//                         `ev` (8 events), record the dispatches of the two kernels into ev[2], ev[3] and ev[4], ev[5]
//   launch_gd_combine     h[p] += res * (sum over p's experts in list order of w * o), then with lnw the codes of
//                         rmsnorm(h[p], lnw)
hipError_t launch_norm_codes(hipStream_t s, int H, int m, const float* h, const float* lnw, float eps,
                             const GroupBufs& g);
hipError_t launch_gd_qkv(hipStream_t s, const Dims& d, int m, int pos0, const float* rope, float* q, uint16_t* kc,
                         uint16_t* vc, const GroupBufs& g);
hipError_t launch_grp_codes(hipStream_t s, int K, int m, const float* x, const GroupBufs& g);
hipError_t launch_gd_oproj(hipStream_t s, int m, float res, float* h, const GroupBufs& g);
hipError_t launch_grp_route_norm(hipStream_t s, const LayerDev& L, int m, int k, const float* h, const float* lnw,
                                 float eps, const GroupBufs& g);
hipError_t launch_grp_experts(hipStream_t s, int H, int E, int m, int k, int inter, const GroupBufs& g,
                              const hipEvent_t* ev = nullptr);
hipError_t launch_gd_combine(hipStream_t s, int H, int m, int k, float res, float* h, const float* lnw, float eps,
                             const GroupBufs& g);

}  // namespace moert

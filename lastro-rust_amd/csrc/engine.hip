// Host side of the decode engine: C++ classes that mirror the reference's GpuModel / GpuLayer
// (rust/moe-rt/src/gpu_model.rs, gpu.rs) and the extern "C" ABI declared in include/moert.h.
//
// Memory: every weight is resident in HBM as struct-of-arrays (payload plane + fp16 scale plane); q/k/v of a
// layer are stacked into one [q; k; v] matrix; experts of a layer are one [E*2I, H] gate_up and one [E*H, I] down
// matrix. The KV cache is fp16 [kv_heads, max_len, head_dim] per layer. One decode step is a fixed sequence of
// kernels captured once into a hipGraph: the token and the position live in device memory (seq, state), so the
// same graph serves every position and greedy generation needs no host synchronisation between tokens.
#include <hip/hip_runtime.h>

#include <atomic>
#include <chrono>
#include <cmath>
#include <memory>
#include <cstdlib>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/moert.h"
#include "host_utils.h"
#include "host_experts.h"
#include "placement.h"
#include "cache.h"
#include "grouped.h"
#include "kernels.h"
#include "layers.h"
#include "moe_norm.h"
#include "noalloc.h"
#include "prefill.h"

using namespace moert;

namespace {

thread_local std::string g_err;

void set_err(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
}

#define CHECK_HIP(expr)                                                           \
  do {                                                                            \
    hipError_t e_ = (expr);                                                       \
    if (e_ != hipSuccess) {                                                       \
      set_err("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__); \
      return MOERT_E_DEVICE;                                                      \
    }                                                                             \
  } while (0)

#define CHECK_CFG(cond, ...)   \
  do {                         \
    if (!(cond)) {             \
      set_err(__VA_ARGS__);    \
      return MOERT_E_CONFIG;   \
    }                          \
  } while (0)

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

}  // namespace

namespace moert {
// The thread-local error message, for the other host files of the library; returns `code`.
int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}
}  // namespace moert

namespace {

// Device allocations owned by one handle, freed only after its stream is idle
// (Release after both streams synced, rust/moe-rt/src/motor/mem.rs:1-13).
struct Arena {
  std::vector<void*> ptrs;
  int alloc(void** p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    CHECK_HIP(hipMalloc(p, bytes));
    ptrs.push_back(*p);
    return MOERT_OK;
  }
  void release() {
    for (void* p : ptrs) (void)hipFree(p);
    ptrs.clear();
  }
};

bool valid_dtype(int dt) { return dt == MOERT_F32 || dt == MOERT_Q8_0 || dt == MOERT_Q4_0; }

size_t payload_bytes(int dtype, int cols) {
  return dtype == MOERT_Q8_0 ? (size_t)cols : dtype == MOERT_Q4_0 ? (size_t)cols / 2 : (size_t)cols * 4;
}

// Rows [row0, row0 + n) of a GGML blob ([*, cols] of dtype) into a payload plane (n * payload_bytes) and a scale
// plane (n * cols/32 fp16; untouched for f32).
void repack_rows(const void* src_, int dtype, int cols, size_t row0, size_t n, uint8_t* q, uint16_t* d) {
  const uint8_t* src = (const uint8_t*)src_;
  const size_t nb = n * (cols / 32);
  if (dtype == MOERT_F32) {
    std::memcpy(q, src + row0 * cols * 4, n * cols * 4);
  } else if (dtype == MOERT_Q8_0) {
    src += row0 * (cols / 32) * 34;
    for (size_t b = 0; b < nb; b++) {
      const uint8_t* blk = src + b * 34;
      d[b] = (uint16_t)(blk[0] | (blk[1] << 8));
      std::memcpy(q + b * 32, blk + 2, 32);
    }
  } else {
    src += row0 * (cols / 32) * 18;
    for (size_t b = 0; b < nb; b++) {
      const uint8_t* blk = src + b * 18;
      d[b] = (uint16_t)(blk[0] | (blk[1] << 8));
      std::memcpy(q + b * 16, blk + 2, 16);
    }
  }
}

// Repacks `parts` (each [rows_i, cols] of one dtype, GGML blocks) into one SoA device matrix.
struct Part {
  const void* data;
  int rows;
};
int upload_matrix(Arena& a, hipStream_t s, const std::vector<Part>& parts, int dtype, int cols, DMat* out) {
  CHECK_CFG(valid_dtype(dtype), "unknown dtype %d", dtype);
  CHECK_CFG(cols % 32 == 0, "row length %d is not a multiple of 32", cols);
  size_t rows = 0;
  for (const Part& p : parts) {
    CHECK_CFG(p.data != nullptr, "missing weight tensor");
    rows += (size_t)p.rows;
  }
  size_t plane = rows * payload_bytes(dtype, cols);
  size_t scales = dtype == MOERT_F32 ? 0 : rows * (cols / 32) * 2;
  void* dev;
  int rc = a.alloc(&dev, align256(plane) + scales);
  if (rc) return rc;
  std::vector<uint8_t> q(plane);
  std::vector<uint16_t> d(scales / 2);
  size_t r0 = 0;
  for (const Part& p : parts) {
    repack_rows(p.data, dtype, cols, 0, (size_t)p.rows, q.data() + r0 * payload_bytes(dtype, cols),
                d.empty() ? nullptr : d.data() + r0 * (cols / 32));
    r0 += (size_t)p.rows;
  }
  CHECK_HIP(hipMemcpyAsync(dev, q.data(), plane, hipMemcpyHostToDevice, s));
  if (scales) CHECK_HIP(hipMemcpyAsync((uint8_t*)dev + align256(plane), d.data(), scales, hipMemcpyHostToDevice, s));
  CHECK_HIP(hipStreamSynchronize(s));
  out->q = (const uint8_t*)dev;
  out->d = scales ? (const uint16_t*)((uint8_t*)dev + align256(plane)) : nullptr;
  out->dtype = dtype;
  out->rows = (int)rows;
  out->cols = cols;
  return MOERT_OK;
}

int upload_f32(Arena& a, hipStream_t s, const float* src, size_t n, float** out) {
  void* p;
  int rc = a.alloc(&p, n * 4);
  if (rc) return rc;
  if (src) CHECK_HIP(hipMemcpyAsync(p, src, n * 4, hipMemcpyHostToDevice, s));
  else CHECK_HIP(hipMemsetAsync(p, 0, n * 4, s));
  *out = (float*)p;
  return MOERT_OK;
}

template <class T>
int zeros(Arena& a, hipStream_t s, size_t n, T** out) {
  void* p;
  int rc = a.alloc(&p, n * sizeof(T));
  if (rc) return rc;
  CHECK_HIP(hipMemsetAsync(p, 0, n * sizeof(T), s));
  *out = (T*)p;
  return MOERT_OK;
}

bool k_supported(int k) { return k == 128 || k == 256 || k == 512 || k == 1024 || k == 1536; }

}  // namespace

// ------------------------------------------------------------------------------------------------------------
// GpuModel (rust/moe-rt/src/gpu_model.rs:180-445).
struct moert_model {
  moert_config cfg{};
  Dims dims{};
  int max_len = 0, splits = 0, host_pos = 0;
  bool poisoned = false;
  hipStream_t stream = nullptr;
  Arena arena;
  std::vector<LayerDev> layers;
  DMat embed{};
  float* norm = nullptr;
  StepBufs b{};
  int n_head_blocks = 0;
  // attention block in one launch (attn_block.hip) when the shape allows it; otherwise q/k/v, split attention and
  // combine as three kernels. MOERT_ATTN_BLOCK=0 at create keeps the three kernels.
  bool use_ab = false;
  // the MoE half spread over the XCDs (moe_block.hip; resident experts with the attention block): k_moe_xcd leaves
  // the experts' down outputs for the next attention block (or k_moe_combine) to combine. MOERT_MOE_XCD=0 at create
  // keeps k_route_up + k_expert_down.
  bool use_mx = false;
  // every layer as one launch (layers.hip), where the shape allows it with the attention block and the MoE kernel
  // over the XCDs; MOERT_LAYER=0 at create keeps three launches per layer
  bool use_px = false;
  PxBufs px{};
  std::vector<PxLayer> pxl;
  int cus = 0;
  AbBufs ab{};
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  // expert cache (ExpertCache, rust/moe-rt/src/cache.rs): experts live in the pinned host store, `cache.slots` of
  // them at a time in the HBM pool
  bool cached = false;
  CacheDev cache{};
  void* host_store = nullptr;
  // prefetch branch of the cached step (moert_cache_prefetch_mode): side stream and its fork / join events
  bool prefetch = false;
  bool pf_blk = false;  // the prefetch inside the attention launch instead of the side branch (cache_pf.h)
  hipStream_t pf_stream = nullptr;
  hipEvent_t ev_fork = nullptr, ev_pred = nullptr, ev_copy = nullptr;
  // runtime metrics (moert_model_attach_metrics): the publisher, the pinned read-back of the device counters and
  // the step state, and the generate call's timing marks
  using Clock = std::chrono::steady_clock;
  moert_metrics* mx = nullptr;
  int mx_interval_ms = 500;
  unsigned char* mx_pin = nullptr;
  hipEvent_t mx_ev = nullptr, mx_t[3] = {};
  bool mx_pending = false;
  Clock::time_point mx_last_read, mx_last_pub, mx_prev_t;
  unsigned long long mx_prev[CS_WORDS] = {};
  int mx_prev_pos = 0;
  double mx_wait_s = 0;
  double mx_speed_last[2] = {};  // decode and prefill tok/s of the last finished request
  // host-CPU hybrid (moert_model_create_hybrid): the placement state machine, the token's table on the device, the
  // pinned read-backs of each layer's routing and normalised input (two layers' worth: the next layer's are queued
  // while this one is served), the host experts' sum (coherent mapped memory, read by the doorbell kernel), and per
  // position and layer: hits, copies, dropped, host-computed requests
  bool hybrid = false;
  std::unique_ptr<Placement> place;
  int hy_threads = 1;
  int* hy_table = nullptr;  // device
  int* hy_table_pin = nullptr;
  int* hy_ids_pin = nullptr;
  float* hy_w_pin = nullptr;
  float* hy_xn_pin = nullptr;
  float* hy_y_pin = nullptr;
  float* hy_y_dev = nullptr;
  float* hy_xn_dev = nullptr;
  // the doorbell: per layer a flag word in coherent host memory (token sequence << 1 | any host expert) that the
  // layer's add kernel waits for, the routing event of every layer, the token's sequence number, and the device word
  // a doorbell that never rang sets
  unsigned* hy_flag_pin = nullptr;
  unsigned* hy_flag_dev = nullptr;
  unsigned* hy_err = nullptr;
  std::vector<hipEvent_t> hy_evs;
  unsigned hy_seq = 0;
  std::vector<float> hy_act, hy_y;
  std::vector<int> hy_tok;  // [max_len][layers][4]

  // Launches one decode step. With `timed` >= 0, every launch of that kernel class records its dispatch start and
  // end into the next event pair of `ev`. With a timeline buffer (measurement build), launch i of the step records
  // its workgroups' phase stamps into record i, and tl_kind / tl_layer say which launch that was.
  int enqueue(int timed, std::vector<hipEvent_t>* ev) {
    ev_i = 0;
    tl_kind.clear();
    tl_layer.clear();
    auto arm = [&](int kind, int layer) -> Tl {
      if (kind == timed) {
        arm_launch_events((*ev)[ev_i], (*ev)[ev_i + 1]);
        ev_i += 2;
      }
      Tl t{tl_buf ? tl_buf + tl_kind.size() * kTlRecord : nullptr};
      tl_kind.push_back(kind);
      tl_layer.push_back(layer);
      return t;
    };
    // the prefetch runs inside the attention launch where the block fits (pf_blk); otherwise the side branch's
    // kernels run beside the attention half on a second stream, and then the attention block (whose workgroups must
    // all be resident at once, dispatched round-robin over the XCDs) is not used
    const bool branch = cached && prefetch && !pf_blk;
    const bool use_blk = use_ab && !branch;
    CHECK_HIP(
        launch_embed(stream, embed, dims, b, ab.step_ctr, use_blk ? ab.rope_cur : nullptr, arm(MOERT_K_EMBED, -1)));
    if (use_px) {
      for (size_t l = 0; l < layers.size(); l++)
        CHECK_HIP(launch_layer(stream, pxl[l], layers[l], (int)l, dims, b, cus, ab, px,
                               l + 1 < layers.size() ? &pxl[l + 1] : nullptr, arm(MOERT_K_LAYER, (int)l)));
      CHECK_HIP(launch_layer_combine(stream, dims, b, (int)layers.size() - 1, ab, px, arm(MOERT_K_LAYER_COMBINE, -1)));
      CHECK_HIP(launch_head(stream, embed, norm, dims, b, arm(MOERT_K_HEAD, -1)));
      CHECK_HIP(launch_head_argmax(stream, embed, dims, b, arm(MOERT_K_HEAD_ARGMAX, -1)));
      return MOERT_OK;
    }
    for (size_t l = 0; l < layers.size(); l++) {
      const LayerDev& L = layers[l];
      const int li = (int)l;
      const bool pf = branch;
      if (pf) {
        // side branch: predict the layer's experts from its input and copy the predicted misses into the pool while
        // the attention half runs; the output projection (which rewrites h) waits for the prediction, the router +
        // gate/up kernel for the copies
        CHECK_HIP(hipEventRecord(ev_fork, stream));
        CHECK_HIP(hipStreamWaitEvent(pf_stream, ev_fork, 0));
        CHECK_HIP(launch_prefetch_decide(pf_stream, L, dims, b, li, cache));
        CHECK_HIP(hipEventRecord(ev_pred, pf_stream));
        CHECK_HIP(launch_prefetch_copy(pf_stream, cache));
        CHECK_HIP(hipEventRecord(ev_copy, pf_stream));
      }
      const bool cmb = use_mx && li > 0;  // the previous layer's experts are combined by this attention block
      if (use_blk) {
        CHECK_HIP(launch_attn_block(stream, L, dims, b, cus, li, ab, cmb, arm(MOERT_K_ATTN_BLOCK, li),
                                    cached && prefetch ? &cache : nullptr));
      } else {
        CHECK_HIP(launch_qkv(stream, L, dims, b, arm(MOERT_K_QKV, li)));
        CHECK_HIP(launch_attn_split(stream, L, dims, b, arm(MOERT_K_ATTN_SPLIT, li)));
        CHECK_HIP(launch_attn_combine(stream, dims, b, arm(MOERT_K_ATTN_COMBINE, li)));
      }
      if (pf) CHECK_HIP(hipStreamWaitEvent(stream, ev_pred, 0));
      CHECK_HIP(launch_oproj(stream, L, dims, b, arm(MOERT_K_OPROJ, li), cmb));
      if (pf) CHECK_HIP(hipStreamWaitEvent(stream, ev_copy, 0));
      if (use_mx) {
        CHECK_HIP(launch_moe_xcd(stream, L, dims, b, cus, li, ab, arm(MOERT_K_MOE_XCD, li)));
      } else if (cached) {
        CHECK_HIP(launch_route_up_cached(stream, L, dims, b, li, cache, arm(MOERT_K_ROUTE_UP, li)));
        CHECK_HIP(launch_expert_down_cached(stream, dims, b, li, cache, arm(MOERT_K_EXPERT_DOWN, li)));
      } else {
        CHECK_HIP(launch_route_up(stream, L, dims, b, li, true, arm(MOERT_K_ROUTE_UP, li)));
        CHECK_HIP(launch_expert_down(stream, L, dims, b, li, true, arm(MOERT_K_EXPERT_DOWN, li)));
      }
    }
    if (use_mx)
      CHECK_HIP(launch_moe_combine(stream, dims, b, (int)layers.size() - 1, ab, arm(MOERT_K_MOE_COMBINE, -1)));
    CHECK_HIP(launch_head(stream, embed, norm, dims, b, arm(MOERT_K_HEAD, -1)));
    CHECK_HIP(launch_head_argmax(stream, embed, dims, b, arm(MOERT_K_HEAD_ARGMAX, -1)));
    return MOERT_OK;
  }
  int ev_i = 0;
  unsigned long long steps_since_clear = 0;  // steps launched since the exchange areas were last cleared
  // timeline records (measurement build): kTlRecord words per launch of a step
  static constexpr size_t kTlRecord = (size_t)kTlMaxBlocks * kTlPhases;
  unsigned long long* tl_buf = nullptr;
  size_t tl_launches = 0;
  std::vector<int> tl_kind, tl_layer;

  // A hybrid record copy (host store -> pool slot), queued on the model stream behind the work queued so far.
  int hy_copy(int slot, int key) {
    const uint8_t* r = (const uint8_t*)host_store + (size_t)key * cache.record_bytes;
    const size_t v = (size_t)slot, dn_d = cache.record_bytes - cache.gu_q - cache.gu_d - cache.dn_q;
    CHECK_HIP(hipMemcpyAsync((void*)(cache.pool_gu.q + v * cache.gu_q), r, cache.gu_q, hipMemcpyHostToDevice, stream));
    if (cache.gu_d)
      CHECK_HIP(hipMemcpyAsync((uint8_t*)cache.pool_gu.d + v * cache.gu_d, r + cache.gu_q, cache.gu_d,
                               hipMemcpyHostToDevice, stream));
    r += cache.gu_q + cache.gu_d;
    CHECK_HIP(hipMemcpyAsync((void*)(cache.pool_dn.q + v * cache.dn_q), r, cache.dn_q, hipMemcpyHostToDevice, stream));
    if (dn_d)
      CHECK_HIP(hipMemcpyAsync((uint8_t*)cache.pool_dn.d + v * dn_d, r + cache.dn_q, dn_d, hipMemcpyHostToDevice,
                               stream));
    return MOERT_OK;
  }

  int hy_copies() {
    for (const CopyOrder& o : place->take_copies()) {
      int rc = hy_copy(o.slot, o.key);
      if (rc) return rc;
    }
    return MOERT_OK;
  }

  // One hybrid decode step (the D1 protocol in its deterministic mode; cuda_backend.rs:919-1014 with the doorbell of
  // motor/backend.rs:17-25): the token's table to the device, then the GPU work of every layer queued one layer ahead
  // of the host: the attention half and the gate/up kernel (experts in the table from their slots), the routing and
  // the normalised input read back behind the layer's event, the down kernel, and the doorbell kernel that waits for
  // the layer's flag and adds the host experts' sum. This thread serves each layer as its event completes: the
  // layer's requests (placement), the experts outside the table computed into the mapped sum, the flag rung, the
  // admissions' copies queued (behind the next layer's queued work; held ones once their victim's layer has passed).
  // The GPU never waits for an enqueue, only for the host experts. At the end of the token every copy queued precedes
  // the next token's work in stream order (the barrier), and the next table is published.
  int hybrid_step() {
    Placement& P = *place;
    const int L = cfg.layers, E = cfg.experts, K = cfg.top_k, H = cfg.hidden;
    // the previous token has ended (so its table copy has been read, and its position is final)
    CHECK_HIP(hipStreamSynchronize(stream));
    unsigned herr = 0;
    CHECK_HIP(hipMemcpy(&herr, hy_err, 4, hipMemcpyDeviceToHost));
    if (herr) {
      set_err("hybrid step: a layer's doorbell was not rung in time (error bits %#x)", herr);
      return MOERT_E_DEVICE;
    }
    int pos = 0;
    CHECK_HIP(hipMemcpy(&pos, b.state + ST_POS, 4, hipMemcpyDeviceToHost));
    std::memcpy(hy_table_pin, P.table().data(), (size_t)L * E * 4);
    CHECK_HIP(hipMemcpyAsync(hy_table, hy_table_pin, (size_t)L * E * 4, hipMemcpyHostToDevice, stream));
    CHECK_HIP(launch_embed(stream, embed, dims, b, ab.step_ctr, use_ab ? ab.rope_cur : nullptr));
    // the token's sequence number in 31 bits, never 0 (the flags start at 0)
    hy_seq = (hy_seq + 1u) & 0x7fffffffu;
    if (hy_seq == 0u) hy_seq = 1u;
    const unsigned seq = hy_seq;
    auto enqueue_layer = [&](int l) -> int {
      const LayerDev& Ld = layers[l];
      if (use_ab) {
        CHECK_HIP(launch_attn_block(stream, Ld, dims, b, cus, l, ab, false));
      } else {
        CHECK_HIP(launch_qkv(stream, Ld, dims, b));
        CHECK_HIP(launch_attn_split(stream, Ld, dims, b));
        CHECK_HIP(launch_attn_combine(stream, dims, b));
      }
      CHECK_HIP(launch_oproj(stream, Ld, dims, b));
      CHECK_HIP(launch_route_up_cached(stream, Ld, dims, b, l, cache));
      CHECK_HIP(hipMemcpyAsync(hy_ids_pin + 8 * (l & 1), b.route_ids + l * K, (size_t)K * 4, hipMemcpyDeviceToHost,
                               stream));
      CHECK_HIP(hipMemcpyAsync(hy_w_pin + 8 * (l & 1), b.route_w + l * K, (size_t)K * 4, hipMemcpyDeviceToHost,
                               stream));
      CHECK_HIP(hipMemcpyAsync(hy_xn_pin + (size_t)H * (l & 1), hy_xn_dev, (size_t)H * 4, hipMemcpyDeviceToHost,
                               stream));
      CHECK_HIP(hipEventRecord(hy_evs[l], stream));
      CHECK_HIP(launch_expert_down_cached(stream, dims, b, l, cache));
      CHECK_HIP(launch_hy_doorbell_add(stream, b.h, hy_y_dev, dims.res_mult, H, hy_flag_dev + l, seq, hy_err));
      return MOERT_OK;
    };
    // on a host-side failure the layers already queued must not wait out their doorbells: ring them all, empty
    auto release = [&]() {
      std::atomic_thread_fence(std::memory_order_release);
      for (int l = 0; l < L; l++) reinterpret_cast<volatile unsigned*>(hy_flag_pin)[l] = seq << 1;
    };
    int rc = enqueue_layer(0);
    if (!rc && L > 1) rc = enqueue_layer(1);
    if (rc) {
      release();
      return rc;
    }
    std::vector<int> keys, n_e;
    std::vector<char> gpu;
    for (int l = 0; l < L; l++) {
      if (hipEventSynchronize(hy_evs[l]) != hipSuccess) {
        release();
        set_err("hybrid step: layer %d routing event", l);
        return MOERT_E_DEVICE;
      }
      const int* ids = hy_ids_pin + 8 * (l & 1);
      const float* wts_l = hy_w_pin + 8 * (l & 1);
      for (int j = 0; j < K; j++)
        if (ids[j] < 0 || ids[j] >= E) {
          release();
          set_err("hybrid step: routed expert %d outside [0, %d)", ids[j], E);
          return MOERT_E_DEVICE;
        }
      const PlacementStats s0 = P.stats();
      P.serve_layer(l, ids, 1, &keys, &n_e, &gpu);
      // the host experts in top-k order (CPU-served requests, HostExperts::compute)
      const uint8_t* recs[8];
      float wts[8];
      int n_host = 0;
      for (int j = 0; j < K; j++) {
        const int key = l * E + ids[j];
        if (P.table()[key] >= 0) continue;
        recs[n_host] = (const uint8_t*)host_store + (size_t)key * cache.record_bytes;
        wts[n_host++] = wts_l[j];
      }
      const bool any = n_host > 0;
      if (any) {
        std::fill(hy_y.begin(), hy_y.end(), 0.0f);
        const HostRecordGeo geo{cache.pool_gu.dtype, H, cfg.inter, cache.gu_q, cache.gu_d, cache.dn_q};
        host_experts_layer(geo, recs, wts, n_host, hy_xn_pin + (size_t)H * (l & 1), hy_act.data(), hy_y.data(),
                           hy_threads);
        // (the previous layer's doorbell kernel has read the sum: it precedes this layer's routing event)
        std::memcpy(hy_y_pin, hy_y.data(), (size_t)H * 4);
      }
      // ring the layer's doorbell: the sum is in host memory before the flag (release fence, then the store)
      std::atomic_thread_fence(std::memory_order_release);
      reinterpret_cast<volatile unsigned*>(hy_flag_pin)[l] = (seq << 1) | (any ? 1u : 0u);
      P.admit_layer();
      const PlacementStats& s1 = P.stats();
      if (pos >= 0 && pos < max_len) {
        int* t = hy_tok.data() + ((size_t)pos * L + l) * 4;
        t[0] = (int)(s1.hits - s0.hits);
        t[1] = (int)(s1.copies - s0.copies);
        t[2] = (int)(s1.dropped - s0.dropped);
        t[3] = (int)(s1.cpu - s0.cpu);
      }
      // the admissions' copies land behind layer l + 1's queued reads (a slot a later layer of this token reads is
      // held by the placement until that layer has passed)
      rc = hy_copies();
      if (!rc && l + 2 < L) rc = enqueue_layer(l + 2);
      if (rc) {
        release();
        return rc;
      }
    }
    P.end_token();
    rc = hy_copies();
    if (rc) return rc;
    CHECK_HIP(launch_head(stream, embed, norm, dims, b));
    CHECK_HIP(launch_head_argmax(stream, embed, dims, b));
    return MOERT_OK;
  }

  int fail(int rc) {
    if (rc == MOERT_E_DEVICE) {
      poisoned = true;
      (void)hipStreamSynchronize(stream);
    }
    return rc;
  }

  int build_graph() {
    CHECK_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue(-1, nullptr);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(stream, &g);
    if (rc) return rc;
    CHECK_HIP(e);
    graph = g;
    CHECK_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    return MOERT_OK;
  }

  // multi-position step buffers, allocated on first use
  PfBufs pf{};
  int ensure_pf() {
    if (pf.h) return MOERT_OK;
    const int H = dims.hidden, qd = dims.heads * 64, I = dims.inter, M = kPfMaxPos, K8 = 8;
    const size_t parts = (size_t)M * dims.heads * attn_splits_for(max_len, dims.tps) * 66;
    int rc;
    if ((rc = zeros(arena, stream, (size_t)M, &pf.toks)) || (rc = zeros(arena, stream, (size_t)1, &pf.pos0)) ||
        (rc = zeros(arena, stream, (size_t)M * H, &pf.h)) || (rc = zeros(arena, stream, (size_t)M * qd, &pf.q)) ||
        (rc = zeros(arena, stream, (size_t)M * qd, &pf.att)) || (rc = zeros(arena, stream, parts, &pf.part)) ||
        (rc = zeros(arena, stream, (size_t)M * kNormItems, &pf.zpart)) ||
        (rc = zeros(arena, stream, (size_t)M * H, &pf.xn)) || (rc = zeros(arena, stream, (size_t)M * K8, &pf.ids)) ||
        (rc = zeros(arena, stream, (size_t)M * K8, &pf.w)) ||
        (rc = zeros(arena, stream, (size_t)M * K8 * I, &pf.act)) ||
        (rc = zeros(arena, stream, (size_t)M * K8 * H, &pf.o)))
      return rc;
    CHECK_HIP(hipStreamSynchronize(stream));
    return MOERT_OK;
  }

  // grouped mode of the multi-position step (moert_batched_mode): the grouped kernels' buffers and every layer's
  // experts in their tiled layout, built on first use
  int batched_mode = 0;
  GroupBufs mg{};
  struct TiledLayer {
    TMat gu, dn, qkv, o;
  };
  std::vector<TiledLayer> tiled;
  int ensure_grouped() {
    if (mg.xh) return MOERT_OK;
    const int H = dims.hidden, I = dims.inter, M = kGrpMaxPos, S = kGrpMaxPos * 8;
    const int X = std::max(H, dims.heads * dims.head_dim);  // code rows: block inputs and attention outputs
    int rc;
    if ((rc = zeros(arena, stream, (size_t)M * X, &mg.xh)) || (rc = zeros(arena, stream, (size_t)M * X, &mg.xl)) ||
        (rc = zeros(arena, stream, (size_t)M * (X / 32), &mg.xd)) ||
        (rc = zeros(arena, stream, (size_t)GRP_WORDS, &mg.grp)) || (rc = zeros(arena, stream, (size_t)S * I, &mg.ah)) ||
        (rc = zeros(arena, stream, (size_t)S * I, &mg.al)) || (rc = zeros(arena, stream, (size_t)S * (I / 32), &mg.ad)) ||
        (rc = zeros(arena, stream, (size_t)S * H, &mg.o)))
      return rc;
    auto tile = [&](const DMat& src, TMat* dst) -> int {
      uint8_t* q;
      uint16_t* d;
      const size_t n = (size_t)src.rows * src.cols;
      int r;
      if ((r = arena.alloc((void**)&q, n)) || (r = arena.alloc((void**)&d, n / 32 * 2))) return r;
      CHECK_HIP(launch_tile_q8(stream, src, q, d));
      *dst = TMat{q, d, src.rows, src.cols};
      return MOERT_OK;
    };
    for (const LayerDev& L : layers) {
      TiledLayer t{};
      if ((rc = tile(L.gate_up, &t.gu)) || (rc = tile(L.down, &t.dn)) || (rc = tile(L.qkv, &t.qkv)) ||
          (rc = tile(L.o, &t.o)))
        return rc;
      tiled.push_back(t);
    }
    CHECK_HIP(hipStreamSynchronize(stream));
    return MOERT_OK;
  }

  // Positions pos0 .. pos0 + nv - 1 through every layer, then the final norm, head and argmax of the last one (the
  // device state already holds pos = pos0 + nv - 1, fixed = pos0 + nv and *pf.pos0 = pos0); its hidden state is
  // left in b.h, as after a decode step.
  int enqueue_batched(int pos0, int nv) {
    CHECK_HIP(launch_embed_b(stream, embed, dims, pf, nv));
    if (batched_mode == 1) CHECK_HIP(launch_norm_codes(stream, dims.hidden, nv, pf.h, layers[0].ln_attn, dims.eps, mg));
    for (size_t l = 0; l < layers.size(); l++) {
      if (batched_mode == 1) {
        GroupBufs g = mg;
        g.gu = tiled[l].gu;
        g.dn = tiled[l].dn;
        g.qkv = tiled[l].qkv;
        g.oproj = tiled[l].o;
        const float* next = l + 1 < layers.size() ? layers[l + 1].ln_attn : nullptr;
        CHECK_HIP(launch_layer_grouped(stream, layers[l], dims, pf, pf.pos0, pos0, nv, b.rope, g, next));
      } else {
        CHECK_HIP(launch_layer_b(stream, layers[l], dims, pf, pf.pos0, pos0, nv, b.rope));
      }
    }
    StepBufs bl = b;
    bl.h = pf.h + (size_t)(nv - 1) * dims.hidden;
    CHECK_HIP(launch_head(stream, embed, norm, dims, bl));
    CHECK_HIP(launch_head_argmax(stream, embed, dims, bl));
    CHECK_HIP(hipMemcpyAsync(b.h, bl.h, (size_t)dims.hidden * 4, hipMemcpyDeviceToDevice, stream));
    return MOERT_OK;
  }

  int write_state(int pos, int fixed) {
    int st[ST_WORDS] = {pos, fixed, 0, 0};
    CHECK_HIP(hipMemcpyAsync(b.state, st, sizeof st, hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipStreamSynchronize(stream));
    host_pos = pos;
    return MOERT_OK;
  }

  // Empties the pool and zeroes the clock and the counters (ExpertCache::clear, rust/moe-rt/src/cache.rs:216-220):
  // both copies of the slot tables, copy 0 current.
  int cache_clear() {
    CHECK_HIP(hipMemsetAsync(cache.slot_key, 0xff, 2 * (size_t)cache.slots * 4, stream));
    CHECK_HIP(hipMemsetAsync(cache.slot_last, 0, 2 * (size_t)cache.slots * 4, stream));
    CHECK_HIP(hipMemsetAsync(cache.clock, 0, 2 * 4, stream));
    CHECK_HIP(hipMemsetAsync(cache.cur, 0, 4, stream));
    CHECK_HIP(hipMemsetAsync(cache.stats, 0, CS_WORDS * 8, stream));
    CHECK_HIP(hipMemsetAsync(cache.pf, 0, 17 * 4, stream));
    CHECK_HIP(hipMemsetAsync(cache.pred_hist, 0xff, (size_t)max_len * cfg.layers * 8 * 4, stream));
    CHECK_HIP(hipMemsetAsync(cache.tok_hist, 0, (size_t)max_len * cfg.layers * 4 * 4, stream));
    CHECK_HIP(hipStreamSynchronize(stream));
    return MOERT_OK;
  }

  // Expert records into pool slots decided on the host, between steps (ExpertCache::fill, rust/moe-rt/src/
  // cache.rs:212-227, and a per-layer prefetch). The model stream is synchronised and the current copy of the slot
  // tables read back; then for `keys` in order:
  //  - prefetch (tick): one clock tick as a layer step's LRU decision makes it (lru_decide): keys already in the
  //    pool are touched first (pinned for the tick); each other key takes the first free slot, else the least
  //    recently used slot not touched at this tick (lowest index on ties);
  //  - fill (!tick): a key not in the pool takes the first free slot, stamped with the current clock (not advanced),
  //    as copy_on_compute stamps last_use: self.clock (rust/moe-rt/src/cache/core.rs:366-377); nothing is evicted
  //    and the fill stops when no slot is free.
  // The records are copied with hipMemcpyAsync from the pinned store on a side stream, the model stream waits for
  // them, the tables and the clock are written back, and the call returns synchronised. The hit and copy counters
  // count the requests of decode steps only and are left alone.
  int cache_load(const int* keys, int n, bool tick, int* copied) {
    const int S = cache.slots;
    CHECK_HIP(hipStreamSynchronize(stream));
    int cur = 0, clock = 0;
    std::vector<int> skey(S), slast(S);
    CHECK_HIP(hipMemcpy(&cur, cache.cur, 4, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(&clock, cache.clock + cur, 4, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(skey.data(), cache.slot_key + (size_t)cur * S, (size_t)S * 4, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(slast.data(), cache.slot_last + (size_t)cur * S, (size_t)S * 4, hipMemcpyDeviceToHost));
    std::vector<std::pair<int, int>> loads;  // (slot, key)
    auto where = [&](int key) {
      for (int i = 0; i < S; i++)
        if (skey[i] == key) return i;
      return -1;
    };
    if (tick) {
      clock++;
      for (int j = 0; j < n; j++) {
        const int i = where(keys[j]);
        if (i >= 0) slast[i] = clock;
      }
    }
    for (int j = 0; j < n; j++) {
      if (where(keys[j]) >= 0) continue;
      int v = -1;
      for (int i = 0; i < S && v < 0; i++)
        if (skey[i] < 0) v = i;
      if (v < 0 && tick)
        for (int i = 0; i < S; i++)
          if (slast[i] < clock && (v < 0 || slast[i] < slast[v])) v = i;
      if (v < 0) {
        if (!tick) break;  // fill: the pool is full
        continue;          // (cannot happen: n <= slots)
      }
      skey[v] = keys[j];
      slast[v] = clock;
      loads.push_back({v, keys[j]});
    }
    if (!loads.empty()) {
      if (!side) CHECK_HIP(hipStreamCreateWithFlags(&side, hipStreamNonBlocking));
      if (!side_done) CHECK_HIP(hipEventCreateWithFlags(&side_done, hipEventDisableTiming));
      const size_t dn_d = cache.record_bytes - cache.gu_q - cache.gu_d - cache.dn_q;
      // a run of loads with consecutive slots and consecutive keys is one strided copy per piece: the records sit
      // record_bytes apart in the store, and each piece's slots are contiguous in its pool plane
      for (size_t a = 0; a < loads.size();) {
        size_t b = a + 1;
        while (b < loads.size() && loads[b].first == loads[b - 1].first + 1 &&
               loads[b].second == loads[b - 1].second + 1)
          b++;
        const uint8_t* r = (const uint8_t*)host_store + (size_t)loads[a].second * cache.record_bytes;
        const size_t v = (size_t)loads[a].first, rows = b - a, rb = cache.record_bytes;
        auto piece = [&](const uint8_t* dst, const uint8_t* src, size_t bytes) -> hipError_t {
          return hipMemcpy2DAsync((void*)dst, bytes, src, rb, bytes, rows, hipMemcpyHostToDevice, side);
        };
        CHECK_HIP(piece(cache.pool_gu.q + v * cache.gu_q, r, cache.gu_q));
        if (cache.gu_d) CHECK_HIP(piece((const uint8_t*)cache.pool_gu.d + v * cache.gu_d, r + cache.gu_q, cache.gu_d));
        r += cache.gu_q + cache.gu_d;
        CHECK_HIP(piece(cache.pool_dn.q + v * cache.dn_q, r, cache.dn_q));
        if (dn_d) CHECK_HIP(piece((const uint8_t*)cache.pool_dn.d + v * dn_d, r + cache.dn_q, dn_d));
        a = b;
      }
      CHECK_HIP(hipEventRecord(side_done, side));
      CHECK_HIP(hipStreamWaitEvent(stream, side_done, 0));
    }
    CHECK_HIP(hipMemcpyAsync(cache.slot_key + (size_t)cur * S, skey.data(), (size_t)S * 4, hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipMemcpyAsync(cache.slot_last + (size_t)cur * S, slast.data(), (size_t)S * 4, hipMemcpyHostToDevice,
                             stream));
    CHECK_HIP(hipMemcpyAsync(cache.clock + cur, &clock, 4, hipMemcpyHostToDevice, stream));
    CHECK_HIP(hipStreamSynchronize(stream));
    if (copied) *copied = (int)loads.size();
    return MOERT_OK;
  }
  hipStream_t side = nullptr;  // copy stream of cache_load
  hipEvent_t side_done = nullptr;

  ~moert_model() {
    if (pf_stream) (void)hipStreamSynchronize(pf_stream);
    if (side) (void)hipStreamSynchronize(side);
    if (side_done) (void)hipEventDestroy(side_done);
    if (side) (void)hipStreamDestroy(side);
    if (stream) (void)hipStreamSynchronize(stream);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (tl_buf) (void)hipFree(tl_buf);
    arena.release();
    if (host_store) (void)hipHostFree(host_store);
    for (hipEvent_t e : {ev_fork, ev_pred, ev_copy, mx_ev, mx_t[0], mx_t[1], mx_t[2]})
      if (e) (void)hipEventDestroy(e);
    if (mx_pin) (void)hipHostFree(mx_pin);
    for (hipEvent_t e : hy_evs)
      if (e) (void)hipEventDestroy(e);
    for (void* p : {(void*)hy_table_pin, (void*)hy_ids_pin, (void*)hy_w_pin, (void*)hy_xn_pin, (void*)hy_y_pin,
                    (void*)hy_flag_pin})
      if (p) (void)hipHostFree(p);
    if (pf_stream) (void)hipStreamDestroy(pf_stream);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

// Experts of every layer into a pinned host store of records [gu payload | gu scales | down payload | down scales]
// (key = layer * E + expert) and an HBM pool of `slots` records as two SoA matrices; LRU tables emptied.
static int cache_create(moert_model* m, const moert_model_weights* w, int slots) {
  const moert_config& c = m->cfg;
  const int H = c.hidden, I = c.inter, E = c.experts, L = c.layers;
  const int dt = w->layers[0].gate_up.dtype;
  for (int l = 0; l < L; l++)
    CHECK_CFG(w->layers[l].gate_up.dtype == dt && w->layers[l].down.dtype == dt,
              "expert cache: every layer's experts must share one dtype");
  CHECK_CFG(slots >= c.top_k && slots <= kCacheMaxSlots && slots <= L * E,
            "expert cache: %d slots outside [top_k, min(%d, layers*experts)]", slots, kCacheMaxSlots);
  CacheDev& cd = m->cache;
  const size_t gu_rows = 2 * (size_t)I, dn_rows = H;
  cd.gu_q = gu_rows * payload_bytes(dt, H);
  cd.gu_d = dt == MOERT_F32 ? 0 : gu_rows * (H / 32) * 2;
  cd.dn_q = dn_rows * payload_bytes(dt, I);
  const size_t dn_d = dt == MOERT_F32 ? 0 : dn_rows * (I / 32) * 2;
  cd.record_bytes = cd.gu_q + cd.gu_d + cd.dn_q + dn_d;
  CHECK_CFG(cd.gu_q % 16 == 0 && cd.gu_d % 16 == 0 && cd.dn_q % 16 == 0 && dn_d % 16 == 0,
            "expert cache: record pieces must be multiples of 16 bytes");
  const size_t total = cd.record_bytes * (size_t)L * E;
  CHECK_HIP(hipHostMalloc(&m->host_store, total, hipHostMallocMapped | hipHostMallocNonCoherent));
  uint8_t* hs = (uint8_t*)m->host_store;
  for (int l = 0; l < L; l++) {
    const moert_layer_weights& W = w->layers[l];
    CHECK_CFG(W.gate_up.data && W.down.data, "layer %d: missing experts", l);
    for (int e = 0; e < E; e++) {
      uint8_t* r = hs + ((size_t)l * E + e) * cd.record_bytes;
      repack_rows(W.gate_up.data, dt, H, (size_t)e * gu_rows, gu_rows, r, (uint16_t*)(r + cd.gu_q));
      uint8_t* rd = r + cd.gu_q + cd.gu_d;
      repack_rows(W.down.data, dt, I, (size_t)e * dn_rows, dn_rows, rd, (uint16_t*)(rd + cd.dn_q));
    }
  }
  void* dev_host = nullptr;
  CHECK_HIP(hipHostGetDevicePointer(&dev_host, m->host_store, 0));
  cd.host = (const uint8_t*)dev_host;
  Arena& a = m->arena;
  void* p;
  int rc;
  auto mat = [&](size_t rows, int cols, DMat* out) -> int {
    const size_t plane = rows * payload_bytes(dt, cols), sc = dt == MOERT_F32 ? 0 : rows * (cols / 32) * 2;
    int r = a.alloc(&p, align256(plane) + sc);
    if (r) return r;
    *out = DMat{(const uint8_t*)p, sc ? (const uint16_t*)((uint8_t*)p + align256(plane)) : nullptr, dt, (int)rows, cols};
    return MOERT_OK;
  };
  if ((rc = mat((size_t)slots * gu_rows, H, &cd.pool_gu)) || (rc = mat((size_t)slots * dn_rows, I, &cd.pool_dn)))
    return rc;
  cd.slots = slots;
  cd.experts = E;
  if ((rc = a.alloc(&p, 2 * (size_t)slots * 4))) return rc;
  cd.slot_key = (int*)p;
  if ((rc = a.alloc(&p, 2 * (size_t)slots * 4))) return rc;
  cd.slot_last = (int*)p;
  if ((rc = a.alloc(&p, 2 * 4))) return rc;
  cd.clock = (int*)p;
  if ((rc = a.alloc(&p, 4))) return rc;
  cd.cur = (int*)p;
  if ((rc = a.alloc(&p, CS_WORDS * 8))) return rc;
  cd.stats = (unsigned long long*)p;
  if ((rc = a.alloc(&p, 16 * 4))) return rc;
  cd.route = (int*)p;
  if ((rc = a.alloc(&p, 17 * 4))) return rc;
  cd.pf = (int*)p;
  if ((rc = a.alloc(&p, 17 * 8))) return rc;
  cd.pfx = (uint2*)p;
  CHECK_HIP(hipMemsetAsync(cd.pfx, 0, 17 * 8, m->stream));  // epoch 0: written by no launch
  if ((rc = a.alloc(&p, (size_t)m->max_len * L * 8 * 4))) return rc;
  cd.pred_hist = (int*)p;
  if ((rc = a.alloc(&p, (size_t)m->max_len * L * 4 * 4))) return rc;
  cd.tok_hist = (int*)p;
  cd.state = m->b.state;
  cd.layers = L;
  m->cached = true;
  return m->cache_clear();
}

static int model_create(const moert_config* c, const moert_model_weights* w, int max_len, int splits,
                        int cache_slots, moert_model** out, bool graph = true) {
  CHECK_CFG(c && w && out, "null argument");
  *out = nullptr;
  CHECK_CFG(c->head_dim == 64, "head_dim %d: the attention kernels are built for 64", c->head_dim);
  CHECK_CFG(c->heads > 0 && c->kv_heads > 0 && c->heads % c->kv_heads == 0 && c->heads / c->kv_heads <= 4,
            "heads %d / kv_heads %d: need a group of at most 4 query heads per KV head", c->heads, c->kv_heads);
  CHECK_CFG(c->experts >= 1 && c->experts <= 64 && c->top_k >= 1 && c->top_k <= 8 && c->top_k <= c->experts,
            "experts %d, top_k %d: need top_k <= 8 and experts <= 64", c->experts, c->top_k);
  CHECK_CFG(k_supported(c->hidden) && k_supported(c->heads * 64) && (c->inter == 128 || c->inter == 256 || c->inter == 512),
            "hidden %d / heads*64 %d / inter %d outside the compiled row lengths", c->hidden, c->heads * 64, c->inter);
  CHECK_CFG(max_len >= 64 && max_len % 64 == 0, "max_len %d must be a positive multiple of 64", max_len);
  CHECK_CFG(splits >= 1 && splits <= 64, "attn_splits %d outside [1, 64]", splits);
  CHECK_CFG(c->layers >= 1 && c->vocab >= 1 && w->layers && w->norm, "empty model");
  const int H = c->hidden, d = 64, qd = c->heads * d, kvd = c->kv_heads * d, I = c->inter, E = c->experts;
  for (int l = 0; l < c->layers; l++) {
    const moert_layer_weights& L = w->layers[l];
    CHECK_CFG(L.q.dtype == L.k.dtype && L.q.dtype == L.v.dtype, "layer %d: q, k, v must share a dtype", l);
    CHECK_CFG(L.router.dtype == L.gate_up.dtype && L.o.dtype == L.router.dtype,
              "layer %d: o, router and gate_up must share a dtype", l);
    CHECK_CFG(L.ln_attn && L.ln_moe, "layer %d: missing norm weights", l);
  }
  moert_model* m = new moert_model;
  m->cfg = *c;
  m->max_len = max_len;
  m->splits = splits;
  // tiles of 64 positions per attention split: the cache is cut into at most `splits` splits
  const int tps = ((max_len / 64) + splits - 1) / splits;
  m->dims = Dims{H, I, c->heads, c->kv_heads, d, c->vocab, E, c->top_k, max_len, tps,
                 c->eps, c->embedding_multiplier, c->residual_multiplier, c->attention_multiplier, c->logits_scaling};
  auto bail = [&](int rc) {
    delete m;
    return rc;
  };
  if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) {
    set_err("hipStreamCreate failed");
    return bail(MOERT_E_DEVICE);
  }
  hipStream_t s = m->stream;
  Arena& a = m->arena;
  int rc;
  m->layers.resize(c->layers);
  for (int l = 0; l < c->layers; l++) {
    const moert_layer_weights& W = w->layers[l];
    LayerDev& L = m->layers[l];
    float* tmp;
    if ((rc = upload_f32(a, s, W.ln_attn, H, &tmp))) return bail(rc);
    L.ln_attn = tmp;
    if ((rc = upload_f32(a, s, W.ln_moe, H, &tmp))) return bail(rc);
    L.ln_moe = tmp;
    if ((rc = upload_matrix(a, s, {{W.q.data, qd}, {W.k.data, kvd}, {W.v.data, kvd}}, W.q.dtype, H, &L.qkv))) return bail(rc);
    if ((rc = upload_matrix(a, s, {{W.o.data, H}}, W.o.dtype, qd, &L.o))) return bail(rc);
    if ((rc = upload_matrix(a, s, {{W.router.data, E}}, W.router.dtype, H, &L.router))) return bail(rc);
    L.router_bias = nullptr;
    if (W.router_bias) {
      if ((rc = upload_f32(a, s, W.router_bias, E, &tmp))) return bail(rc);
      L.router_bias = tmp;
    }
    if (cache_slots == 0) {
      if ((rc = upload_matrix(a, s, {{W.gate_up.data, E * 2 * I}}, W.gate_up.dtype, H, &L.gate_up))) return bail(rc);
      if ((rc = upload_matrix(a, s, {{W.down.data, E * H}}, W.down.dtype, I, &L.down))) return bail(rc);
    }
    if ((rc = zeros(a, s, (size_t)c->kv_heads * max_len * d, &L.k_cache))) return bail(rc);
    if ((rc = zeros(a, s, (size_t)c->kv_heads * max_len * d, &L.v_cache))) return bail(rc);
  }
  if ((rc = upload_matrix(a, s, {{w->embed.data, c->vocab}}, w->embed.dtype, H, &m->embed))) return bail(rc);
  if ((rc = upload_f32(a, s, w->norm, H, &m->norm))) return bail(rc);
  // RoPE table computed on the host as in rust/moe-rt/src/model.rs:63-73 (f32 powf, cosf, sinf).
  std::vector<float> rope((size_t)max_len * d);
  for (int p = 0; p < max_len; p++)
    for (int j = 0; j < d / 2; j++) {
      float f = 1.0f / powf(c->rope_theta, (float)(2 * j) / (float)d);
      float ang = (float)p * f;
      rope[(size_t)p * d + j] = cosf(ang);
      rope[(size_t)p * d + d / 2 + j] = sinf(ang);
    }
  StepBufs& b = m->b;
  float* rp;
  if ((rc = upload_f32(a, s, rope.data(), rope.size(), &rp))) return bail(rc);
  b.rope = rp;
  m->n_head_blocks = head_blocks(m->embed);
  if ((rc = zeros(a, s, H, &b.h)) || (rc = zeros(a, s, qd, &b.q)) || (rc = zeros(a, s, qd, &b.att)) ||
      (rc = zeros(a, s, (size_t)c->heads * attn_splits_for(max_len, tps) * 66, &b.part)) ||
      (rc = zeros(a, s, (size_t)kNormItems, &b.zpart)) ||
      (rc = zeros(a, s, (size_t)c->top_k * I, &b.act)) ||
      (rc = zeros(a, s, (size_t)c->layers * c->top_k, &b.route_ids)) ||
      (rc = zeros(a, s, (size_t)c->layers * c->top_k, &b.route_w)) || (rc = zeros(a, s, c->vocab, &b.logits)) ||
      (rc = zeros(a, s, (size_t)m->n_head_blocks, &b.best)) ||
      (rc = zeros(a, s, max_len, &b.seq)) || (rc = zeros(a, s, max_len, &b.argmax_hist)) ||
      (rc = zeros(a, s, ST_WORDS, &b.state)))
    return bail(rc);
  {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
      set_err("hipGetDeviceProperties failed");
      return bail(MOERT_E_DEVICE);
    }
    m->cus = prop.multiProcessorCount;
    const char* ev = getenv("MOERT_ATTN_BLOCK");
    const bool allow = !(ev && ev[0] == '0');
    unsigned *grp = nullptr, *mx = nullptr;
    if ((rc = zeros(a, s, 8 * sizeof(AbGroup) / 4, &grp)) || (rc = zeros(a, s, 8 * sizeof(MxGroup) / 4, &mx)) ||
        (rc = zeros(a, s, (size_t)8 * H, &m->ab.ys)) || (rc = zeros(a, s, (size_t)H, &b.hc)) ||
        (rc = zeros(a, s, (size_t)1, &m->ab.step_ctr)) || (rc = zeros(a, s, (size_t)2, &m->ab.err)) ||
        (rc = zeros(a, s, (size_t)64, &m->ab.rope_cur)))
      return bail(rc);
    m->ab.groups = reinterpret_cast<AbGroup*>(grp);
    m->ab.moe = reinterpret_cast<MxGroup*>(mx);
    m->use_ab = allow && c->layers <= 63 && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
                attn_block_fits(m->dims, m->layers[0].qkv, m->cus);
    const char* mv = getenv("MOERT_MOE_XCD");
    m->use_mx = m->use_ab && cache_slots == 0 && !(mv && mv[0] == '0') && moe_xcd_fits(m->dims, m->layers[0], m->cus);
    const char* lv = getenv("MOERT_LAYER");
    if (m->use_mx && !(lv && lv[0] == '0') && layers_fit(m->dims, m->layers[0], m->cus)) {
      unsigned *pxx = nullptr, *pxd = nullptr;
      float* hpp = nullptr;
      if ((rc = zeros(a, s, 8 * sizeof(PxXcd) / 4, &pxx)) || (rc = zeros(a, s, sizeof(PxDev) / 4, &pxd)) ||
          (rc = zeros(a, s, (size_t)H, &hpp)))
        return bail(rc);
      m->px = PxBufs{reinterpret_cast<PxXcd*>(pxx), reinterpret_cast<PxDev*>(pxd), hpp};
      for (const LayerDev& L : m->layers)
        m->pxl.push_back(PxLayer{L.qkv, L.o, L.router, L.gate_up, L.down, L.ln_attn, L.ln_moe, L.router_bias,
                                 L.k_cache, L.v_cache});
      m->use_px = true;
    }
  }
  if (hipStreamSynchronize(s) != hipSuccess) {
    set_err("upload failed");
    return bail(MOERT_E_DEVICE);
  }
  if (cache_slots > 0 && (rc = cache_create(m, w, cache_slots))) return bail(rc);
  if (graph && (rc = m->build_graph())) return bail(rc);
  *out = m;
  return MOERT_OK;
}

// ------------------------------------------------------------------------------------------------------------
// One MoE block with every expert resident (GpuLayer, rust/moe-rt/src/gpu.rs:368-541).
struct moert_block {
  Dims dims{};
  hipStream_t stream = nullptr;
  Arena arena;
  LayerDev L{};
  StepBufs b{};
  float* x = nullptr;
  // multi-position (grouped) step buffers, allocated on first use
  GroupBufs g{};
  float* gx = nullptr;
  float* gy = nullptr;
  // the batched step as one launch (moert_block_batched_kernel 1): its exchange buffers (on first use), the launch
  // epoch (never 0) and the device's compute units
  int fused = 0;
  FbBufs fb{};
  unsigned fb_epoch = 0;
  int cus = 0;
  int ensure_fused() {
    if (fb.err) return MOERT_OK;
    const size_t H = dims.hidden, P = kFbPos;
    unsigned *err = nullptr, *lg = nullptr, *xf = nullptr, *act = nullptr, *o = nullptr, *rk = nullptr;
    int rc;
    if ((rc = zeros(arena, stream, 2, &err)) || (rc = zeros(arena, stream, 8 * P * 64 * 2, &lg)) ||
        (rc = zeros(arena, stream, 8 * P * 2, &xf)) || (rc = zeros(arena, stream, 8 * P * H, &fb.xh)) ||
        (rc = zeros(arena, stream, 8 * P * H, &fb.xl)) || (rc = zeros(arena, stream, 8 * P * (H / 32), &fb.xd)) ||
        (rc = zeros(arena, stream, (size_t)kFbExperts * (kFbInter / 32) * kFbActW * P * 2, &act)) ||
        (rc = zeros(arena, stream, P * 8 * H * 2, &o)) || (rc = zeros(arena, stream, 8 * P * 16 * 2, &rk)))
      return rc;
    fb.err = err;
    fb.lg = reinterpret_cast<uint2*>(lg);
    fb.xflag = reinterpret_cast<uint2*>(xf);
    fb.act = reinterpret_cast<uint2*>(act);
    fb.o = reinterpret_cast<uint2*>(o);
    fb.rk = reinterpret_cast<uint2*>(rk);
    CHECK_HIP(hipStreamSynchronize(stream));
    return MOERT_OK;
  }
  // one batched step of m positions from gx into gy on stream s; with `ev`, its dispatches record into the event
  // pairs (the one launch into the first)
  int launch_batched(hipStream_t s, int m, const hipEvent_t* ev) {
    if (!fused) {
      CHECK_HIP(launch_grouped_block(s, L, m, dims.top_k, dims.inter, gx, g, gy, ev));
      return MOERT_OK;
    }
    if (++fb_epoch == 0) {
      // the epochs wrapped: every exchange entry back to epoch 0, which no launch writes, so that an entry left by a
      // launch 2^32 steps ago can never pass for a current one
      const size_t H = dims.hidden, P = kFbPos;
      CHECK_HIP(hipMemsetAsync(fb.lg, 0, 8 * P * 64 * 8, s));
      CHECK_HIP(hipMemsetAsync(fb.xflag, 0, 8 * P * 8, s));
      CHECK_HIP(hipMemsetAsync(fb.act, 0, (size_t)kFbExperts * (kFbInter / 32) * kFbActW * P * 8, s));
      CHECK_HIP(hipMemsetAsync(fb.o, 0, P * 8 * H * 8, s));
      CHECK_HIP(hipMemsetAsync(fb.rk, 0, 8 * P * 16 * 8, s));
      fb_epoch = 1;
    }
    if (ev) arm_launch_events(ev[0], ev[1]);
    CHECK_HIP(launch_grp_fused(s, L, m, dims.top_k, dims.inter, gx, g, fb, fb_epoch, gy, cus));
    return MOERT_OK;
  }
  // the one-launch step's error word: a wait that gave up. A block step carries nothing into the next one, so the
  // word is cleared once reported (the stream is idle) and the next step starts clean.
  int fused_check() {
    if (!fused) return MOERT_OK;
    unsigned e = 0;
    CHECK_HIP(hipMemcpy(&e, fb.err, 4, hipMemcpyDeviceToHost));
    if (e) {
      const unsigned zero = 0;
      CHECK_HIP(hipMemcpy(fb.err, &zero, 4, hipMemcpyHostToDevice));
      set_err("batched step (one launch) gave up waiting for %s%s%s%s(error bits %#x): its workgroups were not "
              "all resident at once or not dealt round-robin over the XCDs", (e & 1u) ? "router logits " : "",
              (e & 2u) ? "act vectors " : "", (e & 4u) ? "expert outputs " : "", (e & 8u) ? "input codes " : "", e);
      return MOERT_E_DEVICE;
    }
    return MOERT_OK;
  }
  int ensure_grouped() {
    if (gx) return MOERT_OK;
    const int H = dims.hidden, I = dims.inter, M = kGrpMaxPos, S = kGrpMaxPos * 8;
    int rc;
    if ((rc = zeros(arena, stream, (size_t)M * H, &gx)) || (rc = zeros(arena, stream, (size_t)M * H, &gy)) ||
        (rc = zeros(arena, stream, (size_t)S, &g.ids)) || (rc = zeros(arena, stream, (size_t)S, &g.w)) ||
        (rc = zeros(arena, stream, (size_t)M * H, &g.xh)) || (rc = zeros(arena, stream, (size_t)M * H, &g.xl)) ||
        (rc = zeros(arena, stream, (size_t)M * (H / 32), &g.xd)) || (rc = zeros(arena, stream, (size_t)GRP_WORDS, &g.grp)) ||
        (rc = zeros(arena, stream, (size_t)S * I, &g.ah)) || (rc = zeros(arena, stream, (size_t)S * I, &g.al)) ||
        (rc = zeros(arena, stream, (size_t)S * (I / 32), &g.ad)) || (rc = zeros(arena, stream, (size_t)S * H, &g.o)))
      return rc;
    // the experts in the tiled layout of the MFMA kernels, copied once from the resident matrices
    auto tiled = [&](const DMat& src, TMat* dst) -> int {
      uint8_t* q;
      uint16_t* d;
      const size_t n = (size_t)src.rows * src.cols;
      int r;
      if ((r = arena.alloc((void**)&q, n)) || (r = arena.alloc((void**)&d, n / 32 * 2))) return r;
      CHECK_HIP(launch_tile_q8(stream, src, q, d));
      *dst = TMat{q, d, src.rows, src.cols};
      return MOERT_OK;
    };
    if ((rc = tiled(L.gate_up, &g.gu)) || (rc = tiled(L.down, &g.dn))) return rc;
    CHECK_HIP(hipStreamSynchronize(stream));
    return MOERT_OK;
  }
  ~moert_block() {
    if (stream) (void)hipStreamSynchronize(stream);
    arena.release();
    if (stream) (void)hipStreamDestroy(stream);
  }
  int enqueue() {
    CHECK_HIP(launch_route_up(stream, L, dims, b, 0, false));
    CHECK_HIP(launch_expert_down(stream, L, dims, b, 0, false));
    return MOERT_OK;
  }
};

// ------------------------------------------------------------------------------------------------------------
// Per-call device context for the unit-parity entry points.
namespace {
struct Scoped {
  std::vector<void*> ptrs;
  hipStream_t s = nullptr;
  ~Scoped() {
    if (s) (void)hipStreamSynchronize(s);
    for (void* p : ptrs) (void)hipFree(p);
    if (s) (void)hipStreamDestroy(s);
  }
  int init() {
    CHECK_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    return MOERT_OK;
  }
  template <class T>
  int dev(T** p, size_t n, const void* src = nullptr) {
    void* q;
    CHECK_HIP(hipMalloc(&q, n * sizeof(T) ? n * sizeof(T) : 4));
    ptrs.push_back(q);
    if (src)
      CHECK_HIP(hipMemcpyAsync(q, src, n * sizeof(T), hipMemcpyHostToDevice, s));
    else
      CHECK_HIP(hipMemsetAsync(q, 0, n * sizeof(T) ? n * sizeof(T) : 4, s));
    *p = (T*)q;
    return MOERT_OK;
  }
  int get(void* dst, const void* src, size_t bytes) {
    CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
    CHECK_HIP(hipStreamSynchronize(s));
    return MOERT_OK;
  }
};

int unit_matrix(Scoped& sc, const moert_tensor* w, int rows, int cols, DMat* out) {
  Arena a;
  int rc = upload_matrix(a, sc.s, {{w->data, rows}}, w->dtype, cols, out);
  for (void* p : a.ptrs) sc.ptrs.push_back(p);
  return rc;
}
}  // namespace

#define TRY(expr)              \
  do {                         \
    int rc_ = (expr);          \
    if (rc_) return rc_;       \
  } while (0)

extern "C" {

const char* moert_last_error(void) { return g_err.c_str(); }

int moert_device_info(int* count, char* name, int name_len) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  if (count) *count = n;
  if (name && name_len > 0) {
    name[0] = 0;
    hipDeviceProp_t p;
    if (n > 0 && hipGetDeviceProperties(&p, 0) == hipSuccess) snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
  }
  return MOERT_OK;
}

int moert_model_create(const moert_config* cfg, const moert_model_weights* w, int max_len, int attn_splits,
                       moert_model** out) {
  return model_create(cfg, w, max_len, attn_splits, 0, out);
}

int moert_model_create_cached(const moert_config* cfg, const moert_model_weights* w, int max_len, int attn_splits,
                              int slots, moert_model** out) {
  CHECK_CFG(slots >= 1, "expert cache: %d slots", slots);
  return model_create(cfg, w, max_len, attn_splits, slots, out);
}

int moert_model_create_hybrid(const moert_config* cfg, const moert_model_weights* w, int max_len, int attn_splits,
                              int slots, int backlog, int cpu_threads, moert_model** out) {
  CHECK_CFG(cfg && out, "null argument");
  CHECK_CFG(slots >= 0 && slots <= cfg->layers * cfg->experts && slots <= kCacheMaxSlots,
            "hybrid: %d slots outside [0, min(layers * experts, %d)]", slots, kCacheMaxSlots);
  CHECK_CFG(backlog >= 0 && cpu_threads >= 1 && cpu_threads <= 64, "hybrid: backlog %d, cpu_threads %d", backlog,
            cpu_threads);
  // the pool and the host store of the expert cache (at least top_k slots are allocated; the placement uses `slots`)
  int rc = model_create(cfg, w, max_len, attn_splits, std::max(slots, cfg->top_k), out, false);
  if (rc) return rc;
  moert_model* m = *out;
  auto bail = [&](int code) {
    delete m;
    *out = nullptr;
    return code;
  };
  const int L = cfg->layers, E = cfg->experts, H = cfg->hidden;
  m->hybrid = true;
  m->hy_threads = cpu_threads;
  m->place.reset(new Placement(L, E, cfg->top_k, slots, backlog));
  m->place->start();
  void* p = nullptr;
  if ((rc = m->arena.alloc(&p, (size_t)L * E * 4))) return bail(rc);
  m->hy_table = (int*)p;
  if ((rc = m->arena.alloc(&p, (size_t)H * 4))) return bail(rc);
  m->hy_xn_dev = (float*)p;
  if (hipHostMalloc((void**)&m->hy_table_pin, (size_t)L * E * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&m->hy_ids_pin, 2 * 8 * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&m->hy_w_pin, 2 * 8 * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&m->hy_xn_pin, 2 * (size_t)H * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&m->hy_y_pin, (size_t)H * 4, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
      hipHostGetDevicePointer((void**)&m->hy_y_dev, m->hy_y_pin, 0) != hipSuccess ||
      hipHostMalloc((void**)&m->hy_flag_pin, (size_t)L * 4, hipHostMallocMapped | hipHostMallocCoherent) !=
          hipSuccess ||
      hipHostGetDevicePointer((void**)&m->hy_flag_dev, m->hy_flag_pin, 0) != hipSuccess) {
    set_err("hybrid: pinned host buffers or event");
    return bail(MOERT_E_DEVICE);
  }
  std::memset(m->hy_flag_pin, 0, (size_t)L * 4);
  m->hy_evs.assign((size_t)L, nullptr);
  for (hipEvent_t& e : m->hy_evs)
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
      set_err("hybrid: events");
      return bail(MOERT_E_DEVICE);
    }
  if ((rc = zeros(m->arena, m->stream, 1, &m->hy_err))) return bail(rc);
  m->cache.table = m->hy_table;
  m->cache.xn = m->hy_xn_dev;
  m->hy_act.assign((size_t)cfg->top_k * cfg->inter, 0.0f);
  m->hy_y.assign((size_t)H, 0.0f);
  m->hy_tok.assign((size_t)max_len * L * 4, 0);
  return MOERT_OK;
}

int moert_model_destroy(moert_model* m) {
  delete m;
  return MOERT_OK;
}

#define MODEL_OK(m)                                                      \
  do {                                                                   \
    if (!(m)) {                                                          \
      set_err("null model");                                             \
      return MOERT_E_CONFIG;                                             \
    }                                                                    \
    if ((m)->poisoned) {                                                 \
      set_err("model unusable after an earlier device error");          \
      return MOERT_E_POISONED;                                           \
    }                                                                    \
  } while (0)

#define MTRY(m, expr)                 \
  do {                                \
    int rc_ = (expr);                 \
    if (rc_) return (m)->fail(rc_);   \
  } while (0)

static int model_copy_in(moert_model* m, void* dst, const void* src, size_t bytes) {
  CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, m->stream));
  return MOERT_OK;
}
static int model_copy_out(moert_model* m, void* dst, const void* src, size_t bytes) {
  CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, m->stream));
  return MOERT_OK;
}
// MOERT_GRAPH=0 launches the step's kernels one by one instead of replaying the captured graph (for tracing
// tools that do not follow graph launches); results are the same.
static bool use_graph() {
  static const bool on = [] {
    const char* v = getenv("MOERT_GRAPH");
    return !(v && v[0] == '0');
  }();
  return on;
}

// A launch's epoch is step_ctr * 64 + layer + 1 in 32 bits. Before the step counter could reach 2^26 - 1 (where
// epochs would wrap, and an exchange entry left by a launch of long ago could carry a current epoch), the exchange
// areas and the counter are cleared in stream order: every entry back to epoch 0, which no launch writes.
constexpr unsigned long long kEpochSteps = (1ull << 26) - 2;
static int epoch_guard(moert_model* m) {
  if (++m->steps_since_clear < kEpochSteps) return MOERT_OK;
  CHECK_HIP(hipMemsetAsync(m->ab.groups, 0, 8 * sizeof(AbGroup), m->stream));
  CHECK_HIP(hipMemsetAsync(m->ab.moe, 0, 8 * sizeof(MxGroup), m->stream));
  CHECK_HIP(hipMemsetAsync(m->ab.step_ctr, 0, 4, m->stream));
  if (m->cached) CHECK_HIP(hipMemsetAsync(m->cache.pfx, 0, 17 * 8, m->stream));
  if (m->use_px) {
    CHECK_HIP(hipMemsetAsync(m->px.xcd, 0, 8 * sizeof(PxXcd), m->stream));
    CHECK_HIP(hipMemsetAsync(m->px.dev, 0, sizeof(PxDev), m->stream));
  }
  m->steps_since_clear = 1;
  return MOERT_OK;
}

static int model_launch(moert_model* m) {
  int rc = epoch_guard(m);
  if (rc) return rc;
  if (m->hybrid) return m->hybrid_step();
  if (!use_graph()) return m->enqueue(-1, nullptr);
  CHECK_HIP(hipGraphLaunch(m->exec, m->stream));
  return MOERT_OK;
}
// A bit that k_attn_block, k_moe_xcd or k_layer set (a bounded wait that gave up) is a device error: 2 = the queries
// or the new K/V row of a KV head, 4 = the split partials of a merge, 8 = the act vector of an expert; k_layer only:
// 32 = the merged heads (device-wide), 64 = h' (device-wide), 128 = the merged heads or h' in the XCD's L2, or the
// router items.
static int ab_check(moert_model* m) {
  if (m->hybrid && m->hy_err) {
    unsigned he = 0;
    CHECK_HIP(hipMemcpy(&he, m->hy_err, 4, hipMemcpyDeviceToHost));
    if (he) {
      set_err("hybrid step: a layer's doorbell was not rung in time (error bits %#x)", he);
      return MOERT_E_DEVICE;
    }
  }
  if (!m->use_ab) return MOERT_OK;
  unsigned e = 0;
  CHECK_HIP(hipMemcpy(&e, m->ab.err, 4, hipMemcpyDeviceToHost));
  if (e) {
    set_err("%s%s%s%s%s%s%sgave up (error bits %#x): the launch's workgroups were not dispatched round-robin over the "
            "XCDs or not all resident at once",
            (e & 2u) ? "attention: the wait for queries / the new K/V row " : "",
            (e & 4u) ? "attention: the wait for split partials " : "",
            (e & 8u) ? "MoE: the wait for an expert's act vector " : "",
            (e & 16u) ? "prefetch: the wait for the layer's predicted misses " : "",
            (e & 32u) ? "layer: the wait for the merged heads " : "",
            (e & 64u) ? "layer: the wait for the post-attention residual " : "",
            (e & 128u) ? "layer: the wait for values relayed inside an XCD or for router items " : "", e);
    return MOERT_E_DEVICE;
  }
  return MOERT_OK;
}
static int model_sync(moert_model* m) {
  CHECK_HIP(hipStreamSynchronize(m->stream));
  return ab_check(m);
}

// ---- runtime metrics during moert_generate ----
// Read-back layout in the pinned buffer: the cache counters [CS_WORDS] (u64), the step state [ST_WORDS], the current
// slot-table copy, then both copies of the slot keys [2][slots].
static size_t mx_pin_bytes(const moert_model* m) {
  return 8 * CS_WORDS + 4 * (ST_WORDS + 1 + 2 * (size_t)(m->cached ? m->cache.slots : 0));
}

// Queues the read-back behind the steps launched so far; its event completes when they have.
static int mx_enqueue_read(moert_model* m) {
  unsigned char* p = m->mx_pin;
  if (m->hybrid) {
    // the placement's counters (host side, current: the host serves every layer before the next is queued);
    // word 3: the requests computed on the host
    unsigned long long* st = (unsigned long long*)p;
    const PlacementStats& s = m->place->stats();
    st[CS_HITS] = s.hits;
    st[CS_COPIES] = s.copies;
    st[CS_PREFETCH] = 0;
    st[3] = s.cpu;
  } else if (m->cached) {
    CHECK_HIP(hipMemcpyAsync(p, m->cache.stats, 8 * CS_WORDS, hipMemcpyDeviceToHost, m->stream));
    CHECK_HIP(hipMemcpyAsync(p + 8 * CS_WORDS + 4 * ST_WORDS, m->cache.cur, 4, hipMemcpyDeviceToHost, m->stream));
    CHECK_HIP(hipMemcpyAsync(p + 8 * CS_WORDS + 4 * (ST_WORDS + 1), m->cache.slot_key, 8 * (size_t)m->cache.slots,
                             hipMemcpyDeviceToHost, m->stream));
  } else {
    memset(p, 0, 8 * CS_WORDS);
  }
  CHECK_HIP(hipMemcpyAsync(p + 8 * CS_WORDS, m->b.state, 4 * ST_WORDS, hipMemcpyDeviceToHost, m->stream));
  CHECK_HIP(hipEventRecord(m->mx_ev, m->stream));
  return MOERT_OK;
}

struct MxCall {
  int pos0, n_prompt, n_new;
  uint64_t started_ms;
  moert_model::Clock::time_point t0;
};

// Fills the publisher from a completed read-back: state, context, speed and the cache fractions over the window
// since the previous read-back, totals since the counters were cleared.
static void mx_consume(moert_model* m, const MxCall& c, moert_model::Clock::time_point now) {
  const unsigned long long* st = (const unsigned long long*)m->mx_pin;
  const int* state = (const int*)(m->mx_pin + 8 * CS_WORDS);
  const int s = state[ST_POS] - c.pos0;  // steps completed
  const double dt = std::chrono::duration<double>(now - m->mx_prev_t).count();
  const int ds = s - m->mx_prev_pos;
  moert_metrics* mx = m->mx;
  const bool reading = s < c.n_prompt - 1;
  if (reading)
    (void)moert_metrics_set_state(mx, MOERT_STATE_READING, (uint64_t)s, (uint64_t)c.n_prompt, nullptr);
  else
    (void)moert_metrics_set_state(mx, MOERT_STATE_GENERATING, (uint64_t)(s - (c.n_prompt - 1)), (uint64_t)c.n_new,
                                  nullptr);
  (void)moert_metrics_set_context(mx, (uint64_t)state[ST_POS], (uint64_t)m->max_len);
  if (dt > 0 && ds > 0) {
    moert_metrics_speed sp{};
    sp.decode_now = reading ? 0.0 : ds / dt;
    sp.prefill_now = reading ? ds / dt : 0.0;
    sp.decode_last = m->mx_speed_last[0];
    sp.prefill_request = m->mx_speed_last[1];
    (void)moert_metrics_set_speed(mx, &sp);
    moert_metrics_window w{};
    w.ms_per_token = dt * 1e3 / ds;
    const double wall = std::chrono::duration<double>(now - c.t0).count();
    w.gpu_wait_frac = wall > 0 ? m->mx_wait_s / wall : 0.0;
    (void)moert_metrics_set_window(mx, &w);
  }
  moert_metrics_cache ca{};
  if (m->hybrid) {
    // requests served from the pool or on the host; copies are background admissions
    const unsigned long long dh = st[CS_HITS] - m->mx_prev[CS_HITS], dc = st[CS_COPIES] - m->mx_prev[CS_COPIES],
                             du = st[3] - m->mx_prev[3];
    const double need = (double)(dh + du);
    ca.slots_total = (uint32_t)m->place->slots();
    ca.slots_resident = (uint32_t)m->place->resident();
    ca.hit_frac = need > 0 ? dh / need : 0.0;
    ca.cpu_frac = need > 0 ? du / need : 0.0;
    ca.h2d_gbs = dt > 0 ? (double)dc * m->cache.record_bytes / dt / 1e9 : 0.0;
    ca.total_hits = st[CS_HITS];
    ca.total_copies = st[CS_COPIES];
    ca.total_cpu = st[3];
    memcpy(m->mx_prev, st, sizeof m->mx_prev);
  } else if (m->cached) {
    const int S = m->cache.slots, cur = state[ST_WORDS];
    const int* keys = state + ST_WORDS + 1 + (size_t)(cur & 1) * S;
    uint32_t res = 0;
    for (int i = 0; i < S; i++) res += keys[i] >= 0;
    const unsigned long long dh = st[CS_HITS] - m->mx_prev[CS_HITS], dc = st[CS_COPIES] - m->mx_prev[CS_COPIES],
                             dp = st[CS_PREFETCH] - m->mx_prev[CS_PREFETCH];
    const double need = (double)(dh + dc);
    ca.slots_total = (uint32_t)S;
    ca.slots_resident = res;
    ca.hit_frac = need > 0 ? dh / need : 0.0;
    ca.copy_frac = need > 0 ? dc / need : 0.0;
    ca.h2d_gbs = dt > 0 ? (double)(dc + dp) * m->cache.record_bytes / dt / 1e9 : 0.0;
    ca.total_hits = st[CS_HITS];
    ca.total_copies = st[CS_COPIES] + st[CS_PREFETCH];
    memcpy(m->mx_prev, st, sizeof m->mx_prev);
  } else {
    ca.slots_total = ca.slots_resident = (uint32_t)(m->cfg.layers * m->cfg.experts);
    ca.hit_frac = 1.0;
  }
  (void)moert_metrics_set_cache(mx, &ca);
  m->mx_prev_t = now;
  m->mx_prev_pos = s;
}

static void mx_publish(moert_model* m, moert_model::Clock::time_point now, bool force) {
  if (!force && now - m->mx_last_pub < std::chrono::milliseconds(m->mx_interval_ms)) return;
  (void)moert_metrics_publish(m->mx);  // a failed publication leaves the previous file (as the reference ignores it)
  m->mx_last_pub = now;
}

// Between step launches: consumes a completed read-back, or queues the next one once the interval has passed.
static int mx_poll(moert_model* m, const MxCall& c) {
  const auto now = moert_model::Clock::now();
  if (m->mx_pending) {
    const hipError_t q = hipEventQuery(m->mx_ev);
    if (q == hipErrorNotReady) return MOERT_OK;
    CHECK_HIP(q);
    m->mx_pending = false;
    mx_consume(m, c, now);
    mx_publish(m, now, false);
  } else if (now - m->mx_last_read >= std::chrono::milliseconds(m->mx_interval_ms)) {
    MTRY(m, mx_enqueue_read(m));
    m->mx_pending = true;
    m->mx_last_read = now;
  }
  return MOERT_OK;
}

int moert_decode_step(moert_model* m, int token, float* logits, int* route_ids, float* route_weights, int* argmax) {
  MODEL_OK(m);
  if (m->host_pos >= m->max_len) {
    set_err("KV cache full (%d positions)", m->max_len);
    return MOERT_E_FULL;
  }
  if (token < 0 || token >= m->cfg.vocab) {
    set_err("token %d outside the vocabulary (%d)", token, m->cfg.vocab);
    return MOERT_E_RANGE;
  }
  int pos = m->host_pos;
  int st[2] = {pos, pos + 1};
  MTRY(m, model_copy_in(m, m->b.seq + pos, &token, 4));
  MTRY(m, model_copy_in(m, m->b.state, st, sizeof st));
  MTRY(m, model_launch(m));
  const moert_config& c = m->cfg;
  if (logits) MTRY(m, model_copy_out(m, logits, m->b.logits, (size_t)c.vocab * 4));
  if (route_ids) MTRY(m, model_copy_out(m, route_ids, m->b.route_ids, (size_t)c.layers * c.top_k * 4));
  if (route_weights) MTRY(m, model_copy_out(m, route_weights, m->b.route_w, (size_t)c.layers * c.top_k * 4));
  int am = 0;
  MTRY(m, model_copy_out(m, &am, m->b.argmax_hist + pos, 4));
  MTRY(m, model_sync(m));
  if (argmax) *argmax = am;
  m->host_pos = pos + 1;
  return MOERT_OK;
}

int moert_step_batched(moert_model* m, const int* tokens, int n, float* logits, int* argmax) {
  MODEL_OK(m);
  CHECK_CFG(tokens && n >= 1 && n <= kPfMaxPos, "step_batched: %d positions outside [1, %d]", n, kPfMaxPos);
  CHECK_CFG(!m->cached, "step_batched: the multi-position step runs on a resident model");
  if (m->host_pos + n > m->max_len) {
    set_err("KV cache full: %d + %d positions > %d", m->host_pos, n, m->max_len);
    return MOERT_E_FULL;
  }
  for (int i = 0; i < n; i++)
    if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab) {
      set_err("token %d outside the vocabulary (%d)", tokens[i], m->cfg.vocab);
      return MOERT_E_RANGE;
    }
  MTRY(m, m->ensure_pf());
  const int pos0 = m->host_pos;
  int st[2] = {pos0 + n - 1, pos0 + n};
  MTRY(m, model_copy_in(m, m->pf.toks, tokens, (size_t)n * 4));
  MTRY(m, model_copy_in(m, m->b.seq + pos0, tokens, (size_t)n * 4));
  MTRY(m, model_copy_in(m, m->pf.pos0, &pos0, 4));
  MTRY(m, model_copy_in(m, m->b.state, st, sizeof st));
  MTRY(m, m->enqueue_batched(pos0, n));
  if (logits) MTRY(m, model_copy_out(m, logits, m->b.logits, (size_t)m->cfg.vocab * 4));
  int am = 0;
  MTRY(m, model_copy_out(m, &am, m->b.argmax_hist + pos0 + n - 1, 4));
  MTRY(m, model_sync(m));
  if (argmax) *argmax = am;
  m->host_pos = pos0 + n;
  return MOERT_OK;
}

int moert_batched_mode(moert_model* m, int mode) {
  MODEL_OK(m);
  CHECK_CFG(mode == 0 || mode == 1, "batched mode %d: 0 (per-row FMA) or 1 (grouped int8 MFMA experts)", mode);
  if (mode == 1) {
    CHECK_CFG(!m->cached, "batched mode: the multi-position step runs on a resident model");
    const moert_config& c = m->cfg;
    const int qd = c.heads * c.head_dim;
    CHECK_CFG((c.hidden == 1024 || c.hidden == 1536) && (qd == 1024 || qd == 1536) && c.head_dim == 64 &&
                  (c.inter == 128 || c.inter == 256 || c.inter == 512) && c.experts <= 64 && c.top_k <= 8,
              "grouped mode: hidden %d and heads x head_dim %d (1024 or 1536, head_dim 64), inter %d (128, 256 or 512)",
              c.hidden, qd, c.inter);
    for (const LayerDev& L : m->layers)
      CHECK_CFG(L.gate_up.dtype == DT_Q8_0 && L.down.dtype == DT_Q8_0 && L.qkv.dtype == DT_Q8_0 &&
                    L.o.dtype == DT_Q8_0 && L.router.dtype == DT_Q8_0,
                "grouped mode: Q8_0 weights only (q/k/v, output, router and experts)");
    MTRY(m, m->ensure_grouped());
  }
  m->batched_mode = mode;
  return MOERT_OK;
}

int moert_prefill(moert_model* m, const int* tokens, int n, float* logits, int* argmax) {
  MODEL_OK(m);
  // the checks of valida (rust/moe-rt/src/motor/leitura.rs:62-76), in its order, before any block runs
  CHECK_CFG(tokens && n >= 1, "prefill: %d tokens", n);
  for (int i = 0; i < n; i++)
    if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab) {
      set_err("token %d (index %d) outside the vocabulary (%d)", tokens[i], i, m->cfg.vocab);
      return MOERT_E_RANGE;
    }
  if (m->host_pos + n > m->max_len) {
    set_err("KV cache full: %d + %d positions > %d", m->host_pos, n, m->max_len);
    return MOERT_E_FULL;
  }
  for (int i = 0; i < n; i += kPfMaxPos) {
    const int nb = std::min(kPfMaxPos, n - i), last = i + nb == n;
    const int rc = moert_step_batched(m, tokens + i, nb, last ? logits : nullptr, last ? argmax : nullptr);
    if (rc) return rc;
  }
  return MOERT_OK;
}

static int generate(moert_model* m, const int* prompt, int n_prompt, int n_new, int* out_tokens, float* gaps,
                    MxCall* mc) {
  if (!prompt || n_prompt < 1 || n_new < 1 || !out_tokens) {
    set_err("generate needs a prompt of at least one token and n_new >= 1");
    return MOERT_E_CONFIG;
  }
  int pos0 = m->host_pos, steps = n_prompt + n_new - 1;
  if (pos0 + steps > m->max_len) {
    set_err("KV cache full: %d + %d steps > %d positions", pos0, steps, m->max_len);
    return MOERT_E_FULL;
  }
  for (int i = 0; i < n_prompt; i++)
    if (prompt[i] < 0 || prompt[i] >= m->cfg.vocab) {
      set_err("prompt token %d outside the vocabulary", prompt[i]);
      return MOERT_E_RANGE;
    }
  int st[2] = {pos0, pos0 + n_prompt};
  MTRY(m, model_copy_in(m, m->b.seq + pos0, prompt, (size_t)n_prompt * 4));
  MTRY(m, model_copy_in(m, m->b.state, st, sizeof st));
  if (mc) {
    mc->pos0 = pos0;
    mc->n_prompt = n_prompt;
    mc->n_new = n_new;
    m->mx_prev_pos = 0;
    m->mx_wait_s = 0;
    (void)moert_metrics_set_state(m->mx, n_prompt > 1 ? MOERT_STATE_READING : MOERT_STATE_GENERATING, 0,
                                  (uint64_t)(n_prompt > 1 ? n_prompt : n_new), nullptr);
    (void)moert_metrics_set_context(m->mx, (uint64_t)pos0, (uint64_t)m->max_len);
    mx_publish(m, moert_model::Clock::now(), true);
    CHECK_HIP(hipEventRecord(m->mx_t[0], m->stream));
    if (n_prompt == 1) CHECK_HIP(hipEventRecord(m->mx_t[1], m->stream));
  }
  std::vector<float> lg(gaps ? m->cfg.vocab : 0);
  for (int i = 0; i < steps; i++) {
    MTRY(m, model_launch(m));
    if (mc) {
      if (i == n_prompt - 2) CHECK_HIP(hipEventRecord(m->mx_t[1], m->stream));
      MTRY(m, mx_poll(m, *mc));
    }
    if (gaps && i >= n_prompt - 1) {
      MTRY(m, model_copy_out(m, lg.data(), m->b.logits, lg.size() * 4));
      const auto w0 = moert_model::Clock::now();
      MTRY(m, model_sync(m));
      m->mx_wait_s += std::chrono::duration<double>(moert_model::Clock::now() - w0).count();
      float t1 = -INFINITY, t2 = -INFINITY;
      for (float v : lg) {
        if (v > t1) {
          t2 = t1;
          t1 = v;
        } else if (v > t2) {
          t2 = v;
        }
      }
      gaps[i - (n_prompt - 1)] = t1 - t2;
    }
  }
  // token i was chosen at position pos0 + n_prompt - 1 + i (the last one is never fed back)
  MTRY(m, model_copy_out(m, out_tokens, m->b.argmax_hist + pos0 + n_prompt - 1, (size_t)n_new * 4));
  if (mc) CHECK_HIP(hipEventRecord(m->mx_t[2], m->stream));
  const auto w0 = moert_model::Clock::now();
  MTRY(m, model_sync(m));
  m->mx_wait_s += std::chrono::duration<double>(moert_model::Clock::now() - w0).count();
  m->host_pos = pos0 + steps;
  return MOERT_OK;
}

int moert_generate(moert_model* m, const int* prompt, int n_prompt, int n_new, int* out_tokens, float* gaps) {
  MODEL_OK(m);
  if (!m->mx) return generate(m, prompt, n_prompt, n_new, out_tokens, gaps, nullptr);
  // with a metrics publisher: state and counters while the steps run, then the request entry (Request,
  // rust/moe-monitor/src/snapshot.rs:121-135), an event and a forced publication
  MxCall mc{0, n_prompt, n_new, 0, moert_model::Clock::now()};
  mc.started_ms = (uint64_t)std::chrono::duration_cast<std::chrono::milliseconds>(
                      std::chrono::system_clock::now().time_since_epoch())
                      .count();
  m->mx_prev_t = mc.t0;
  const int rc = generate(m, prompt, n_prompt, n_new, out_tokens, gaps, &mc);
  const auto now = moert_model::Clock::now();
  const double wall = std::chrono::duration<double>(now - mc.t0).count();
  moert_metrics_request r{};
  r.started_ms = mc.started_ms;
  r.prompt_tokens = (uint64_t)(n_prompt > 0 ? n_prompt : 0);
  r.duration_ms = (uint64_t)(wall * 1e3);
  char msg[320];
  if (rc != MOERT_OK) {
    // the message of the failure (the model may be poisoned: nothing more is read from the device)
    snprintf(msg, sizeof msg, "generate: %s", moert_last_error());
    (void)moert_metrics_set_state(m->mx, MOERT_STATE_ERROR, 0, 0, msg);
    r.status = "erro";
    (void)moert_metrics_add_request(m->mx, &r);
    (void)moert_metrics_event(m->mx, "erro", msg);
    m->mx_pending = false;
    mx_publish(m, now, true);
    return rc;
  }
  // the final read-back (after the stream has drained), and the phase times from the timing marks
  int rc2 = mx_enqueue_read(m);
  if (rc2 == MOERT_OK) rc2 = model_sync(m);
  if (rc2 != MOERT_OK) return m->fail(rc2);
  m->mx_pending = false;
  mx_consume(m, mc, now);
  float pre_ms = 0, dec_ms = 0;
  CHECK_HIP(hipEventElapsedTime(&pre_ms, m->mx_t[0], m->mx_t[1]));
  CHECK_HIP(hipEventElapsedTime(&dec_ms, m->mx_t[1], m->mx_t[2]));
  r.output_tokens = (uint64_t)n_new;
  r.prefill_tok_s = n_prompt > 1 && pre_ms > 0 ? (n_prompt - 1) / (pre_ms * 1e-3) : 0.0;
  r.decode_tok_s = dec_ms > 0 ? n_new / (dec_ms * 1e-3) : 0.0;
  r.status = "ok";
  m->mx_speed_last[0] = r.decode_tok_s;
  m->mx_speed_last[1] = r.prefill_tok_s;
  moert_metrics_speed sp{};
  sp.decode_last = r.decode_tok_s;
  sp.prefill_request = r.prefill_tok_s;
  (void)moert_metrics_set_speed(m->mx, &sp);
  moert_metrics_window w{};
  w.ms_per_token = n_new > 0 ? dec_ms / n_new : 0.0;
  w.gpu_wait_frac = wall > 0 ? m->mx_wait_s / wall : 0.0;
  (void)moert_metrics_set_window(m->mx, &w);
  (void)moert_metrics_set_state(m->mx, MOERT_STATE_IDLE, 0, 0, nullptr);
  (void)moert_metrics_add_request(m->mx, &r);
  snprintf(msg, sizeof msg, "generate: %d prompt tokens, %d new tokens, %.1f tok/s decode, %.1f tok/s prompt",
           n_prompt, n_new, r.decode_tok_s, r.prefill_tok_s);
  (void)moert_metrics_event(m->mx, "info", msg);
  mx_publish(m, now, true);
  return MOERT_OK;
}

int moert_model_attach_metrics(moert_model* m, moert_metrics* mx, int min_interval_ms) {
  MODEL_OK(m);
  CHECK_CFG(min_interval_ms >= 0, "metrics interval %d ms", min_interval_ms);
  CHECK_HIP(hipStreamSynchronize(m->stream));
  m->mx = nullptr;
  m->mx_pending = false;
  if (!mx) return MOERT_OK;
  if (!m->mx_pin) {
    CHECK_HIP(hipHostMalloc((void**)&m->mx_pin, mx_pin_bytes(m), hipHostMallocDefault));
    CHECK_HIP(hipEventCreateWithFlags(&m->mx_ev, hipEventDisableTiming));
    for (hipEvent_t& e : m->mx_t) CHECK_HIP(hipEventCreate(&e));
  }
  m->mx = mx;
  m->mx_interval_ms = min_interval_ms;
  char buf[96];
  (void)moert_metrics_set_model(mx, "granite-moe", m->cfg.layers, m->cfg.experts, m->cfg.top_k);
  snprintf(buf, sizeof buf, "%d", m->max_len);
  (void)moert_metrics_setting(mx, "positions", buf);
  snprintf(buf, sizeof buf, "%d", m->splits);
  (void)moert_metrics_setting(mx, "attention splits", buf);
  if (m->cached)
    snprintf(buf, sizeof buf, "%d of %d", m->cache.slots, m->cfg.layers * m->cfg.experts);
  else
    snprintf(buf, sizeof buf, "all %d resident", m->cfg.layers * m->cfg.experts);
  (void)moert_metrics_setting(mx, "expert pool slots", buf);
  // the counters as they stand now, as the base of the first window
  MTRY(m, mx_enqueue_read(m));
  MTRY(m, model_sync(m));
  memcpy(m->mx_prev, m->mx_pin, sizeof m->mx_prev);
  MxCall mc{m->host_pos, 1, 0, 0, moert_model::Clock::now()};
  m->mx_prev_pos = 0;
  m->mx_prev_t = mc.t0;
  mx_consume(m, mc, mc.t0);
  (void)moert_metrics_set_state(mx, MOERT_STATE_IDLE, 0, 0, nullptr);
  m->mx_last_pub = mc.t0;
  m->mx_last_read = mc.t0;
  return moert_metrics_publish(mx);
}

int moert_reset_sequence(moert_model* m) {
  MODEL_OK(m);
  MTRY(m, m->write_state(0, 0));
  return MOERT_OK;
}

int moert_set_position(moert_model* m, int pos) {
  MODEL_OK(m);
  if (pos < 0 || pos >= m->max_len) {
    set_err("position %d outside [0, %d)", pos, m->max_len);
    return MOERT_E_RANGE;
  }
  MTRY(m, m->write_state(pos, 0));
  return MOERT_OK;
}

int moert_get_position(moert_model* m, int* pos) {
  MODEL_OK(m);
  if (pos) *pos = m->host_pos;
  return MOERT_OK;
}

int moert_kv_prefill_fp16(moert_model* m, int layer, const uint16_t* k, const uint16_t* v, int n) {
  MODEL_OK(m);
  const moert_config& c = m->cfg;
  if (layer < 0 || layer >= c.layers || n < 0 || n > m->max_len || !k || !v) {
    set_err("kv prefill: layer %d, n %d", layer, n);
    return MOERT_E_RANGE;
  }
  const LayerDev& L = m->layers[layer];
  for (int g = 0; g < c.kv_heads; g++) {
    size_t src = (size_t)g * n * 64, dst = (size_t)g * m->max_len * 64;
    MTRY(m, model_copy_in(m, L.k_cache + dst, k + src, (size_t)n * 64 * 2));
    MTRY(m, model_copy_in(m, L.v_cache + dst, v + src, (size_t)n * 64 * 2));
  }
  MTRY(m, model_sync(m));
  return MOERT_OK;
}

int moert_read_kv_fp16(moert_model* m, int layer, uint16_t* k, uint16_t* v, int n) {
  MODEL_OK(m);
  const moert_config& c = m->cfg;
  if (layer < 0 || layer >= c.layers || n < 0 || n > m->max_len || !k || !v) {
    set_err("read kv: layer %d, n %d", layer, n);
    return MOERT_E_RANGE;
  }
  const LayerDev& L = m->layers[layer];
  for (int g = 0; g < c.kv_heads; g++) {
    size_t dst = (size_t)g * n * 64, src = (size_t)g * m->max_len * 64;
    MTRY(m, model_copy_out(m, k + dst, L.k_cache + src, (size_t)n * 64 * 2));
    MTRY(m, model_copy_out(m, v + dst, L.v_cache + src, (size_t)n * 64 * 2));
  }
  MTRY(m, model_sync(m));
  return MOERT_OK;
}

int moert_read_hidden(moert_model* m, float* h) {
  MODEL_OK(m);
  MTRY(m, model_copy_out(m, h, m->b.h, (size_t)m->cfg.hidden * 4));
  MTRY(m, model_sync(m));
  return MOERT_OK;
}

int moert_read_logits(moert_model* m, float* logits) {
  MODEL_OK(m);
  CHECK_CFG(logits, "null output");
  MTRY(m, model_copy_out(m, logits, m->b.logits, (size_t)m->cfg.vocab * 4));
  MTRY(m, model_sync(m));
  return MOERT_OK;
}

// One graph replay of the decode step with every workgroup of every launch stamping its phases (timeline build).
// out: [launches][1024][8] u64 records (see timeline.h); kinds / layers: [launches]. The first call rebuilds the step
// graph with the records attached.
int moert_timeline_step(moert_model* m, unsigned long long* out, int* kinds, int* layers, int max_launches,
                        int* n_launches) {
  MODEL_OK(m);
  CHECK_CFG(!m->hybrid, "the hybrid model steps from the host, layer by layer: no per-kernel timing");
#ifndef MOERT_TIMELINE
  (void)out; (void)kinds; (void)layers; (void)max_launches; (void)n_launches;
  set_err("timeline: this library was built without MOERT_TIMELINE (use libmoert_tl.so)");
  return MOERT_E_CONFIG;
#else
  CHECK_CFG(out && kinds && layers && n_launches, "null argument");
  if (m->host_pos >= m->max_len) {
    set_err("KV cache full (%d positions)", m->max_len);
    return MOERT_E_FULL;
  }
  if (!m->tl_buf) {
    const size_t launches = 3 + 6 * m->layers.size();
    CHECK_HIP(hipMalloc(&m->tl_buf, launches * moert_model::kTlRecord * 8));
    m->tl_launches = launches;
    CHECK_HIP(hipStreamSynchronize(m->stream));
    if (m->exec) CHECK_HIP(hipGraphExecDestroy(m->exec));
    if (m->graph) CHECK_HIP(hipGraphDestroy(m->graph));
    m->exec = nullptr;
    m->graph = nullptr;
    MTRY(m, m->build_graph());
  }
  const size_t n = m->tl_kind.size();
  CHECK_CFG((int)n <= max_launches, "timeline: %zu launches, room for %d", n, max_launches);
  int st[2] = {m->host_pos, 0};
  MTRY(m, model_copy_in(m, m->b.state, st, sizeof st));
  CHECK_HIP(hipMemsetAsync(m->tl_buf, 0, n * moert_model::kTlRecord * 8, m->stream));
  MTRY(m, model_launch(m));
  MTRY(m, model_copy_out(m, out, m->tl_buf, n * moert_model::kTlRecord * 8));
  MTRY(m, model_sync(m));
  for (size_t i = 0; i < n; i++) {
    kinds[i] = m->tl_kind[i];
    layers[i] = m->tl_layer[i];
  }
  *n_launches = (int)n;
  m->host_pos++;
  return MOERT_OK;
#endif
}

static int time_steps_impl(moert_model* m, int warmup, int iters, double* ms) {
  hipEvent_t e0, e1;
  CHECK_HIP(hipEventCreate(&e0));
  CHECK_HIP(hipEventCreate(&e1));
  for (int i = 0; i < warmup; i++) TRY(model_launch(m));
  CHECK_HIP(hipEventRecord(e0, m->stream));
  for (int i = 0; i < iters; i++) TRY(model_launch(m));
  CHECK_HIP(hipEventRecord(e1, m->stream));
  CHECK_HIP(hipEventSynchronize(e1));
  TRY(ab_check(m));
  float t = 0.0f;
  CHECK_HIP(hipEventElapsedTime(&t, e0, e1));
  *ms = iters > 0 ? t / iters : 0.0;
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  m->host_pos += warmup + iters;
  return MOERT_OK;
}

int moert_time_steps(moert_model* m, int warmup, int iters, double* ms_per_step) {
  MODEL_OK(m);
  if (warmup < 0 || iters < 0 || m->host_pos + warmup + iters > m->max_len) {
    set_err("time_steps: %d + %d + %d positions exceed max_len %d", m->host_pos, warmup, iters, m->max_len);
    return MOERT_E_FULL;
  }
  int st[2] = {m->host_pos, 0};
  MTRY(m, model_copy_in(m, m->b.state, st, sizeof st));
  MTRY(m, time_steps_impl(m, warmup, iters, ms_per_step));
  return MOERT_OK;
}

static int time_kernel_impl(moert_model* m, int kind, int iters, double* us, int* launches) {
  // at most one launch of a class per layer; a class the step does not launch gives no launches
  std::vector<hipEvent_t> ev(2 * (size_t)m->cfg.layers + 2);
  for (auto& e : ev) CHECK_HIP(hipEventCreate(&e));
  double total = 0.0;
  int n = 0;
  for (int it = 0; it < iters; it++) {
    TRY(epoch_guard(m));
    TRY(m->enqueue(kind, &ev));
    const int per_step = m->ev_i / 2;
    CHECK_HIP(hipStreamSynchronize(m->stream));
    TRY(ab_check(m));
    for (int i = 0; i < per_step; i++) {
      float t = 0.0f;
      CHECK_HIP(hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]));
      total += t;
      n++;
    }
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  *us = n ? total * 1000.0 / n : 0.0;
  if (launches) *launches = n;
  m->host_pos += iters;
  return MOERT_OK;
}

int moert_model_path(const moert_model* m, int* layer, int* attn_block, int* moe_xcd) {
  if (!m || !layer || !attn_block || !moe_xcd) {
    set_err("model_path: null argument");
    return MOERT_E_CONFIG;
  }
  const bool blk = m->use_ab && !(m->cached && m->prefetch && !m->pf_blk);
  *layer = m->use_px ? 1 : 0;
  *attn_block = blk && !m->use_px ? 1 : 0;
  *moe_xcd = blk && m->use_mx && !m->use_px ? 1 : 0;
  return MOERT_OK;
}

int moert_fault_inject(moert_model* m, unsigned bits) {
  MODEL_OK(m);
  CHECK_CFG((bits & ~30u) == 0, "fault_inject: bits %#x outside 2 | 4 | 8 | 16", bits);
  if (bits & 16u) {
    // the prefetch's copy wait alone: the decision before it ran normally, so the slot tables stay consistent;
    // the step that fails reports and poisons the handle before any later step reads the uncopied slots
    CHECK_CFG(bits == 16u && m->cached && m->prefetch && m->pf_blk,
              "fault_inject: bit 16 (alone) needs a cached model with the prefetch inside the attention launch");
  } else {
    // resident models only: there every index a failed launch leaves behind (token, routed expert) is still in
    // range, while the expert cache would take slot-table decisions from the garbage values of a failed launch
    CHECK_CFG(m->use_ab && !m->hybrid && !m->cached, "fault_inject: a resident model with the fused kernels only");
  }
  CHECK_CFG(bits == 0 || (bits & 8u) == 0 || m->use_mx, "fault_inject: bit 8 needs the MoE kernel spread over the XCDs");
  MTRY(m, model_sync(m));
  MTRY(m, model_copy_in(m, m->ab.err + 1, &bits, 4));
  return m->fail(model_sync(m));
}

int moert_time_kernel(moert_model* m, int kind, int iters, double* us_per_launch, int* launches) {
  MODEL_OK(m);
  CHECK_CFG(!m->hybrid, "the hybrid model steps from the host, layer by layer: no per-kernel timing");
  if (kind < 0 || kind >= MOERT_K_COUNT || iters < 1 || !us_per_launch) {
    set_err("time_kernel: kind %d, iters %d", kind, iters);
    return MOERT_E_CONFIG;
  }
  if (m->host_pos + iters > m->max_len) {
    set_err("time_kernel: %d + %d positions exceed max_len %d", m->host_pos, iters, m->max_len);
    return MOERT_E_FULL;
  }
  int st[2] = {m->host_pos, 0};
  MTRY(m, model_copy_in(m, m->b.state, st, sizeof st));
  MTRY(m, time_kernel_impl(m, kind, iters, us_per_launch, launches));
  return MOERT_OK;
}

int moert_cache_stats(moert_model* m, unsigned long long* hits, unsigned long long* copies) {
  MODEL_OK(m);
  CHECK_CFG(m->cached, "model has no expert cache");
  if (m->hybrid) {
    if (hits) *hits = m->place->stats().hits;
    if (copies) *copies = m->place->stats().copies;
    return MOERT_OK;
  }
  unsigned long long st[CS_WORDS];
  MTRY(m, model_copy_out(m, st, m->cache.stats, sizeof st));
  MTRY(m, model_sync(m));
  if (hits) *hits = st[CS_HITS];
  if (copies) *copies = st[CS_COPIES];
  return MOERT_OK;
}

int moert_cache_clear(moert_model* m) {
  MODEL_OK(m);
  CHECK_CFG(m->cached, "model has no expert cache");
  if (m->hybrid) {
    // an empty pool, a fresh frequency and zero counters (the pool's contents are never read without a table entry)
    MTRY(m, model_sync(m));
    const Placement& P = *m->place;
    m->place.reset(new Placement(m->cfg.layers, m->cfg.experts, m->cfg.top_k, P.slots(), m->place->backlog()));
    m->place->start();
    std::fill(m->hy_tok.begin(), m->hy_tok.end(), 0);
    return MOERT_OK;
  }
  MTRY(m, m->cache_clear());
  return MOERT_OK;
}

int moert_cache_prefetch_mode(moert_model* m, int on) {
  MODEL_OK(m);
  CHECK_CFG(m->cached, "model has no expert cache");
  CHECK_CFG(!m->hybrid, "prefetch mode: the hybrid model's copies are decided by its placement");
  CHECK_CFG(on == 0 || on == 1, "prefetch mode %d: 0 (off) or 1 (each layer's experts predicted from its input)", on);
  if ((on != 0) == m->prefetch) return MOERT_OK;
  if (!m->pf_stream) {
    CHECK_HIP(hipStreamCreateWithFlags(&m->pf_stream, hipStreamNonBlocking));
    for (hipEvent_t* e : {&m->ev_fork, &m->ev_pred, &m->ev_copy})
      CHECK_HIP(hipEventCreateWithFlags(e, hipEventDisableTiming));
  }
  CHECK_HIP(hipStreamSynchronize(m->stream));
  CHECK_HIP(hipStreamSynchronize(m->pf_stream));
  if (m->exec) CHECK_HIP(hipGraphExecDestroy(m->exec));
  if (m->graph) CHECK_HIP(hipGraphDestroy(m->graph));
  m->exec = nullptr;
  m->graph = nullptr;
  m->prefetch = on != 0;
  // inside the attention launch when the block and every layer fit (MOERT_PF_BLOCK=0: the side branch)
  const char* pv = std::getenv("MOERT_PF_BLOCK");
  bool fits = m->prefetch && m->use_ab && !(pv && pv[0] == '0');
  for (size_t l = 0; fits && l < m->layers.size(); l++)
    fits = attn_block_fits(m->dims, m->layers[l].qkv, m->cus) &&
           attn_block_prefetch_fits(m->dims, m->layers[l], m->cache);
  m->pf_blk = fits;
  MTRY(m, m->build_graph());
  return MOERT_OK;
}

int moert_cache_predictions(moert_model* m, int pos0, int n, int* ids) {
  MODEL_OK(m);
  CHECK_CFG(m->cached && !m->hybrid, "model has no expert cache with a prefetch branch");
  CHECK_CFG(ids && pos0 >= 0 && n >= 0 && pos0 + n <= m->max_len, "predictions: positions [%d, %d)", pos0, pos0 + n);
  const size_t row = (size_t)m->cfg.layers * 8;
  MTRY(m, model_copy_out(m, ids, m->cache.pred_hist + (size_t)pos0 * row, (size_t)n * row * 4));
  MTRY(m, model_sync(m));
  return MOERT_OK;
}

int moert_cache_token_counts(moert_model* m, int pos0, int n, int* counts) {
  MODEL_OK(m);
  CHECK_CFG(m->cached, "model has no expert cache");
  CHECK_CFG(counts && pos0 >= 0 && n >= 0 && pos0 + n <= m->max_len, "token counts: positions [%d, %d)", pos0,
            pos0 + n);
  const size_t row = (size_t)m->cfg.layers * 4;
  if (m->hybrid) {
    MTRY(m, model_sync(m));
    std::memcpy(counts, m->hy_tok.data() + (size_t)pos0 * row, (size_t)n * row * 4);
    return MOERT_OK;
  }
  MTRY(m, model_copy_out(m, counts, m->cache.tok_hist + (size_t)pos0 * row, (size_t)n * row * 4));
  MTRY(m, model_sync(m));
  return MOERT_OK;
}

int moert_cache_counters_get(moert_model* m, moert_cache_counters* out) {
  MODEL_OK(m);
  CHECK_CFG(m->cached && out, "model has no expert cache (or null output)");
  if (m->hybrid) {
    MTRY(m, model_sync(m));
    const PlacementStats& s = m->place->stats();
    moert_cache_counters c{};
    c.needed = s.needed;
    c.hits = s.hits;
    c.cpu = s.cpu;
    c.copies = s.copies;
    c.dropped = s.dropped;
    c.deferred = s.deferred;
    c.bytes_copied = s.copies * (unsigned long long)m->cache.record_bytes;
    c.slots = m->place->slots();
    *out = c;
    return MOERT_OK;
  }
  unsigned long long st[CS_WORDS];
  MTRY(m, model_copy_out(m, st, m->cache.stats, sizeof st));
  MTRY(m, model_sync(m));
  moert_cache_counters c{};
  c.hits = st[CS_HITS];
  c.copies = st[CS_COPIES];
  c.prefetched = st[CS_PREFETCH];
  c.needed = c.hits + c.copies;
  c.bytes_copied = (c.copies + c.prefetched) * (unsigned long long)m->cache.record_bytes;
  c.slots = m->cache.slots;
  *out = c;
  return MOERT_OK;
}

int moert_cache_fill(moert_model* m, int* copied) {
  MODEL_OK(m);
  CHECK_CFG(m->cached && !m->hybrid, "model has no expert cache with device-side placement");
  std::vector<int> keys((size_t)m->cfg.layers * m->cfg.experts);
  for (size_t i = 0; i < keys.size(); i++) keys[i] = (int)i;
  MTRY(m, m->cache_load(keys.data(), (int)keys.size(), false, copied));
  return MOERT_OK;
}

int moert_cache_prefetch(moert_model* m, int layer, const int* experts, int n, int* copied) {
  MODEL_OK(m);
  CHECK_CFG(m->cached && !m->hybrid, "model has no expert cache with device-side placement");
  CHECK_CFG(layer >= 0 && layer < m->cfg.layers, "layer %d outside [0, %d)", layer, m->cfg.layers);
  CHECK_CFG(experts && n >= 1 && n <= m->cache.slots && n <= m->cfg.experts,
            "prefetch of %d experts: between 1 and min(slots %d, experts %d)", n, m->cache.slots, m->cfg.experts);
  std::vector<int> keys(n);
  for (int j = 0; j < n; j++) {
    CHECK_CFG(experts[j] >= 0 && experts[j] < m->cfg.experts, "expert %d outside [0, %d)", experts[j],
              m->cfg.experts);
    for (int i = 0; i < j; i++) CHECK_CFG(experts[i] != experts[j], "expert %d requested twice", experts[j]);
    keys[j] = layer * m->cfg.experts + experts[j];
  }
  MTRY(m, m->cache_load(keys.data(), n, true, copied));
  return MOERT_OK;
}

// ---- MoE block ----------------------------------------------------------------------------------------------
int moert_block_create(int hidden, int inter, int experts, int top_k, const moert_tensor* router,
                       const float* router_bias, const moert_tensor* gate_up, const moert_tensor* down,
                       moert_block** out) {
  CHECK_CFG(out && router && gate_up && down, "null argument");
  *out = nullptr;
  CHECK_CFG(k_supported(hidden) && (inter == 128 || inter == 256 || inter == 512), "hidden %d / inter %d", hidden, inter);
  CHECK_CFG(experts >= 1 && experts <= 64 && top_k >= 1 && top_k <= 8 && top_k <= experts, "experts %d, top_k %d",
            experts, top_k);
  CHECK_CFG(router->dtype == gate_up->dtype, "router and gate_up must share a dtype");
  moert_block* b = new moert_block;
  auto bail = [&](int rc) {
    delete b;
    return rc;
  };
  if (hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking) != hipSuccess) {
    set_err("hipStreamCreate failed");
    return bail(MOERT_E_DEVICE);
  }
  b->dims = Dims{hidden, inter, 1, 1, 64, hidden, experts, top_k, 64, 1, 0.0f, 1.0f, 1.0f, 1.0f, 1.0f};
  hipStream_t s = b->stream;
  Arena& a = b->arena;
  int rc;
  if ((rc = upload_matrix(a, s, {{router->data, experts}}, router->dtype, hidden, &b->L.router))) return bail(rc);
  if ((rc = upload_matrix(a, s, {{gate_up->data, experts * 2 * inter}}, gate_up->dtype, hidden, &b->L.gate_up))) return bail(rc);
  if ((rc = upload_matrix(a, s, {{down->data, experts * hidden}}, down->dtype, inter, &b->L.down))) return bail(rc);
  float* tmp;
  b->L.router_bias = nullptr;
  if (router_bias) {
    if ((rc = upload_f32(a, s, router_bias, experts, &tmp))) return bail(rc);
    b->L.router_bias = tmp;
  }
  if ((rc = zeros(a, s, hidden, &b->x)) ||
      (rc = zeros(a, s, (size_t)top_k * inter, &b->b.act)) || (rc = zeros(a, s, top_k, &b->b.route_ids)) ||
      (rc = zeros(a, s, top_k, &b->b.route_w)) || (rc = zeros(a, s, hidden, &b->b.logits)))
    return bail(rc);
  b->b.h = b->x;
  if (hipStreamSynchronize(s) != hipSuccess) {
    set_err("block upload failed");
    return bail(MOERT_E_DEVICE);
  }
  *out = b;
  return MOERT_OK;
}

int moert_block_destroy(moert_block* b) {
  delete b;
  return MOERT_OK;
}

int moert_block_forward(moert_block* b, const float* x, float* y, int* ids, float* weights) {
  CHECK_CFG(b && x, "null argument");
  const Dims& d = b->dims;
  CHECK_HIP(hipMemcpyAsync(b->x, x, (size_t)d.hidden * 4, hipMemcpyHostToDevice, b->stream));
  TRY(b->enqueue());
  if (y) CHECK_HIP(hipMemcpyAsync(y, b->b.logits, (size_t)d.hidden * 4, hipMemcpyDeviceToHost, b->stream));
  if (ids) CHECK_HIP(hipMemcpyAsync(ids, b->b.route_ids, (size_t)d.top_k * 4, hipMemcpyDeviceToHost, b->stream));
  if (weights) CHECK_HIP(hipMemcpyAsync(weights, b->b.route_w, (size_t)d.top_k * 4, hipMemcpyDeviceToHost, b->stream));
  CHECK_HIP(hipStreamSynchronize(b->stream));
  return MOERT_OK;
}

int moert_block_time(moert_block* b, int iters, double* us) {
  CHECK_CFG(b && us && iters > 0, "bad argument");
  hipEvent_t e0, e1;
  CHECK_HIP(hipEventCreate(&e0));
  CHECK_HIP(hipEventCreate(&e1));
  TRY(b->enqueue());
  CHECK_HIP(hipEventRecord(e0, b->stream));
  for (int i = 0; i < iters; i++) TRY(b->enqueue());
  CHECK_HIP(hipEventRecord(e1, b->stream));
  CHECK_HIP(hipEventSynchronize(e1));
  float t = 0;
  CHECK_HIP(hipEventElapsedTime(&t, e0, e1));
  *us = (double)t * 1000.0 / iters;
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return MOERT_OK;
}

static int check_grouped(moert_block* b, int m) {
  CHECK_CFG(m >= 1 && m <= kGrpMaxPos, "batched step: m %d outside [1, %d]", m, kGrpMaxPos);
  CHECK_CFG(b->L.router.dtype == MOERT_Q8_0 && b->L.gate_up.dtype == MOERT_Q8_0 && b->L.down.dtype == MOERT_Q8_0,
            "batched step: the grouped MFMA path takes Q8_0 router and experts");
  CHECK_CFG(b->dims.hidden % 256 == 0 && (b->dims.hidden == 1024 || b->dims.hidden == 1536),
            "batched step: hidden %d not compiled", b->dims.hidden);
  return b->ensure_grouped();
}

int moert_block_forward_batched(moert_block* b, int m, const float* x, float* y, int* ids, float* weights) {
  CHECK_CFG(b && x, "null argument");
  TRY(check_grouped(b, m));
  const Dims& d = b->dims;
  CHECK_CFG(!b->fused || m <= kFbPos, "batched step: the one-launch kernel takes at most %d positions", kFbPos);
  CHECK_HIP(hipMemcpyAsync(b->gx, x, (size_t)m * d.hidden * 4, hipMemcpyHostToDevice, b->stream));
  TRY(b->launch_batched(b->stream, m, nullptr));
  if (y) CHECK_HIP(hipMemcpyAsync(y, b->gy, (size_t)m * d.hidden * 4, hipMemcpyDeviceToHost, b->stream));
  if (ids) CHECK_HIP(hipMemcpyAsync(ids, b->g.ids, (size_t)m * d.top_k * 4, hipMemcpyDeviceToHost, b->stream));
  if (weights) CHECK_HIP(hipMemcpyAsync(weights, b->g.w, (size_t)m * d.top_k * 4, hipMemcpyDeviceToHost, b->stream));
  CHECK_HIP(hipStreamSynchronize(b->stream));
  return b->fused_check();
}

int moert_block_batched_kernel(moert_block* b, int mode) {
  CHECK_CFG(b && (mode == 0 || mode == 1), "batched kernel mode %d (0: four kernels, 1: one launch)", mode);
  if (mode == 1) {
    CHECK_CFG(b->L.router.dtype == MOERT_Q8_0 && b->L.gate_up.dtype == MOERT_Q8_0 && b->L.down.dtype == MOERT_Q8_0,
              "one-launch batched step: Q8_0 router and experts");
    CHECK_CFG(b->dims.inter == kFbInter && b->dims.experts <= kFbExperts && b->dims.top_k <= 8,
              "one-launch batched step: ffn %d (needs %d), %d experts (at most %d)", b->dims.inter, kFbInter,
              b->dims.experts, kFbExperts);
    if (!b->cus) {
      int dev = 0, n = 0;
      CHECK_HIP(hipGetDevice(&dev));
      CHECK_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
      b->cus = n;
    }
    CHECK_CFG(b->cus == 256, "one-launch batched step: needs 256 compute units (this device has %d)", b->cus);
    TRY(check_grouped(b, 1));
    TRY(b->ensure_fused());
  }
  b->fused = mode;
  return MOERT_OK;
}

int moert_block_fault_inject(moert_block* b, unsigned bits) {
  CHECK_CFG(b, "null argument");
  CHECK_CFG((bits & ~15u) == 0, "block fault_inject: bits %#x outside 1 | 2 | 4 | 8", bits);
  CHECK_CFG(b->fused && b->fb.err, "block fault_inject: the block runs its batched steps as one launch only");
  CHECK_HIP(hipStreamSynchronize(b->stream));
  CHECK_HIP(hipMemcpy(b->fb.err + 1, &bits, 4, hipMemcpyHostToDevice));
  return MOERT_OK;
}

int moert_block_experts_in_step(moert_block* b, int* n_experts) {
  CHECK_CFG(b && n_experts && b->gx, "no batched step has run on this block");
  int nu = 0;
  CHECK_HIP(hipMemcpy(&nu, b->g.grp + GRP_NU, 4, hipMemcpyDeviceToHost));
  *n_experts = nu;
  return MOERT_OK;
}

int moert_block_time_batched(moert_block* const* blocks, int nblocks, int m, int iters, double* us) {
  CHECK_CFG(blocks && nblocks >= 1 && iters >= 1 && us, "bad argument");
  for (int i = 0; i < nblocks; i++) {
    CHECK_CFG(blocks[i] && blocks[i]->gx, "block %d: run moert_block_forward_batched first", i);
    TRY(check_grouped(blocks[i], m));
  }
  hipStream_t s = blocks[0]->stream;
  for (int i = 1; i < nblocks; i++) CHECK_HIP(hipStreamSynchronize(blocks[i]->stream));
  const int n = iters * nblocks;
  std::vector<hipEvent_t> ev(8 * n + 2);
  for (auto& e : ev) CHECK_HIP(hipEventCreate(&e));
  auto run = [&](bool per_kernel) -> int {
    for (int it = 0; it < iters; it++)
      for (int i = 0; i < nblocks; i++) {
        moert_block* b = blocks[i];
        const hipEvent_t* e = per_kernel ? &ev[8 * (it * nblocks + i)] : nullptr;
        CHECK_CFG(!b->fused || m <= kFbPos, "time_batched: the one-launch kernel takes at most %d positions", kFbPos);
        TRY(b->launch_batched(s, m, e));
      }
    return MOERT_OK;
  };
  int rc = run(false);  // warm-up
  if (!rc) rc = hipEventRecord(ev[8 * n], s) == hipSuccess ? run(false) : MOERT_E_DEVICE;
  if (!rc) rc = hipEventRecord(ev[8 * n + 1], s) == hipSuccess ? run(true) : MOERT_E_DEVICE;
  if (!rc && hipStreamSynchronize(s) != hipSuccess) rc = MOERT_E_DEVICE;
  if (!rc) {
    float t = 0.0f;
    (void)hipEventElapsedTime(&t, ev[8 * n], ev[8 * n + 1]);
    us[0] = (double)t * 1000.0 / n;
    for (int k = 0; k < 4; k++) {
      double tot = 0.0;
      for (int i = 0; i < n; i++) {
        float x = 0.0f;
        // a one-launch step records only its first pair
        if (k == 0 || !blocks[i % nblocks]->fused) (void)hipEventElapsedTime(&x, ev[8 * i + 2 * k], ev[8 * i + 2 * k + 1]);
        tot += x;
      }
      us[1 + k] = tot * 1000.0 / n;
    }
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  if (rc == MOERT_E_DEVICE && g_err.empty()) set_err("time_batched: device error");
  for (int i = 0; i < nblocks && !rc; i++) rc = blocks[i]->fused_check();
  return rc;
}

// ---- unit-parity entry points ---------------------------------------------------------------------------------
int moert_router_topk(const float* logits, int n, int k, int* ids, float* weights) {
  CHECK_CFG(logits && ids && weights && n >= 1 && n <= 64 && k >= 1 && k <= n, "router_topk: n %d, k %d", n, k);
  Scoped sc;
  TRY(sc.init());
  float *dl, *dw;
  int* di;
  TRY(sc.dev(&dl, n, logits));
  TRY(sc.dev(&di, k));
  TRY(sc.dev(&dw, k));
  CHECK_HIP(launch_topk(sc.s, dl, nullptr, n, k, di, dw));
  TRY(sc.get(ids, di, (size_t)k * 4));
  TRY(sc.get(weights, dw, (size_t)k * 4));
  return MOERT_OK;
}

int moert_argmax(const float* v, int n, int* idx) {
  CHECK_CFG(v && idx && n >= 1, "argmax: n %d", n);
  Scoped sc;
  TRY(sc.init());
  float* dv;
  int2* best;
  int *cnt, *out;
  TRY(sc.dev(&dv, n, v));
  TRY(sc.dev(&best, 1024));
  TRY(sc.dev(&cnt, 1));
  TRY(sc.dev(&out, 1));
  CHECK_HIP(launch_argmax(sc.s, dv, n, best, cnt, out));
  TRY(sc.get(idx, out, 4));
  return MOERT_OK;
}

int moert_gemv(const moert_tensor* w, int rows, int cols, const float* x, float* y) {
  CHECK_CFG(w && x && y && rows >= 1 && k_supported(cols), "gemv: rows %d, cols %d", rows, cols);
  Scoped sc;
  TRY(sc.init());
  DMat m;
  TRY(unit_matrix(sc, w, rows, cols, &m));
  float *dx, *dy;
  TRY(sc.dev(&dx, cols, x));
  TRY(sc.dev(&dy, rows));
  CHECK_HIP(launch_gemv(sc.s, m, dx, dy));
  TRY(sc.get(y, dy, (size_t)rows * 4));
  return MOERT_OK;
}

int moert_dequant(const moert_tensor* w, int rows, int cols, float* out) {
  CHECK_CFG(w && out && rows >= 1 && cols >= 32 && cols % 32 == 0, "dequant: rows %d, cols %d", rows, cols);
  Scoped sc;
  TRY(sc.init());
  DMat m;
  TRY(unit_matrix(sc, w, rows, cols, &m));
  float* d;
  TRY(sc.dev(&d, (size_t)rows * cols));
  CHECK_HIP(launch_dequant(sc.s, m, d));
  TRY(sc.get(out, d, (size_t)rows * cols * 4));
  return MOERT_OK;
}

int moert_rmsnorm(const float* x, const float* w, int n, float eps, float* out) {
  CHECK_CFG(x && w && out && n >= 16 && n % 16 == 0, "rmsnorm: n %d must be a multiple of 16", n);
  Scoped sc;
  TRY(sc.init());
  float *dx, *dw, *dout;
  TRY(sc.dev(&dx, n, x));
  TRY(sc.dev(&dw, n, w));
  TRY(sc.dev(&dout, n));
  CHECK_HIP(launch_rmsnorm(sc.s, dx, dw, n, eps, dout));
  TRY(sc.get(out, dout, (size_t)n * 4));
  return MOERT_OK;
}

int moert_rope(float* x, int heads, int head_dim, float theta, int pos) {
  CHECK_CFG(x && heads >= 1 && head_dim >= 2 && head_dim % 2 == 0, "rope: heads %d, head_dim %d", heads, head_dim);
  std::vector<float> cs(head_dim);
  for (int j = 0; j < head_dim / 2; j++) {
    float f = 1.0f / powf(theta, (float)(2 * j) / (float)head_dim);
    float a = (float)pos * f;
    cs[j] = cosf(a);
    cs[head_dim / 2 + j] = sinf(a);
  }
  Scoped sc;
  TRY(sc.init());
  float *dx, *dc;
  TRY(sc.dev(&dx, (size_t)heads * head_dim, x));
  TRY(sc.dev(&dc, head_dim, cs.data()));
  CHECK_HIP(launch_rope(sc.s, dx, heads, head_dim, dc));
  TRY(sc.get(x, dx, (size_t)heads * head_dim * 4));
  return MOERT_OK;
}

int moert_attn_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, int heads, int kv_heads,
                      int head_dim, int max_len, int len, float scale, int tiles_per_split, float* out) {
  CHECK_CFG(q && k_cache && v_cache && out, "null argument");
  CHECK_CFG(head_dim == 64 && heads % kv_heads == 0 && heads / kv_heads <= 4 && max_len % 64 == 0 && len >= 1 &&
                len <= max_len && tiles_per_split >= 1 && attn_splits_for(max_len, tiles_per_split) <= 64,
            "attn: heads %d, kv %d, d %d, max_len %d, len %d, tiles_per_split %d", heads, kv_heads, head_dim, max_len,
            len, tiles_per_split);
  Scoped sc;
  TRY(sc.init());
  float *dq, *part, *dout;
  uint16_t *dk, *dv;
  int* dlen;
  size_t kvn = (size_t)kv_heads * max_len * 64;
  TRY(sc.dev(&dq, (size_t)heads * 64, q));
  TRY(sc.dev(&dk, kvn, k_cache));
  TRY(sc.dev(&dv, kvn, v_cache));
  TRY(sc.dev(&part, (size_t)heads * attn_splits_for(max_len, tiles_per_split) * 66));
  TRY(sc.dev(&dlen, 1, &len));
  TRY(sc.dev(&dout, (size_t)heads * 64));
  CHECK_HIP(launch_attn_unit(sc.s, dq, dk, dv, heads, kv_heads, max_len, dlen, scale, tiles_per_split, part, dout));
  TRY(sc.get(out, dout, (size_t)heads * 64 * 4));
  return MOERT_OK;
}

int moert_attn_decode_noalloc(const float* q_dev, const uint16_t* k_cache_dev, const uint16_t* v_cache_dev, int heads,
                              int kv_heads, int head_dim, int max_len, int len, float scale, int tiles_per_split,
                              float* out_dev, void* stream) {
  CHECK_CFG(q_dev && k_cache_dev && v_cache_dev && out_dev, "attn_noalloc: null argument");
  CHECK_CFG(head_dim == 64 && heads >= 1 && kv_heads >= 1 && heads % kv_heads == 0 && heads / kv_heads <= 4 &&
                max_len >= 64 && max_len % 64 == 0 && len >= 1 && len <= max_len && tiles_per_split >= 1 &&
                attn_splits_for(max_len, tiles_per_split) <= 64,
            "attn_noalloc: heads %d, kv %d, d %d, max_len %d, len %d, tiles_per_split %d", heads, kv_heads, head_dim,
            max_len, len, tiles_per_split);
  const size_t need = kNoallocHeader + (size_t)heads * attn_splits_for(max_len, tiles_per_split) * 66 * 4;
  CHECK_CFG(need <= kNoallocScratchBytes,
            "attn_noalloc: %d heads x %d splits need %zu bytes of partials; the fixed scratch holds %zu", heads,
            attn_splits_for(max_len, tiles_per_split), need - kNoallocHeader, kNoallocScratchBytes - kNoallocHeader);
  hipError_t e;
  uint8_t* base = (uint8_t*)noalloc_scratch(&e);
  CHECK_HIP(e);
  hipStream_t s = (hipStream_t)stream;
  int* lenp = (int*)base;
  float* part = (float*)(base + kNoallocHeader);
  CHECK_HIP(launch_set_int(s, lenp, len));
  CHECK_HIP(launch_attn_unit(s, q_dev, k_cache_dev, v_cache_dev, heads, kv_heads, max_len, lenp, scale,
                             tiles_per_split, part, out_dev));
  return MOERT_OK;
}

int moert_exp_device(const float* x, float* y, int n) {
  CHECK_CFG(x && y && n >= 1, "exp: n %d", n);
  Scoped sc;
  TRY(sc.init());
  float *dx, *dy;
  TRY(sc.dev(&dx, n, x));
  TRY(sc.dev(&dy, n));
  CHECK_HIP(launch_exp(sc.s, dx, dy, n));
  TRY(sc.get(y, dy, (size_t)n * 4));
  return MOERT_OK;
}

int moert_copy_probe(size_t bytes, int iters, double* us_per_copy) {
  CHECK_CFG(bytes >= 16 && bytes % 16 == 0 && iters >= 1 && us_per_copy, "copy_probe: bytes %zu, iters %d", bytes,
            iters);
  Scoped sc;
  TRY(sc.init());
  uint8_t *src, *dst;
  TRY(sc.dev(&src, bytes));
  TRY(sc.dev(&dst, bytes));
  CHECK_HIP(launch_copy(sc.s, src, dst, bytes));  // warm-up
  std::vector<hipEvent_t> ev(2 * iters);
  for (auto& e : ev) CHECK_HIP(hipEventCreate(&e));
  int rc = MOERT_OK;
  for (int i = 0; i < iters && rc == MOERT_OK; i++) {
    arm_launch_events(ev[2 * i], ev[2 * i + 1]);
    if (launch_copy(sc.s, src, dst, bytes) != hipSuccess) rc = MOERT_E_DEVICE;
  }
  double total = 0.0;
  if (rc == MOERT_OK && hipStreamSynchronize(sc.s) == hipSuccess) {
    for (int i = 0; i < iters; i++) {
      float t = 0.0f;
      if (hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]) != hipSuccess) rc = MOERT_E_DEVICE;
      total += t;
    }
  } else {
    rc = MOERT_E_DEVICE;
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  if (rc) {
    set_err("copy_probe: device error");
    return rc;
  }
  *us_per_copy = total * 1000.0 / iters;
  return MOERT_OK;
}

int moert_read_probe(size_t bytes, int iters, double* us_per_read) {
  CHECK_CFG(bytes >= 16 && bytes % 16 == 0 && iters >= 1 && us_per_read, "read_probe: bytes %zu, iters %d", bytes,
            iters);
  // each launch reads its own window of a buffer larger than the 256 MB last-level cache, so every read is cold
  const size_t span = std::max<size_t>(bytes, (size_t)1 << 30);
  const size_t windows = std::max<size_t>(span / bytes, 1);
  Scoped sc;
  TRY(sc.init());
  uint8_t* src;
  unsigned* out;
  TRY(sc.dev(&src, span));
  TRY(sc.dev(&out, (size_t)read_probe_blocks(bytes) * 256));
  CHECK_HIP(launch_read(sc.s, src + (windows - 1) % windows * bytes, bytes, out));  // warm-up (code, queues)
  std::vector<hipEvent_t> ev(2 * iters);
  for (auto& e : ev) CHECK_HIP(hipEventCreate(&e));
  int rc = MOERT_OK;
  for (int i = 0; i < iters && rc == MOERT_OK; i++) {
    arm_launch_events(ev[2 * i], ev[2 * i + 1]);
    if (launch_read(sc.s, src + (size_t)i % windows * bytes, bytes, out) != hipSuccess) rc = MOERT_E_DEVICE;
  }
  double total = 0.0;
  if (rc == MOERT_OK && hipStreamSynchronize(sc.s) == hipSuccess) {
    for (int i = 0; i < iters; i++) {
      float t = 0.0f;
      if (hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]) != hipSuccess) rc = MOERT_E_DEVICE;
      total += t;
    }
  } else {
    rc = MOERT_E_DEVICE;
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  if (rc) {
    set_err("read_probe: device error");
    return rc;
  }
  *us_per_read = total * 1000.0 / iters;
  return MOERT_OK;
}

int moert_h2d_probe(size_t bytes, int iters, double* kernel_us, double* memcpy_us) {
  CHECK_CFG(bytes >= 16 && bytes % 16 == 0 && iters >= 1 && kernel_us && memcpy_us, "h2d_probe: bytes %zu", bytes);
  Scoped sc;
  TRY(sc.init());
  uint8_t* dst;
  TRY(sc.dev(&dst, bytes));
  void* host = nullptr;
  CHECK_HIP(hipHostMalloc(&host, bytes, hipHostMallocMapped | hipHostMallocNonCoherent));
  std::memset(host, 1, bytes);
  void* dev_host = nullptr;
  int rc = MOERT_OK;
  std::vector<hipEvent_t> ev(2 * iters + 2);
  for (auto& e : ev)
    if (hipEventCreate(&e) != hipSuccess) rc = MOERT_E_DEVICE;
  if (!rc && hipHostGetDevicePointer(&dev_host, host, 0) != hipSuccess) rc = MOERT_E_DEVICE;
  if (!rc && launch_h2d_copy(sc.s, dev_host, dst, bytes) != hipSuccess) rc = MOERT_E_DEVICE;  // warm-up
  for (int i = 0; i < iters && !rc; i++) {
    arm_launch_events(ev[2 * i], ev[2 * i + 1]);
    if (launch_h2d_copy(sc.s, dev_host, dst, bytes) != hipSuccess) rc = MOERT_E_DEVICE;
  }
  if (!rc && hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, sc.s) != hipSuccess) rc = MOERT_E_DEVICE;
  if (!rc && hipEventRecord(ev[2 * iters], sc.s) != hipSuccess) rc = MOERT_E_DEVICE;
  for (int i = 0; i < iters && !rc; i++)
    if (hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, sc.s) != hipSuccess) rc = MOERT_E_DEVICE;
  if (!rc && hipEventRecord(ev[2 * iters + 1], sc.s) != hipSuccess) rc = MOERT_E_DEVICE;
  if (!rc && hipStreamSynchronize(sc.s) != hipSuccess) rc = MOERT_E_DEVICE;
  if (!rc) {
    double tk = 0.0;
    for (int i = 0; i < iters; i++) {
      float t = 0.0f;
      (void)hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]);
      tk += t;
    }
    float tm = 0.0f;
    (void)hipEventElapsedTime(&tm, ev[2 * iters], ev[2 * iters + 1]);
    *kernel_us = tk * 1000.0 / iters;
    *memcpy_us = (double)tm * 1000.0 / iters;
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  (void)hipStreamSynchronize(sc.s);
  (void)hipHostFree(host);
  if (rc) set_err("h2d_probe: device error");
  return rc;
}

// ---- host utilities --------------------------------------------------------------------------------------------
int moert_quantize(const float* x, size_t n, int dtype, void* out) {
  CHECK_CFG(x && out && valid_dtype(dtype) && n % 32 == 0, "quantize: n %zu, dtype %d", n, dtype);
  return quantize(x, n, dtype, out);
}

size_t moert_dtype_bytes(int dtype, size_t n) { return dtype_bytes(dtype, n); }

int moert_synth_normal(uint64_t seed, uint64_t stream, size_t n, float scale, float offset, float* out) {
  CHECK_CFG(out, "null output");
  return synth_normal(seed, stream, n, scale, offset, out);
}

int moert_synth_quantized(uint64_t seed, uint64_t stream, size_t n, float scale, int dtype, void* out) {
  CHECK_CFG(out && valid_dtype(dtype) && n % 32 == 0, "synth_quantized: n %zu, dtype %d", n, dtype);
  return synth_quantized(seed, stream, n, scale, dtype, out);
}

int moert_synth_fp16(uint64_t seed, uint64_t stream, size_t n, float scale, uint16_t* out) {
  CHECK_CFG(out, "null output");
  return synth_fp16(seed, stream, n, scale, out);
}

}  // extern "C"

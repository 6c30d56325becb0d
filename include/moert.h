/*
 * moert.h — C ABI of the MI355X (gfx950) Granite-MoE decode engine.
 *
 * The library (libmoert.so, built with hipcc for gfx950) replaces the GPU side of the reference crate
 * `rust/moe-rt` (brenoperucchi/lastro-rust). Every entry point names the reference item it stands in for.
 * Paths are relative to the reference repository root.
 *
 * Conventions
 *  - Every function returns an int status: 0 (MOERT_OK) or a negative MOERT_E_* code. moert_last_error()
 *    returns a thread-local message for the last failure on the calling thread
 *    (mirrors CudaError::{Driver, Kernel, Config}, rust/moe-rt/src/cuda_backend.rs:61-67).
 *  - After a device error the handle is poisoned: the stream is synchronised before any buffer is released,
 *    and later calls on the handle return MOERT_E_POISONED (rust/moe-rt/src/gpu_model.rs:249-267,
 *    rust/moe-rt/src/gpu.rs:451-466).
 *  - All pointers in signatures are host pointers unless a name ends in `_dev`. Sizes are element counts.
 *  - Matrices are row-major [rows, cols]. Quantised matrices use the GGML block layouts:
 *      Q8_0: 34-byte blocks {fp16 d; int8 q[32]}, w = q * d
 *      Q4_0: 18-byte blocks {fp16 d; uint8 nib[16]}, w[j] = ((nib[j] & 15) - 8) * d,
 *            w[j + 16] = ((nib[j] >> 4) - 8) * d
 *    Blocks run along a row; cols must be a multiple of 32.
 *  - One handle must not be used from two threads at once (the reference keeps backend state behind a
 *    Mutex, rust/moe-rt/src/cuda_backend.rs:243).
 */
#ifndef MOERT_H
#define MOERT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MOERT_OK = 0,
  MOERT_E_DEVICE = -1,   /* a HIP call failed (CudaError::Driver) */
  MOERT_E_CONFIG = -2,   /* shape or argument refused before any launch (CudaError::Config) */
  MOERT_E_POISONED = -3, /* the handle saw an earlier device error */
  MOERT_E_FULL = -4,     /* KV cache full (rust/moe-rt/src/gpu_model.rs:252-254) */
  MOERT_E_RANGE = -5     /* token or index out of range (rust/moe-rt/src/gpu_model.rs:255-257) */
};

typedef enum { MOERT_F32 = 0, MOERT_Q8_0 = 1, MOERT_Q4_0 = 2 } moert_dtype;

/* Model constants; mirrors `Config` (rust/moe-rt/src/model.rs:14-31). */
typedef struct {
  int hidden, inter, layers, heads, kv_heads, head_dim, vocab, experts, top_k;
  float rope_theta, eps, embedding_multiplier, residual_multiplier, attention_multiplier, logits_scaling;
} moert_config;

/* A host matrix in one of the dtypes above. */
typedef struct {
  const void* data;
  int dtype; /* moert_dtype */
} moert_tensor;

/* One decoder layer; mirrors `HostDecoder` + `HostLayer` (rust/moe-rt/src/model.rs:76-85,
 * rust/moe-rt/src/block.rs:9-19). */
typedef struct {
  const float* ln_attn;      /* [H] */
  const float* ln_moe;       /* [H] */
  moert_tensor q, k, v, o;   /* [heads*d, H], [kv*d, H], [kv*d, H], [H, heads*d] */
  moert_tensor router;       /* [E, H] */
  const float* router_bias;  /* [E] added to the router logits, or NULL (the Granite router has none;
                                the skewed-routing workloads use one) */
  moert_tensor gate_up;      /* [E, 2I, H]: rows [0, I) gate, [I, 2I) up */
  moert_tensor down;         /* [E, H, I] */
} moert_layer_weights;

/* Whole model; mirrors `HostModel` (rust/moe-rt/src/model.rs:87-93). The embedding is tied to the head. */
typedef struct {
  moert_tensor embed;                /* [V, H] */
  const float* norm;                 /* [H] */
  const moert_layer_weights* layers; /* [layers] */
} moert_model_weights;

typedef struct moert_model moert_model;
typedef struct moert_block moert_block;
typedef struct moert_pool moert_pool;

const char* moert_last_error(void);

/* Device count and name of device 0 (0 devices is not an error). */
int moert_device_info(int* count, char* name, int name_len);

/* ---------------------------------------------------------------------------------------------------------
 * Whole-model decode. Replaces GpuModel::{upload, step, reset} (rust/moe-rt/src/gpu_model.rs:191-267) and the
 * model-mode inherent methods of CudaBackend (new_model, begin_token, read_logits, reset_sequence,
 * rust/moe-rt/src/cuda_backend.rs:466-633).
 * ------------------------------------------------------------------------------------------------------- */

/* Uploads every weight to HBM (all experts resident) and allocates an fp16 KV cache of max_len positions.
 * attn_splits (1..64) caps the split-KV blocks per KV head (ATTN_NS, rust/moe-rt/src/gpu_model.rs:22): each split
 * covers ceil(ceil(max_len/64) / attn_splits) tiles of 64 positions.
 * Replaces GpuModel::upload (rust/moe-rt/src/gpu_model.rs:191-194). */
int moert_model_create(const moert_config* cfg, const moert_model_weights* w, int max_len, int attn_splits,
                       moert_model** out);
int moert_model_destroy(moert_model* m);

/* Same model with the experts served from an expert cache: every expert of every layer lives in pinned host memory
 * and `slots` of them at a time in an HBM pool (top_k <= slots <= min(4096, layers*experts)). Each layer step
 * routes on the device, then applies the LRU rule of the reference's LruSync cache: every requested expert already
 * in the pool is pinned for the step, each miss (in top-k order) takes the first free slot or else the least
 * recently used slot not used in this step (lowest slot index on ties). The kernels that use a missed expert read
 * it from host memory and write it into its slot as they go. No host synchronisation per layer: a step stays one
 * graph of the same kernels as moert_model_create's, and its outputs are identical to that model's. Replaces GpuModel::upload_cached + ExpertCache (rust/moe-rt/src/gpu_model.rs:
 * 197-200, rust/moe-rt/src/cache.rs:140-354, LRU rule of rust/moe-rt/tests/model.rs:380-412). */
int moert_model_create_cached(const moert_config* cfg, const moert_model_weights* w, int max_len, int attn_splits,
                              int slots, moert_model** out);
/* Host-CPU hybrid (the reference's D1 engine in its deterministic mode, AdmitMode::TokenBarrier with the LfuCpu
 * policy: rust/moe-rt/src/motor/engine.rs, motor/line.rs run 802-840, serve_layer 512-583; HostExperts::compute for
 * the misses, rust/moe-rt/src/cpu.rs:116-148; cuda_backend.rs:940-1014). Every expert lives in pinned host memory;
 * a pool of `slots` (0 <= slots <= min(4096, layers*experts); fewer than top_k allowed) holds some of them. Each
 * step is driven from the calling thread: the token's table (the experts resident when it starts) goes to the
 * device; per layer the GPU computes attention, the routing and the experts in the table, the routing and the
 * normalised input come back, the host computes every other routed expert (cpu_threads threads) and a kernel adds
 * their weighted sum into the residual stream; then the placement (moert_placement_*) admits the misses with LFU
 * and the backlog bound, and their records are copied into the pool behind the work already queued, or held until
 * the victim's layer has passed. Outputs equal the resident model's up to the order of the expert sum (the host
 * part is added after the GPU part). moert_cache_stats / _counters / _token_counts / _clear apply; the prefetch and
 * fill entry points, moert_time_kernel, the timeline and the multi-position step refuse a hybrid model. */
int moert_model_create_hybrid(const moert_config* cfg, const moert_model_weights* w, int max_len, int attn_splits,
                              int slots, int backlog, int cpu_threads, moert_model** out);
/* Cache counters since creation or the last clear: requests served from the pool, and copies from host memory
 * (CacheStats::{hits, sync_copies}, rust/moe-rt/src/cache.rs:112-124). */
int moert_cache_stats(moert_model* m, unsigned long long* hits, unsigned long long* copies);
/* Empties the pool and zeroes the counters (ExpertCache::clear, rust/moe-rt/src/cache.rs:216-220). */
int moert_cache_clear(moert_model* m);
/* Copies into the free slots of the pool every expert not yet in it, in key order (key = layer * experts + expert),
 * evicting nothing; stops when no slot is free. *copied = experts copied. Returns synchronised
 * (ExpertCache::fill, rust/moe-rt/src/cache.rs:212-227). The hit/copy counters are not changed. */
int moert_cache_fill(moert_model* m, int* copied);
/* Brings experts[0..n) of `layer` into the pool ahead of a step (the expert-cache prefetch of the proposed
 * moert_pool_prefetch; copy_expert on the copy stream, rust/moe-rt/src/motor/line.rs:423-439): one tick of the
 * step's LRU rule (rust/moe-rt/tests/model.rs:380-412) over these keys, the records copied from the pinned store
 * with hipMemcpyAsync on a side stream that the model stream waits for. Experts distinct, 1 <= n <= min(slots,
 * experts). *copied = experts that were not in the pool. Returns synchronised; counters not changed. */
int moert_cache_prefetch(moert_model* m, int layer, const int* experts, int n, int* copied);
/* Prefetch inside the step (transfers overlapping attention): with on = 1, each layer step of the cached model also
 * predicts the layer's experts (the layer's router applied to rmsnorm of the layer's input, top-k), takes one
 * uncounted tick of the LRU rule over the predicted keys (as moert_cache_prefetch), and copies the predicted misses
 * from the pinned store into their slots before the router + gate/up kernel reads the pool. Where the attention
 * block applies this runs inside its launch (extra workgroups after the attention workgroups; a wait of theirs that
 * gives up is reported as MOERT_E_DEVICE); elsewhere, or with MOERT_PF_BLOCK=0 in the environment when the mode is
 * switched on, on a side stream of the step graph beside the three-kernel attention. Outputs are unchanged (a
 * misprediction is read from the host as before); the counters count the step's requests as before and the
 * prefetched copies apart. on = 0 restores the plain cached step. No reference counterpart beyond
 * copy_in_background (rust/moe-rt/src/cache/core.rs:380), whose copies start only after the miss. */
int moert_cache_prefetch_mode(moert_model* m, int on);
/* The experts predicted for positions [pos0, pos0 + n): [n][layers][8] ids in top-k order (-1 past top_k, and for
 * positions not decoded with prefetch since the last clear). */
int moert_cache_predictions(moert_model* m, int pos0, int n, int* ids);
/* Per position and layer of [pos0, pos0 + n): [n][layers][4] = requests served from the pool, copies inside the step,
 * experts copied ahead by the prefetch branch, 0 (the reference's per-token counters, CacheStats,
 * rust/moe-rt/src/cache.rs:111-124, per token). For a hybrid model: hits, admissions (copies), admissions refused
 * (dropped), requests computed on the host. */
int moert_cache_token_counts(moert_model* m, int pos0, int n, int* counts);
/* Cumulative counters since creation or the last clear; mirrors CacheStats (rust/moe-rt/src/cache.rs:111-124) and
 * the engine's Stats (rust/moe-rt/src/motor/mod.rs:96-109): needed = requests, hits, copies (sync_copies: inside the
 * step), prefetched (copies ahead of the layer), cpu / dropped / deferred (experts served on the host, admissions
 * refused, copies deferred past the victim's layer: 0 for the in-kernel cache), bytes moved host -> HBM by copies,
 * pool slots. */
typedef struct {
  unsigned long long needed, hits, copies, prefetched, cpu, dropped, deferred, bytes_copied;
  int slots;
} moert_cache_counters;
int moert_cache_counters_get(moert_model* m, moert_cache_counters* out);

/* One token at the current position: logits of the next position (vocab floats, divided by logits_scaling),
 * the router decision of every layer (layers*top_k ids and weights, top-k order) and the greedy argmax.
 * Any output pointer may be NULL. Replaces GpuModel::step (rust/moe-rt/src/gpu_model.rs:251-267). */
int moert_decode_step(moert_model* m, int token, float* logits, int* route_ids, float* route_weights,
                      int* argmax);

/* Mode of the multi-position step (moert_step_batched, moert_prefill): 0 (default) the per-row FMA kernels, bit for
 * bit equal to decode steps; 1 the routed experts through the grouped int8 MFMA kernels of the block API
 * (moert_block_forward_batched): the step's own routing, the normalised inputs as 15-bit hi/lo codes, every expert's
 * rows read once for its member positions, exact int32 block products, the sum in first-appearance order, then the
 * residual. Mode 1 needs Q8_0 experts, hidden 1024 or 1536 and inter 128/256/512 on a resident model, and keeps a
 * tiled copy of every layer's experts (built on the first switch). The block prefill through the grouped GEMM
 * (rust/moe-rt/src/cuda_dense.rs:236-288, motor/leitura.rs:79-85). */
int moert_batched_mode(moert_model* m, int mode);

/* Greedy generation with no host synchronisation between tokens: feeds the n_prompt tokens one position at a
 * time, then n_new tokens chosen by argmax (last index on ties). out_tokens receives the n_new generated ids;
 * gaps (optional, n_new floats) receives top1 - top2 of the logits each generated token was chosen from.
 * Replaces the prompt + generation loop of rust/moe-rt/src/bin/m1b-gulosa.rs:85-105. */
int moert_generate(moert_model* m, const int* prompt, int n_prompt, int n_new, int* out_tokens, float* gaps);

/* Multi-position step: tokens[0..n) at positions pos .. pos + n - 1 (n <= 32) in one pass per layer, every weight row
 * read once for the block of positions. Appends their KV rows; logits (nullable, vocab floats) and argmax are
 * those of the last position, which becomes the next token of the sequence; the position advances by n. The
 * result equals n decode steps bit for bit (KV rows, hidden state, logits). Replaces the block step of the model
 * mode: CudaBackend::begin_step_tokens (rust/moe-rt/src/cuda_backend.rs:499-516) and the per-position loops of
 * the step (cuda_backend.rs:751-917, Dense::begin_step cuda_dense.rs:236-288); limit 1..=32 as
 * cuda_backend.rs:272-274. Resident models only (MOERT_E_CONFIG on a cached one). */
int moert_step_batched(moert_model* m, const int* tokens, int n, float* logits, int* argmax);

/* Reads n tokens from the current position in blocks of at most 32 positions (moert_step_batched each; the block
 * plan of plano_blocos, rust/moe-rt/src/motor/leitura.rs:53-60), as
 * le_ids (rust/moe-rt/src/motor/leitura.rs:79-85, validation leitura.rs:62-76): the tokens are checked and the
 * cache bound (MOERT_E_FULL) before any block runs; logits / argmax of the last position. */
int moert_prefill(moert_model* m, const int* tokens, int n, float* logits, int* argmax);

/* Back to position 0 (old KV stays, masked by the length). Replaces GpuModel::reset
 * (rust/moe-rt/src/gpu_model.rs:245-247) and CudaBackend::reset_sequence (cuda_backend.rs:555-558). */
int moert_reset_sequence(moert_model* m);

/* Writes positions [0, n) of layer `layer`'s KV cache from fp16 host arrays laid out [kv_heads, n, head_dim]
 * and leaves the position unchanged. moert_set_position then selects where decoding resumes. */
int moert_kv_prefill_fp16(moert_model* m, int layer, const uint16_t* k, const uint16_t* v, int n);
int moert_set_position(moert_model* m, int pos);
int moert_get_position(moert_model* m, int* pos);

/* Reads positions [0, n) of layer `layer` back (fp16, layout as above). Replaces CudaBackend::read_kv
 * (rust/moe-rt/src/cuda_backend.rs:597-604). */
int moert_read_kv_fp16(moert_model* m, int layer, uint16_t* k, uint16_t* v, int n);

/* Hidden state after the last step (hidden floats, before the final norm). */
int moert_read_hidden(moert_model* m, float* h);

/* Logits of the last step (vocab floats, divided by logits_scaling), e.g. after moert_generate. Replaces
 * Dense::read_logits / CudaBackend::read_logits (rust/moe-rt/src/cuda_dense.rs:446-459,
 * rust/moe-rt/src/cuda_backend.rs:629-633). */
int moert_read_logits(moert_model* m, float* logits);

/* Times `iters` graph replays of the decode step (after `warmup`) with HIP events on the model's stream.
 * ms_per_step receives the mean. The position advances by warmup + iters. */
int moert_time_steps(moert_model* m, int warmup, int iters, double* ms_per_step);

/* Per-kernel timing: replays the step `iters` times as individual launches; every launch of kernel class `kind`
 * (see moert_kernel_kind) is made with start/stop events taken from its own dispatch (hipExtLaunchKernelGGL), and
 * the mean duration of one launch in microseconds and the number of launches timed are returned (0 launches and
 * 0 us for a class the step does not launch). The position advances by iters. */
typedef enum {
  MOERT_K_EMBED = 0,        /* embedding row */
  MOERT_K_QKV = 1,          /* rmsnorm + q/k/v + RoPE + KV write */
  MOERT_K_ATTN_SPLIT = 2,   /* split-KV attention partials */
  MOERT_K_ATTN_COMBINE = 3, /* combine of the split partials */
  MOERT_K_OPROJ = 4,        /* output projection + residual */
  MOERT_K_ROUTE_UP = 5,     /* rmsnorm + router + top-k (+ LRU decision) + gate/up + SwiGLU of the routed experts */
  MOERT_K_EXPERT_DOWN = 6,  /* down of the routed experts + weighted combine + residual */
  MOERT_K_HEAD = 7,         /* final rmsnorm + LM head + per-block argmax */
  MOERT_K_HEAD_ARGMAX = 8,  /* argmax over the head blocks, token and position update */
  MOERT_K_ATTN_BLOCK = 9,   /* q/k/v + RoPE + KV write, split-KV attention and merge in one launch (replaces
                               MOERT_K_QKV, MOERT_K_ATTN_SPLIT and MOERT_K_ATTN_COMBINE where its shape applies) */
  MOERT_K_MOE_XCD = 10,     /* rmsnorm + router + top-8 + gate/up + down with the routed experts spread over the 8
                               XCDs (replaces MOERT_K_ROUTE_UP and MOERT_K_EXPERT_DOWN where it applies) */
  MOERT_K_MOE_COMBINE = 11, /* weighted combine of the last layer's experts + residual, before the head */
  MOERT_K_LAYER = 12,       /* a whole layer in one launch: attention, output projection, router and the routed
                               experts, exchanging through the XCDs' L2s and device-wide (replaces
                               MOERT_K_ATTN_BLOCK, MOERT_K_OPROJ and MOERT_K_MOE_XCD where its shape applies) */
  MOERT_K_LAYER_COMBINE = 13, /* the last layer's experts combined into the head's input after MOERT_K_LAYER */
  MOERT_K_COUNT = 14
} moert_kernel_kind;
int moert_time_kernel(moert_model* m, int kind, int iters, double* us_per_launch, int* launches);

/* Which kernels the model's decode step launches: *layer = 1 when each layer is one launch (MOERT_K_LAYER);
 * otherwise *attn_block = 1 when the attention half is the one-launch attention block (MOERT_K_ATTN_BLOCK) rather
 * than q/k/v + split attention + combine, and *moe_xcd = 1 when the MoE half is the kernel spread over the XCDs
 * (MOERT_K_MOE_XCD) rather than router + gate/up and down. They depend on the shapes, the model kind and its modes
 * (the cache's prefetch side branch uses none of them; its prefetch inside the attention launch keeps the
 * attention block); MOERT_LAYER=0 at create keeps the three launches per layer. No reference counterpart. */
int moert_model_path(const moert_model* m, int* layer, int* attn_block, int* moe_xcd);

/* Test hook for the failure path of the fused kernels (MOERT_K_ATTN_BLOCK, MOERT_K_MOE_XCD); it has no counterpart
 * in the reference. `bits` (a subset of 2 = the wait for queries / the new K/V row, 4 = the wait for split partials,
 * 8 = the wait for an expert's act vector; 0 clears the mask) makes the named waits of the following launches look
 * for an epoch no launch writes, with every wait of those launches bounded to a few hundred polls, so that the wait
 * gives up and the kernels still end normally; the next synchronising call then reports MOERT_E_DEVICE naming the
 * wait, and the model is poisoned. MOERT_E_CONFIG for an expert-cache or hybrid model, or one that does not use
 * the fused kernels. Bit 16 alone (the wait of the cache prefetch's copy workgroups for the layer's predicted misses)
 * applies to an expert-cache model whose prefetch runs inside the attention launch, and to no other. */
int moert_fault_inject(moert_model* m, unsigned bits);

/* Phase timeline of one decode step (measurement build libmoert_tl.so only; MOERT_E_CONFIG otherwise): one graph
 * replay in which every workgroup of every launch stamps the 100 MHz real-time clock at its phase boundaries.
 * out receives [launches][1024][12] u64 records: word 0 = ~(earliest wave start), word 1 = latest wave start,
 * words 2..10 = phase ends seen by wave 0 (0 = no such phase), word 11 = latest wave end; kinds / layers receive each
 * launch's moert_kernel_kind and layer (-1 outside the layers). The position advances by one. No reference
 * counterpart (the reference's phase instrument is perfil_bloco.rs, host-side); used for the latency analysis. */
int moert_timeline_step(moert_model* m, unsigned long long* out, int* kinds, int* layers, int max_launches,
                        int* n_launches);

/* ---------------------------------------------------------------------------------------------------------
 * One MoE block with every expert resident. Replaces GpuLayer::{upload, add_into_routed, run}
 * (rust/moe-rt/src/gpu.rs:430-541) and HostLayer::forward_cpu (rust/moe-rt/src/block.rs:56-62).
 * ------------------------------------------------------------------------------------------------------- */
int moert_block_create(int hidden, int inter, int experts, int top_k, const moert_tensor* router,
                       const float* router_bias, const moert_tensor* gate_up, const moert_tensor* down,
                       moert_block** out);
int moert_block_destroy(moert_block* b);
/* y = sum_j w_j * expert_{id_j}(x) over the top_k experts, ids/weights in top-k order. x is the already
 * normalised block input (hidden floats). */
int moert_block_forward(moert_block* b, const float* x, float* y, int* ids, float* weights);
/* Mean microseconds of one block forward over `iters` launches (inputs resident in HBM). */
int moert_block_time(moert_block* b, int iters, double* us);

/* m positions (1..32) through the block at once: per-position router + top-k, then the routed experts regrouped
 * per expert (first-appearance order) and computed as a grouped int8 MFMA GEMM, each weight row read once for all
 * of its member positions, and y[p] = y[p] + w * o summed in that list order. Activations enter the MFMA as
 * 15-bit block codes (see the kernel header), so the result differs from the f32 per-position path by that
 * rounding only. Q8_0 router and experts. x, y: [m, hidden]; ids, weights: [m, top_k] (nullable outputs).
 * Replaces Cpu::experts_step (rust/moe-rt/src/cpu.rs:239-296) and the per-position GPU loops of the multi-position
 * step (rust/moe-rt/src/cuda_backend.rs:751-917). */
int moert_block_forward_batched(moert_block* b, int m, const float* x, float* y, int* ids, float* weights);
/* The kernels of the block's batched steps: mode 0 (default) the four kernels (route, gate/up, down, combine);
 * mode 1 one launch of 256 workgroups that must all be resident at once, one per compute unit, dealt round-robin
 * over the 8 XCDs (router logits, top-k and input codes through each XCD's L2; gate/up items and down tiles spread
 * over all workgroups, act vectors and expert outputs device-wide), bit-identical to mode 0, for m <= 16 positions,
 * ffn 512, at most 48 experts, Q8_0, on a device with 256 compute units (MOERT_E_CONFIG otherwise). The device
 * must run nothing else meanwhile: a wait of that launch that gives up makes the step return MOERT_E_DEVICE. In
 * mode 1, moert_block_time_batched reports the launch in us[1] and 0 in us[2..4]. No reference counterpart. */
int moert_block_batched_kernel(moert_block* b, int mode);
/* Test hook of the one-launch batched step (mode 1): the waits named by `bits` (1 router logits, 2 act vectors,
 * 4 expert outputs, 8 input codes) look for an epoch no launch writes in the following steps and give up after a few
 * polls, so the step returns MOERT_E_DEVICE while every workgroup still ends normally; 0 restores normal steps. The
 * error is cleared once reported (a block step carries no state into the next). No reference counterpart: it
 * exercises the failure path of the bounded waits. */
int moert_block_fault_inject(moert_block* b, unsigned bits);
/* Number of distinct experts routed by the last batched step on this block (the grouped GEMM's expert count). */
int moert_block_experts_in_step(moert_block* b, int* n_experts);
/* Times `iters` rounds of the batched step over `nblocks` blocks in turn (rotating weights beyond the caches),
 * each block's inputs being those of its last moert_block_forward_batched. us[0] = mean microseconds of one
 * block step; us[1..4] = mean dispatch time of the route, gate/up, down and combine kernels. */
int moert_block_time_batched(moert_block* const* blocks, int nblocks, int m, int iters, double* us);

/* ---------------------------------------------------------------------------------------------------------
 * Unit-parity entry points: one kernel on host buffers (copied in and out). For tests of each subsystem.
 * ------------------------------------------------------------------------------------------------------- */

/* Top-k of logits (ties to the lower index, total order on floats) and softmax over the k.
 * Replaces route_topk (rust/moe-rt/src/route.rs:18-75) / Routing::from_logits (rust/moe-rt/src/block.rs:81-89). */
int moert_router_topk(const float* logits, int n_experts, int k, int* ids, float* weights);

/* Greedy sampler: index of the largest value, last index on ties (rust/moe-rt/src/bin/m1b-gulosa.rs:22-24). */
int moert_argmax(const float* v, int n, int* idx);

/* y = W x for a host matrix of any dtype (rust/moe-rt/src/gpu.rs:21-38, Cpu::gemv cpu.rs:108-113). */
int moert_gemv(const moert_tensor* w, int rows, int cols, const float* x, float* y);

/* Device dequantisation of a quantised matrix to f32 (for the bit-exact dequant check). */
int moert_dequant(const moert_tensor* w, int rows, int cols, float* out);

/* out = w * x / sqrt(mean(x^2) + eps) (rust/moe-rt/src/model.rs:141-145; gpu.rs:108-128). */
int moert_rmsnorm(const float* x, const float* w, int n, float eps, float* out);

/* rotate_half RoPE of `heads` heads of head_dim in place, at position pos (model.rs:148-158, gpu.rs:133-144). */
int moert_rope(float* x, int heads, int head_dim, float theta, int pos);

/* Decode attention of `heads` query heads against an fp16 cache [kv_heads, max_len, head_dim] holding `len`
 * valid positions; split-KV blocks of tiles_per_split 64-position tiles (at most 64 splits per cache)
 * (attn_split + attn_combine, rust/moe-rt/src/gpu.rs:205-292; CpuSession attention model.rs:200-222). */
int moert_attn_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, int heads, int kv_heads,
                      int head_dim, int max_len, int len, float scale, int tiles_per_split, float* out);

/* moert_attn_decode for callers that cannot allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc); it has no counterpart in the reference. q_dev, k_cache_dev, v_cache_dev and
 * out_dev are the caller's device buffers (layouts as moert_attn_decode); the work is enqueued on `stream` (a
 * hipStream_t, NULL for the default stream) and the call returns without synchronising. The split partials and the
 * length word live in a fixed device scratch of 1,081,600 bytes per GPU, held until the process ends: heads x splits
 * must not exceed 64 x 64 (MOERT_E_CONFIG otherwise). No hipMalloc, hipFree or memset is made. Calls that overlap
 * on one GPU (several streams or threads) share that GPU's scratch and race. */
int moert_attn_decode_noalloc(const float* q_dev, const uint16_t* k_cache_dev, const uint16_t* v_cache_dev, int heads,
                              int kv_heads, int head_dim, int max_len, int len, float scale, int tiles_per_split,
                              float* out_dev, void* stream);

/* Achievable HBM bandwidth reference: mean microseconds of one device-to-device streaming copy of `bytes`
 * (multiple of 16) over `iters` launches, each timed by its own dispatch events. No reference counterpart (the
 * reference measures PCIe and HBM rates with separate CUDA tools); used to calibrate the roofline. */
int moert_copy_probe(size_t bytes, int iters, double* us_per_copy);

/* Achievable HBM read bandwidth reference: mean microseconds of one streaming read of `bytes` (multiple of 16) over
 * `iters` launches, each reading its own window of a buffer larger than the last-level cache and timed by its own
 * dispatch events. No reference counterpart; the ceiling a weight-streaming kernel of that size can reach. */
int moert_read_probe(size_t bytes, int iters, double* us_per_read);

/* PCIe reference for the expert cache: mean microseconds of one copy of `bytes` (multiple of 16) from pinned,
 * device-mapped host memory into HBM, by a copy kernel (the way the cached kernels read missed experts) and by hipMemcpyAsync
 * (the DMA engines). The analogue of the reference's PCIe measurement programs (tools/llama-forcado/banda.cu,
 * qual-runs/PCIE-X8-20261031/banda2.cu), which are not on its runtime path. */
int moert_h2d_probe(size_t bytes, int iters, double* kernel_us, double* memcpy_us);

/* Canonical exponential used by every kernel (softmax, SiLU, top-k weights), evaluated on the device. */
int moert_exp_device(const float* x, float* y, int n);

/* ---------------------------------------------------------------------------------------------------------
 * Checkpoint loading (host only, no device needed). Replaces Checkpoint::{open, bf16}
 * (rust/moe-rt/src/weights.rs:52-122), Config::from_json (rust/moe-rt/src/model.rs:34-61) and HostModel::load
 * (rust/moe-rt/src/model.rs:100-132, HostLayer::load rust/moe-rt/src/block.rs:31-53), with the BF16 matrices
 * quantised on load to the engine's formats.
 * ------------------------------------------------------------------------------------------------------- */
typedef struct moert_checkpoint moert_checkpoint;
typedef struct moert_host_model moert_host_model;

/* Granite config.json (len bytes of JSON): refuses model_type other than granitemoe, rope_scaling, attention_bias
 * and untied embeddings; head_dim defaults to hidden / heads. */
int moert_config_from_json(const char* json, size_t len, moert_config* out);
/* Index of every *.safetensors file of `dir` (sorted by name): 8-byte little-endian header length (at most
 * 100 MiB), JSON header {name: {dtype, shape, data_offsets}}, data. Malformed headers, offsets outside a file and
 * a directory without safetensors files are refused with MOERT_E_CONFIG; tensors are read on demand. */
int moert_checkpoint_open(const char* dir, moert_checkpoint** out);
int moert_checkpoint_close(moert_checkpoint* ck);
/* dtype string, shape (up to max_dims) and rank of a tensor; MOERT_E_RANGE when it is missing. */
int moert_checkpoint_tensor(const moert_checkpoint* ck, const char* name, char* dtype, int dtype_len,
                            uint64_t* shape, int max_dims, int* ndim);
/* The n BF16 values (bits) of a tensor; refuses another dtype, a size that does not match the shape and n that
 * differs from the element count. */
int moert_checkpoint_read_bf16(const moert_checkpoint* ck, const char* name, uint16_t* out, size_t n);
/* The Granite-MoE weights of `cfg` (transformers names: model.embed_tokens / model.norm / model.layers.{l}.
 * input_layernorm, post_attention_layernorm, self_attn.{q,k,v,o}_proj, block_sparse_moe.router.layer,
 * block_sparse_moe.input_linear [E, 2I, H], block_sparse_moe.output_linear [E, H, I]), each BF16 matrix widened to
 * f32 and quantised to wdtype (embedding / tied head: embed_dtype), norm weights f32. Shapes are checked. */
int moert_checkpoint_load(const moert_checkpoint* ck, const moert_config* cfg, int wdtype, int embed_dtype,
                          moert_host_model** out);
/* The loaded weights as moert_model_create takes them (valid while the host model lives). */
const moert_model_weights* moert_host_model_weights(const moert_host_model* hm);
int moert_host_model_config(const moert_host_model* hm, moert_config* cfg);
int moert_host_model_destroy(moert_host_model* hm);

/* ---------------------------------------------------------------------------------------------------------
 * Runtime metrics (host only). Replaces the runtime side of the monitor's transport,
 * rust/moe-monitor/src/snapshot.rs: a JSON snapshot of schema 1 (Snapshot, snapshot.rs:18-40, with Model, State,
 * Speed, Context, ExpertCache, Window, Request and Event as snapshot.rs:42-139 define them), rewritten atomically
 * (temporary file in the same directory, data synced, then rename; Publisher::publish, snapshot.rs:172-185), by
 * default at $XDG_RUNTIME_DIR/moe-rt/metrics.json or /tmp/moe-rt-<uid>/metrics.json (default_path,
 * snapshot.rs:146-156). Fractions are over the last window between two publications; totals since the start.
 * ------------------------------------------------------------------------------------------------------- */
typedef struct moert_metrics moert_metrics;

enum { MOERT_STATE_IDLE = 0, MOERT_STATE_READING = 1, MOERT_STATE_GENERATING = 2, MOERT_STATE_QUEUED = 3,
       MOERT_STATE_ERROR = 4 };

typedef struct { double decode_now, decode_last, prefill_now, prefill_request; } moert_metrics_speed;
typedef struct {
  uint32_t slots_total, slots_resident, slots_loading;
  double hit_frac, copy_frac, cpu_frac;
  uint32_t copies_inflight;
  double h2d_gbs;
  uint64_t total_hits, total_copies, total_cpu;
} moert_metrics_cache;
typedef struct { double exposure_frac, gpu_wait_frac, ms_per_token; } moert_metrics_window;
typedef struct {
  uint64_t started_ms, prompt_tokens, reused_tokens, output_tokens, duration_ms;
  double prefill_tok_s, decode_tok_s;
  const char* status; /* "ok", "erro", "em curso", "cancelada" */
} moert_metrics_request;

/* A publisher for `path` (NULL: the default path; its directory is created). started_ms and pid are set here. */
int moert_metrics_create(const char* path, moert_metrics** out);
int moert_metrics_destroy(moert_metrics* mx);
/* The file the publisher writes (NUL-terminated, truncated to len). */
int moert_metrics_path(const moert_metrics* mx, char* buf, int len);
int moert_metrics_set_model(moert_metrics* mx, const char* name, int layers, int experts, int experts_per_tok);
/* kind MOERT_STATE_*: READING (a = done, b = total), GENERATING (a = tokens, b = max_tokens), QUEUED (a = waiting),
 * ERROR (message). */
int moert_metrics_set_state(moert_metrics* mx, int kind, uint64_t a, uint64_t b, const char* message);
int moert_metrics_set_speed(moert_metrics* mx, const moert_metrics_speed* s);
int moert_metrics_set_context(moert_metrics* mx, uint64_t used, uint64_t max);
int moert_metrics_set_cache(moert_metrics* mx, const moert_metrics_cache* c);
int moert_metrics_set_window(moert_metrics* mx, const moert_metrics_window* w);
/* Most recent first; the publisher keeps the last 32. */
int moert_metrics_add_request(moert_metrics* mx, const moert_metrics_request* r);
int moert_metrics_setting(moert_metrics* mx, const char* key, const char* value);
/* level "info", "aviso" or "erro"; oldest first, the publisher keeps the last 64. */
int moert_metrics_event(moert_metrics* mx, const char* level, const char* message);
/* The snapshot as JSON with ts_ms = now (NUL-terminated into buf when it fits; *needed = its length + 1). */
int moert_metrics_json(moert_metrics* mx, char* buf, size_t len, size_t* needed);
/* Writes the snapshot (ts_ms = now) to a temporary file beside the path, syncs it and renames it over the path. */
int moert_metrics_publish(moert_metrics* mx);

/* Lets the model fill `mx` during moert_generate (NULL detaches; the publisher must outlive the attachment): model
 * constants and settings on attach; state (reading the prompt, then generating), context, speed, expert-cache
 * fractions and totals, copy rate and window from the device counters, read back asynchronously every
 * min_interval_ms while the steps run (publications throttled to that interval); on return a request entry, an
 * event and a forced publication. The engine's per-token counters are those of moert_cache_token_counts. */
int moert_model_attach_metrics(moert_model* m, moert_metrics* mx, int min_interval_ms);

/* ---------------------------------------------------------------------------------------------------------
 * Expert placement of the host-CPU hybrid (host only). Replaces the service line of the D1 engine in its
 * deterministic mode (rust/moe-rt/src/motor/line.rs: serve_layer 512-583, victim 605-648, copy_after_reader
 * 653-674, end_token 678-716; AdmitMode::TokenBarrier, policy LfuCpu) and Freq (rust/moe-rt/src/cache.rs:60-87).
 * A token reads the table published at its start: resident experts are computed on the GPU, all other requests on
 * the host; after a layer's host work its missed keys without a slot are admitted when fewer than `backlog` copies
 * are pending in the token and a slot is free or the weakest resident outside the layer's keys (lowest (score,
 * version, key)) scores below the candidate; a copy into the slot of a victim whose layer has not run yet in the
 * token is held until that layer has passed; at the token's end every copy has landed and the next table is
 * published. The counters are those of moert_cache_counters (needed, hits, cpu, copies, dropped, deferred).
 * ------------------------------------------------------------------------------------------------------- */
typedef struct moert_placement moert_placement;
typedef struct moert_freq moert_freq;

/* slots may be 0 (every request on the host); slots <= layers * experts. */
int moert_placement_create(int layers, int experts, int top_k, int slots, int backlog, moert_placement** out);
int moert_placement_destroy(moert_placement* p);
/* One step of m positions through every layer: ids [layers][m][top_k] (distinct ids within a position). Optional
 * outputs: the requests served on the GPU, the copies queued. */
int moert_placement_step(moert_placement* p, const int* ids, int m, int* gpu_requests, int* copies);
int moert_placement_counters(const moert_placement* p, moert_cache_counters* out);
/* The table of the next token: [layers * experts] slot of each key, -1 when not resident. */
int moert_placement_table(const moert_placement* p, int* table);

/* Freq alone (cache.rs:33-71): touch(key, step) with steps that do not go back per key; score = log2 of the decayed
 * value + step / (128 * layers); -inf for a key never touched. */
int moert_freq_create(int keys, int layers, moert_freq** out);
int moert_freq_destroy(moert_freq* f);
int moert_freq_touch(moert_freq* f, int key, uint64_t step);
int moert_freq_score(const moert_freq* f, int key, double* score);
int moert_freq_clear(moert_freq* f);

/* ---------------------------------------------------------------------------------------------------------
 * Tokenizer (host only). Replaces rust/moe-rt/src/tokenizador.rs: the byte-level BPE of the Granite 3.1 tokenizer.json
 * (no normalizer; ByteLevel pre-tokenizer with the GPT-2 pattern and no prefix space; BPE by merge rank without
 * dropout, byte fallback or unknown token; ByteLevel decoder; added tokens found in the raw text by the longest match
 * at the leftmost position). Other configurations are refused at load (MOERT_E_CONFIG), as are sparse ids. Bytes
 * whose ByteLevel character is not in the vocabulary are dropped, as the library does without an unknown token.
 * ------------------------------------------------------------------------------------------------------- */
typedef struct moert_tokenizer moert_tokenizer;

/* Tokenizador::carrega / de_bytes (tokenizador.rs:214-330). */
int moert_tokenizer_load(const char* path, moert_tokenizer** out);
int moert_tokenizer_from_json(const char* json, size_t len, moert_tokenizer** out);
int moert_tokenizer_destroy(moert_tokenizer* t);
/* Size of the id table (largest id + 1). */
int moert_tokenizer_vocab_size(const moert_tokenizer* t, int* n);
/* Text (valid UTF-8) to ids, as the library's encode without special-token post-processing (Tokenizador::codifica,
 * tokenizador.rs:420-448). *n_ids = the count; ids may be NULL to ask for it, else max_ids must hold them (at most len
 * ids). */
int moert_tokenizer_encode(moert_tokenizer* t, const char* text, size_t len, uint32_t* ids, size_t max_ids,
                           size_t* n_ids);
/* Ids to bytes (Tokenizador::decodifica_bytes; added tokens as their literal text); with lossy_text, to UTF-8 with each
 * maximal invalid subpart replaced by U+FFFD (Tokenizador::decodifica). MOERT_E_RANGE for an id outside the
 * vocabulary. *n_bytes = the length; out may be NULL to ask for it. */
int moert_tokenizer_decode(const moert_tokenizer* t, const uint32_t* ids, size_t n, int lossy_text, char* out,
                           size_t max, size_t* n_bytes);
/* The GPT-2 pattern's pieces of a text (pre_tokeniza, tokenizador.rs:118-179): byte offsets of their ends. */
int moert_tokenizer_pretokenize(const char* text, size_t len, size_t* ends, size_t max, size_t* n);
/* The fixed rendering of the Granite 3.1 chat template (renderiza_chat, tokenizador.rs:494-528): roles 0 system,
 * 1 user, 2 assistant; a first system message replaces the default one, which carries `date`; with
 * add_generation_prompt the assistant's opening follows the last message. *needed = the length. */
int moert_chat_render(const int* roles, const char* const* contents, int n, int add_generation_prompt,
                      const char* date, char* out, size_t max, size_t* needed);
/* strftime('%B %d, %Y') in English, validated (formata_data, tokenizador.rs:531-548): NUL-terminated into out. */
int moert_format_date(int year, int month, int day, char* out, size_t max);

/* ---------------------------------------------------------------------------------------------------------
 * Host utilities (no device needed).
 * ------------------------------------------------------------------------------------------------------- */

/* f32 -> GGML Q8_0 / Q4_0 blocks (n multiple of 32). */
int moert_quantize(const float* x, size_t n, int dtype, void* out);
/* Bytes of n elements of a dtype. */
size_t moert_dtype_bytes(int dtype, size_t n);

/* Seeded synthetic data: N(0, 1) * scale + offset as f32, a counter-based generator so that any sub-range can
 * be produced independently (stream = tensor id). */
int moert_synth_normal(uint64_t seed, uint64_t stream, size_t n, float scale, float offset, float* out);
/* Same values quantised straight to Q8_0 / Q4_0 blocks (n multiple of 32), multithreaded. */
int moert_synth_quantized(uint64_t seed, uint64_t stream, size_t n, float scale, int dtype, void* out);
/* Same values rounded to fp16. */
int moert_synth_fp16(uint64_t seed, uint64_t stream, size_t n, float scale, uint16_t* out);

#ifdef __cplusplus
}
#endif
#endif

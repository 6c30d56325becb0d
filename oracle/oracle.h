/*
 * Oracle: CPU restatement of the reference decode path (brenoperucchi/lastro-rust, rust/moe-rt), used ONLY as
 * test infrastructure — by tests/, by __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline
 * leg. Nothing in the product (lastro-rust_amd/) links or calls it.
 *
 * It follows rust/moe-rt/src/model.rs:181-243 (CpuSession::step), block.rs:56-89 (forward_cpu, Routing),
 * cpu.rs:65-150 (swiglu, Cpu::gemv, Cpu::experts), cpu.rs:239-296 (experts_step), pool.rs:96-199 (Pool) and
 * gpu.rs:205-292 (split-KV decode attention), with these build formats in place of the reference's BF16:
 *   - weights are GGML Q8_0 / Q4_0 blocks or f32, dequantised exactly (q * d fits the f32 mantissa);
 *   - the KV cache is fp16, laid out [kv_heads, max_len, head_dim] per layer.
 *
 * Floating-point evaluation order ("canonical order"), shared with the HIP kernels so that results can be
 * compared bit for bit:
 *   dot(w_row, x): the row is cut into chunks of 16 bytes of payload (Q8_0: 16 elements, Q4_0: 32, f32: 4);
 *     chunk j belongs to lane j % 64; each lane accumulates its chunks in increasing j, elements in increasing
 *     index, acc = fmaf(w, x, acc) from +0; the 64 lane sums are added as a balanced pairwise tree
 *     (strides 1, 2, 4, ..., 32).
 *   exp: orc_exp below (Cody-Waite reduction + degree-7 Taylor polynomial), not libm.
 *   division and sqrt are IEEE correctly rounded; no other operation is fused.
 */
#ifndef MOERT_ORACLE_H
#define MOERT_ORACLE_H
#include "../include/moert.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_session orc_session;

float orc_exp(float x);
void orc_exp_n(const float* x, float* y, size_t n);
void orc_h2f_n(const uint16_t* h, float* f, size_t n);
void orc_f2h_n(const float* f, uint16_t* h, size_t n);

/* Exact dequantisation of a GGML blob (or f32 copy). */
void orc_dequant(const void* w, int dtype, size_t n, float* out);
/* Canonical dot of row `row` of a [rows, cols] matrix with x. */
float orc_dot(const void* w, int dtype, int cols, size_t row, const float* x);
void orc_gemv(const void* w, int dtype, int rows, int cols, const float* x, float* y, int threads);

void orc_rmsnorm(const float* x, const float* w, int n, float eps, float* out);
void orc_rope_cos_sin(float theta, int head_dim, int pos, float* cs);
void orc_rope(float* x, int n, int head_dim, const float* cs);
/* Routing::from_logits with an optional bias added first. */
void orc_route(const float* logits, const float* bias, int n, int k, int* ids, float* weights);
void orc_swiglu(const float* h, int inter, float* a);
/* The MoE half's rmsnorm + router logits (bias included) in the engine's partial-block order: per 8-row block b,
 * z[e][b] and ss[b] as fmaf chains, reduced over b in the 64-lane order; r = 1/sqrtf(ss/H + eps),
 * xn = lnw * (h * r), logits[e] = z[e] * r (+ bias[e]). */
void orc_moe_norm_route(const float* h, const float* lnw, const moert_tensor* router, const float* bias, int H, int E,
                        float eps, float* xn, float* logits);
int orc_argmax(const float* v, int n);

/* HostLayer::forward_cpu on a normalised x. */
void orc_moe_block(int hidden, int inter, int experts, int k, const moert_tensor* router, const float* bias,
                   const moert_tensor* gate_up, const moert_tensor* down, const float* x, float* y, int* ids,
                   float* weights, int threads);

/* Split-KV decode attention, canonical order (see oracle.cpp): splits of tiles_per_split 64-position tiles. */
void orc_attention(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, int heads, int kv_heads,
                   int head_dim, int max_len, int len, float scale, int tiles_per_split, float* out);
/* Tiles per split of a cache of max_len positions cut into at most attn_splits splits. */
int orc_tiles_per_split(int max_len, int attn_splits);

/* Cpu::experts_step: m positions, per-position top-k routing; y written for every position. */
void orc_experts_step(int hidden, int inter, int m, int k, const moert_tensor* gate_up, const moert_tensor* down,
                      const float* x, const int* ids, const float* weights, float* y, int threads);

/* Split of x (n multiple of 32) into 15-bit integer codes per 32-element block: d = amax/32639,
 * v = rint(x/d) = 256*hi + lo with lo in [-128, 127] (d = 0 and v = 0 for an all-zero block). */
void orc_quant_hilo(const float* x, int n, int8_t* hi, int8_t* lo, float* d);
/* Row `row` of a Q8_0/Q4_0 matrix against hi/lo codes: per block the exact integer product, then
 * acc = fmaf((float)S, d_w * d_x, acc) in block order. */
float orc_dot_hilo(const void* w, int dtype, int cols, size_t row, const int8_t* hi, const int8_t* lo,
                   const float* dx);
/* experts_step (first-appearance grouping, list-order combine) in the integer block order of the grouped MFMA
 * path; Q8_0/Q4_0 weights. */
void orc_experts_grouped(int hidden, int inter, int m, int k, const moert_tensor* gate_up, const moert_tensor* down,
                         const float* x, const int* ids, const float* weights, float* y, int threads);
/* m positions through one MoE block: per-position router + top-k (canonical order), then orc_experts_grouped. */
void orc_moe_block_batched(int hidden, int inter, int experts, int k, const moert_tensor* router, const float* bias,
                           const moert_tensor* gate_up, const moert_tensor* down, int m, const float* x, float* y,
                           int* ids, float* weights, int threads);

/* LRU expert cache (LruSync rule) replayed over routes [steps][layers][k]: out = {hits, copies, cpu}. */
void orc_lru_replay(const int* routes, int steps, int layers, int k, int experts, int slots,
                    unsigned long long* out);

/* The same cache as a state machine, for traces that mix decode steps with fills and prefetches:
 * step_layer = one counted tick over a layer's routed ids; prefetch = one uncounted tick over `ids` (returns the
 * number copied); fill = ExpertCache::fill (free slots in key order, stamped with the current clock, no tick;
 * returns the number copied); slots = the key held by each slot (-1 free). */
typedef struct orc_lru orc_lru;
orc_lru* orc_lru_create(int layers, int experts, int slots);
void orc_lru_destroy(orc_lru* c);
void orc_lru_step_layer(orc_lru* c, int layer, const int* ids, int k);
int orc_lru_prefetch(orc_lru* c, int layer, const int* ids, int n);
int orc_lru_fill(orc_lru* c);
void orc_lru_stats(const orc_lru* c, unsigned long long* out);
void orc_lru_slots(const orc_lru* c, int* keys);

/* CpuSession. */
int orc_session_create(const moert_config* cfg, const moert_model_weights* w, int max_len, int attn_splits,
                       int threads, orc_session** out);
void orc_session_destroy(orc_session* s);
int orc_session_step(orc_session* s, int token, float* logits, int* route_ids, float* route_weights, float* hidden);
void orc_session_set_pos(orc_session* s, int pos);
int orc_session_pos(orc_session* s);
int orc_session_kv_prefill(orc_session* s, int layer, const uint16_t* k, const uint16_t* v, int n);
int orc_session_read_kv(orc_session* s, int layer, uint16_t* k, uint16_t* v, int n);

/* The grouped mode of the engine's multi-position step (moert_batched_mode 1) over n <= 32 positions from the
 * session's position: q/k/v and output projections as exact integer block products over 15-bit activation codes,
 * each row's blocks in four quarters (orc_dot_hilo_quarters), the norms in the engine's thread orders
 * (orc_rmsnorm_threads: 256 for the attention input, 1024 for the router input), the experts grouped
 * (orc_experts_grouped); route_ids / route_weights [n][layers][k], logits and hidden of the last position. */
float orc_dot_hilo_quarters(const void* w, int dtype, int cols, size_t row, const int8_t* hi, const int8_t* lo,
                            const float* dx);
void orc_rmsnorm_threads(const float* h, const float* lnw, int H, float eps, int threads, float* xn);
int orc_session_step_grouped(orc_session* s, const int* tokens, int n, float* logits, int* route_ids,
                             float* route_weights, float* hidden);
/* CPU port of the reference's CPU decode path (cpu_port.cpp): the reference's own arithmetic shape (dot_avx2's
 * 4 x 8-lane accumulation, f32 KV cache, attention on the calling thread), timed as bench.py's CPU baseline; it
 * agrees with the session above within float rounding, not bit for bit. */
typedef struct port_session port_session;
int port_session_create(const moert_config* cfg, const moert_model_weights* w, int max_len, int threads,
                        port_session** out);
void port_session_destroy(port_session* s);
void port_session_set_pos(port_session* s, int pos);
int port_session_kv_prefill(port_session* s, int layer, const uint16_t* k, const uint16_t* v, int n);
int port_session_step(port_session* s, int token, float* logits, int* route_ids, float* route_weights);
float port_dot(const void* w, int dtype, int cols, size_t row, const float* x);
#ifdef __cplusplus
}
#endif
#endif

/*
 * gh_oracle — CPU restatement of graph_horizon_engine's CPU backend (TEST INFRASTRUCTURE).
 *
 * This library is the numeric checker for the HIP backend. Only tests/, the smoke() entry
 * and bench.py's cpu_baseline leg may load it; the product library never links it.
 * Every function names the reference file:line it restates (paths relative to
 * crates/graph_horizon_engine/src/ of etufarini/graph-horizon).
 *
 * Conventions shared with the reference:
 *   - FP16 values travel as little-endian uint16 bits; widening is exact, narrowing is RNE.
 *   - Weight tensors are GGUF row-major [out][in/256 blocks]; Q4_K 144 B/block, Q6_K 210 B/block.
 *   - matmul writes FP16, logits writes FP32, both FP32-accumulated.
 *   - No FMA contraction except where the reference uses an explicit fused intrinsic
 *     (_mm256_fmadd_ps / _mm256_fmsub_ps), which this restatement uses identically.
 */
#ifndef GH_ORACLE_H
#define GH_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- thread pool (backend/cpu/parallel.rs:41-102) ---- */
void gho_set_threads(int n);
int gho_threads(void);

/* ---- f16 (backend/f16.rs:11-71, backend/cpu/f16.rs:131-218) ---- */
float gho_f16_to_f32(uint16_t h);
uint16_t gho_f32_to_f16(float f);
void gho_f16_to_f32_slice(const uint16_t* src, float* dst, size_t n);
void gho_f32_to_f16_slice(const float* src, uint16_t* dst, size_t n);

/* ---- dequant (backend/cpu/dequant.rs:78-410) ---- */
void gho_scale_min(const uint8_t* scales12, uint32_t j, uint32_t* sc, uint32_t* mn);
/* format: 12 = Q4_K, 14 = Q6_K, 1 = F16. Returns 0, or -1 for an unsupported format. */
int gho_dequant_row(uint32_t format, const uint8_t* bytes, size_t row, size_t in_dim, float* out);
int gho_validate(uint32_t format, size_t byte_len);

/* ---- fused GEMV (backend/cpu/kernels/matmul/{q4k,q4k_simd,q6k,q6k_simd}.rs) ---- */
float gho_row_dot_q4k_scalar(const float* a, const uint8_t* w, size_t row, size_t in_dim);
float gho_row_dot_q4k_avx2(const float* a, const uint8_t* w, size_t row, size_t in_dim);
float gho_row_dot_q6k_scalar(const float* a, const uint8_t* w, size_t row, size_t in_dim);
float gho_row_dot_q6k_avx2(const float* a, const uint8_t* w, size_t row, size_t in_dim);
/* kernels::matmul::{matmul,logits} (matmul/mod.rs:186-332): a is FP16[in]. */
int gho_matmul(uint32_t format, uint16_t* out_f16, const uint16_t* a_f16, const uint8_t* w,
               size_t in_dim, size_t out_dim);
int gho_logits(uint32_t format, float* out_f32, const uint16_t* x_f16, const uint8_t* w,
               size_t in_dim, size_t out_dim);
/* kernels::matmul::matmul_batched (matmul/mod.rs:223-275): a FP16[n][in], out FP16[n][out]. */
int gho_matmul_batched(uint32_t format, uint16_t* out_f16, const uint16_t* a_f16,
                       const uint8_t* w, size_t in_dim, size_t out_dim, size_t n);
/* batched per-row kernels (q4k_simd.rs:117-181, q6k_simd.rs:145-192), out[n] f32 */
void gho_row_dot_q4k_avx2_batched(const float* a, const uint8_t* w, size_t row, size_t in_dim,
                                  float* out, size_t n);
void gho_row_dot_q6k_avx2_batched(const float* a, const uint8_t* w, size_t row, size_t in_dim,
                                  float* out, size_t n);

/* ---- attention (backend/cpu/kernels/attention/mod.rs:458-725) ----
 * Caches are FP16 [layer][context][kv_heads][head_dim]. */
void gho_attention_decode(uint16_t* out, const uint16_t* q, const uint16_t* k_cache,
                          const uint16_t* v_cache, size_t key_dim, size_t value_dim,
                          size_t kv_heads, size_t q_heads, size_t pos, size_t layer,
                          size_t context);
void gho_attention_prefill(uint16_t* out, const uint16_t* q, const uint16_t* k_cache,
                           const uint16_t* v_cache, size_t key_dim, size_t value_dim,
                           size_t kv_heads, size_t q_heads, size_t base, size_t n, size_t layer,
                           size_t context);
/* serial scalar three-pass reference (attention/mod.rs:876-913 test body) */
void gho_attention_decode_serial(uint16_t* out, const uint16_t* q, const uint16_t* k_cache,
                                 const uint16_t* v_cache, size_t head_dim, size_t kv_heads,
                                 size_t q_heads, size_t pos, size_t layer, size_t context);

/* ---- elementwise (backend/cpu/kernels/elementwise/ normalization, activation, residual, embedding) ---- */
void gho_rmsnorm_x(uint16_t* out, const float* x, const uint16_t* w, size_t dim, float eps,
                   size_t rows);
void gho_silu_mul(uint16_t* out, const uint16_t* gate, const uint16_t* up, size_t n);
void gho_residual_add(float* x, const uint16_t* y, size_t n);
int gho_embed(float* x, uint32_t format, const uint8_t* token_embd, size_t token, size_t embd);

/* ---- YaRN RoPE (backend/rope.rs:11-133, cpu/kernels/elementwise/rope.rs:14-39) ---- */
typedef struct gho_yarn {
    uint32_t rope_dim;
    uint32_t original_context;
    float freq_base;
    float factor;
    float beta_fast;
    float beta_slow;
    float log_multiplier;
    float q_temperature_scale;
} gho_yarn;
/* role 0 = Query, 1 = Key. Returns 0 or -1 on invalid parameters / pair index. */
int gho_yarn_pair(const gho_yarn* y, int role, size_t pair, size_t position, float* cos_out,
                  float* sin_out);
float gho_yarn_post_scale(const gho_yarn* y, int role, size_t position);
void gho_yarn_correction_dims(const gho_yarn* y, float* start, float* end);
int gho_rope_yarn(uint16_t* x, size_t heads, size_t head_dim, size_t pos, const gho_yarn* y,
                  int role);

/* ---- readback (backend/cpu/readback.rs:45-69) ---- */
uint32_t gho_argmax(const float* logits, size_t vocab);
/* writes min(k, vocab) pairs; returns the count */
size_t gho_topk(const float* logits, size_t vocab, size_t k, uint32_t* idx, float* val);

/* ---- KV layout (kv_cache/layout.rs:22-89, f16 scheme) ---- */
uint64_t gho_kv_payload_offset(size_t layer, size_t pos, size_t kv_heads, size_t head_dim,
                               size_t context);
uint64_t gho_kv_buffer_bytes(size_t block_count, size_t context, size_t kv_heads,
                             size_t head_dim);

/* ---- Graph restatement (family/mistral/graph/{forward,block,mlp,tail}.rs,
 *      graph/prefill/{encode,layer}.rs) over host buffers ---- */
typedef struct gho_model_cfg {
    uint32_t block_count;
    uint32_t context_length;
    uint32_t embedding_length;
    uint32_t feed_forward_length;
    uint32_t head_count;
    uint32_t kv_head_count;
    uint32_t key_length;
    uint32_t value_length;
    uint32_t vocab_size;
    float rms_epsilon;
    gho_yarn yarn;
} gho_model_cfg;

/* tensors per layer, in this order (backend/source.rs canonical order restated) */
enum {
    GHO_ATTN_NORM = 0,
    GHO_ATTN_Q = 1,
    GHO_ATTN_K = 2,
    GHO_ATTN_V = 3,
    GHO_ATTN_OUTPUT = 4,
    GHO_FFN_NORM = 5,
    GHO_FFN_GATE = 6,
    GHO_FFN_UP = 7,
    GHO_FFN_DOWN = 8,
    GHO_LAYER_TENSORS = 9
};

typedef struct gho_tensor {
    const uint8_t* bytes; /* F16 norms (already narrowed), or Q4_K/Q6_K GGUF blocks */
    uint32_t format;
} gho_tensor;

typedef struct gho_model gho_model;
gho_model* gho_model_create(const gho_model_cfg* cfg, const gho_tensor* token_embd,
                            const gho_tensor* output_norm, const gho_tensor* output,
                            const gho_tensor* layers /* block_count*GHO_LAYER_TENSORS */,
                            uint32_t kv_context);
void gho_model_destroy(gho_model* m);
/* forward::token (graph/forward.rs:68-83): logits f32[vocab] of the token at pos */
int gho_model_token(gho_model* m, uint32_t token, uint32_t pos);
/* prefill::prefill (graph/prefill/encode.rs:16-106), one chunk of row_capacity rows at a time */
int gho_model_prefill(gho_model* m, const uint32_t* tokens, uint32_t n, uint32_t base,
                      uint32_t row_capacity);
const float* gho_model_logits(const gho_model* m);
/* KV cache bytes of one role (0 = K, 1 = V), for cross-checks */
const uint16_t* gho_model_kv(const gho_model* m, int role);
/* last-layer hidden residual x (f32[embedding_length]) after the most recent call */
const float* gho_model_x(const gho_model* m);
/* Copies positions [0, positions) of every layer's K and V from caches laid out like this
 * model's ([layer][src_context][kv_heads][dim]) into the model's cache: lets a test resume a
 * sequence from another implementation's cache and recompute the following positions. */
int gho_model_load_kv(gho_model* m, const uint16_t* k, const uint16_t* v, uint32_t src_context,
                      uint32_t positions);
/* op trace of the following token/prefill calls (on != 0 clears and starts it): one name per
 * op, the tensor's name (l<i>.q, output_norm, logits:output, ...) when the op takes one */
void gho_model_set_trace(gho_model* m, int on);
const char* gho_model_trace(gho_model* m); /* newline-separated, valid until the next call */
/* A planted mistake for tests that show a parity check can fail (never set otherwise):
 * GHO_PLANT_NONE, or the YaRN post-scale (rope.rs:91-100) applied to K as well as Q, or
 * dropped from Q. Only the per-row RoPE roles of layer_rows change. */
enum { GHO_PLANT_NONE = 0, GHO_PLANT_POST_SCALE_ON_K = 1, GHO_PLANT_NO_POST_SCALE_ON_Q = 2 };
int gho_model_set_plant(gho_model* m, int plant);

#ifdef __cplusplus
}
#endif
#endif

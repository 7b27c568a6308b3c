/*
 * gh_backend.h — C ABI of the MI355X (gfx950) numeric backend for graph_horizon_engine.
 *
 * This is the drop-in boundary: every entry point below replaces one method of the engine's
 * `trait Backend` (crates/graph_horizon_engine/src/backend/contract.rs:20-319, cited per
 * function as contract.rs:LINE), in the same argument order, so a Rust `backend/hip/` crate
 * is a set of thin `extern "C"` delegators. Plain pointers and integers only.
 *
 * Conventions
 *   - Status: 0 = GH_OK, negative = a bounded GH_E_* code. No exception crosses the ABI.
 *   - Ops the trait declares infallible (matmul, logits, rmsnorm_x, silu_mul, residual_add,
 *     attention_*) still return a status; an error is also latched in the encoder and
 *     reported again by gh_submit, as the Vulkan backend reports at submit_wait.
 *   - One backend = one HIP device + one HIP stream. The caller serializes calls
 *     (generation is serialized in the engine, runtime/homogeneous.rs:18-124).
 *   - Dimensions are u32, byte offsets u64 (contract.rs:29-56).
 *   - FP16 activations, FP32 residual and logits, FP16 KV cache (the f16 scheme).
 *   - Weight format travels with the buffer (cpu/buffer.rs:48-53): ggml type ids
 *     F32 = 0, F16 = 1, Q4_K = 12, Q6_K = 14 (gguf/tensor_index.rs:36-54).
 */
#ifndef GH_BACKEND_H
#define GH_BACKEND_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum gh_status {
    GH_OK = 0,
    GH_E_INVALID = -1,     /* bad argument, size or shape */
    GH_E_NO_DEVICE = -2,   /* no HIP device, or the device is not gfx950 */
    GH_E_HIP = -3,         /* a HIP runtime call failed */
    GH_E_OOM = -4,         /* device allocation failed */
    GH_E_RANGE = -5,       /* position/offset beyond a buffer or the context */
    GH_E_MODULE = -6,      /* the gfx950 code object could not be loaded */
    GH_E_STATE = -7,       /* call out of order (no encoder, double begin, ...) */
    GH_E_UNSUPPORTED = -8  /* format/scheme outside the admitted Q4_K_M profile */
};

enum gh_format { GH_FMT_F32 = 0, GH_FMT_F16 = 1, GH_FMT_Q4_K = 12, GH_FMT_Q6_K = 14 };

enum gh_buf_kind {
    GH_BUF_ALLOC = 1,  /* owns a device allocation; free with gh_free_buffer */
    GH_BUF_VIEW = 2,   /* aliases a parent window; never freed (contract.rs:32-48) */
    GH_BUF_WEIGHT = 3  /* owns a quantized weight in the device layout; free with gh_free_buffer */
};

/* A buffer handle, passed by value like the trait's `Buffer`. `addr` is the device address of
 * byte 0 of the window. For GH_BUF_WEIGHT, rows = out_dim and cols = in_dim of the matrix. */
typedef struct gh_buf {
    uint64_t addr;
    uint64_t bytes;
    uint32_t format;
    uint32_t kind;
    uint32_t rows;
    uint32_t cols;
} gh_buf;

typedef struct gh_config {
    int32_t device;               /* HIP device ordinal */
    const char* code_object_path; /* directory of the gh_<module>_gfx950.co code objects;
                                     NULL: the directory libgh_hip.so was loaded from */
} gh_config;

/* Ministral YaRN parameters (backend/rope.rs:11-21). */
typedef struct gh_yarn {
    uint32_t rope_dim;
    uint32_t original_context;
    float freq_base;
    float factor;
    float beta_fast;
    float beta_slow;
    float log_multiplier;
    float q_temperature_scale;
} gh_yarn;

enum gh_rope_role { GH_ROPE_QUERY = 0, GH_ROPE_KEY = 1 }; /* backend/rope.rs:23-27 */
enum gh_kv_scheme { GH_KV_F16 = 0, GH_KV_INT8 = 1 };      /* kv_cache/scheme.rs */

/* Request KV handle (kv_cache/mod.rs:29-38). Caches are [layer][context][kv_heads][dim]. */
typedef struct gh_kv {
    gh_buf k;
    gh_buf v;
    uint32_t scheme;
    uint32_t block_count;
    uint32_t context;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t value_dim;
} gh_kv;

typedef struct gh_backend gh_backend;
typedef struct gh_encoder gh_encoder;

/* ---- lifecycle: backend/selection.rs:40-81 (load) — device init, gfx950 check,
 *      hipModuleLoad of the kernels' code object ---- */
int gh_create(const gh_config* cfg, gh_backend** out);
void gh_destroy(gh_backend* b);
/* Short description of the most recent error on this backend (static storage, never NULL). */
const char* gh_last_error(const gh_backend* b);

/* ---- buffers ---- */
/* alloc_buffer, contract.rs:29 */
int gh_alloc_buffer(gh_backend* b, uint64_t bytes, gh_buf* out);
/* free_buffer, contract.rs:30 (views are rejected with GH_E_INVALID, contract.rs:38-40) */
int gh_free_buffer(gh_backend* b, gh_buf* buf);
/* view, contract.rs:48: alias of [offset, offset+len) of `buf`, no allocation, no copy;
 * offset_bytes must be a multiple of gh_min_buffer_offset_alignment (GH_E_INVALID otherwise) */
int gh_view(gh_backend* b, const gh_buf* buf, uint64_t offset_bytes, uint64_t len_bytes,
            gh_buf* out);
/* min_buffer_offset_alignment, contract.rs:56: 16 (rows are read with 16-byte loads) */
uint64_t gh_min_buffer_offset_alignment(const gh_backend* b);
/* host<->device copies (the CPU backend's buffer read/write; vulkan/mem/buffers.rs staging);
 * synchronous with respect to the backend stream */
int gh_upload(gh_backend* b, const gh_buf* dst, uint64_t offset, const void* src, uint64_t len);
int gh_download(gh_backend* b, const gh_buf* src, uint64_t offset, void* dst, uint64_t len);
/* Weight load (cpu/weights.rs:37-174, vulkan/mem/weights.rs): GGUF block bytes of an
 * [out_dim][in_dim] matrix. Q4_K/Q6_K are validated as whole blocks (cpu/dequant.rs:35-41) and
 * repacked losslessly into the device layout; F32 is narrowed RNE to F16 (cpu/weights.rs:155),
 * F16 is copied. in_dim must be a multiple of 256 for quantized formats. */
int gh_load_weight(gh_backend* b, uint32_t format, const void* bytes, uint64_t len,
                   uint32_t in_dim, uint32_t out_dim, gh_buf* out);
/* Decode rows [row0, row0+rows) of a quantized weight to FP32 [rows][in_dim] on the device
 * (dequant_row, cpu/dequant.rs:47-67); the bit-exact reference for the dequant parity check. */
int gh_dequant_rows(gh_backend* b, gh_encoder* enc, const gh_buf* out_f32, const gh_buf* w,
                    uint32_t row0, uint32_t rows);

/* ---- encoder: begin, contract.rs:78; submit, contract.rs:79 (synchronous);
 *      no_barrier, contract.rs:87 (a scheduling hint; never changes the math) ---- */
int gh_begin(gh_backend* b, gh_encoder** enc);
int gh_submit(gh_backend* b, gh_encoder* enc);
void gh_no_barrier(gh_backend* b);

/* ---- numeric ops ---- */
/* kv_write, contract.rs:64-75 (f16 scheme: raw copy of `vectors` K and V vectors to the
 * payload byte offsets computed by kv_cache/layout.rs) */
int gh_kv_write(gh_backend* b, gh_encoder* enc, const gh_kv* kv, const gh_buf* k,
                const gh_buf* v, uint64_t k_payload_offset, uint64_t v_payload_offset,
                uint64_t k_meta_offset, uint64_t v_meta_offset, uint32_t vectors);
/* embed, contract.rs:91-98: dequantize row `token` of token_embd into FP32 x */
int gh_embed(gh_backend* b, gh_encoder* enc, const gh_buf* x, const gh_buf* token_embd,
             uint32_t token, uint32_t embd);
/* matmul, contract.rs:101-109: out FP16[out_dim] = W · a (a FP16[in_dim]) */
int gh_matmul(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* a,
              const gh_buf* w, uint32_t in_dim, uint32_t out_dim);
/* matmul_batched, contract.rs:119-145: a FP16[n][in_dim] -> out FP16[n][out_dim] */
int gh_matmul_batched(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* a,
                      const gh_buf* w, uint32_t in_dim, uint32_t out_dim, uint32_t n);
/* logits, contract.rs:148-156: out FP32[out_dim] = W · x */
int gh_logits(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* x,
              const gh_buf* w, uint32_t in_dim, uint32_t out_dim);
/* rmsnorm_x, contract.rs:159-168: FP32 x rows -> FP16 out, FP16 weight */
int gh_rmsnorm_x(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* x,
                 const gh_buf* w, uint32_t dim, float eps, uint32_t rows);
/* rope_yarn, contract.rs:172-181: in place on FP16 x[heads][head_dim] at position pos.
 * Rotations come from a table built for the YaRN parameters (rebuilt when they change):
 * positions at or beyond 262144 (MAX_CONTEXT, family/mistral/version.rs:16) are GH_E_RANGE. */
int gh_rope_yarn(gh_backend* b, gh_encoder* enc, const gh_buf* x, uint32_t heads,
                 uint32_t head_dim, uint32_t pos, const gh_yarn* yarn, uint32_t role);
/* rope_yarn_batched, contract.rs:187-246: rows packed Q then K rows at base..base+rows */
int gh_rope_yarn_batched(gh_backend* b, gh_encoder* enc, const gh_buf* q, const gh_buf* k,
                         uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim, uint32_t base,
                         uint32_t rows, const gh_yarn* yarn);
/* silu_mul, contract.rs:252-259: out = f16(f16(silu(gate)) * up) */
int gh_silu_mul(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* gate,
                const gh_buf* up, uint32_t n);
/* residual_add, contract.rs:261: FP32 x[i] += FP16 y[i] */
int gh_residual_add(gh_backend* b, gh_encoder* enc, const gh_buf* x, const gh_buf* y,
                    uint32_t n);
/* attention_decode, contract.rs:267-276 */
int gh_attention_decode(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* q,
                        const gh_kv* kv, uint32_t q_heads, uint32_t pos, uint32_t layer);
/* attention_prefill, contract.rs:288-298 */
int gh_attention_prefill(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* q,
                         const gh_kv* kv, uint32_t q_heads, uint32_t base, uint32_t n,
                         uint32_t layer);

/* attention_decode without allocation. No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same arguments, kernels and results as gh_attention_decode; the
 * split partials and merge counters live in a fixed 1 MiB device array per GPU (4 KiB of
 * counters, then q_heads x splits x 520 B of partials — 32 query heads at the 32-split
 * maximum use 532 KiB), and launches that need more are rejected with GH_E_RANGE. Nothing is
 * allocated. Calls on one GPU share the array: calls that overlap on the same GPU (other
 * streams or backends) race. */
int gh_attention_decode_noalloc(gh_backend* b, gh_encoder* enc, const gh_buf* out,
                                const gh_buf* q, const gh_kv* kv, uint32_t q_heads, uint32_t pos,
                                uint32_t layer);

/* ---- read-back, contract.rs:300-318 (synchronous) ---- */
int gh_read_logits(gh_backend* b, const gh_buf* logits, uint64_t vocab, float* dst);
/* lowest index wins on equal logits (strict `>`) */
int gh_read_argmax(gh_backend* b, const gh_buf* logits, uint64_t vocab, uint32_t* out);
/* min(k, vocab) pairs ordered by (logit desc by IEEE total order, index asc); k <= 128 is
 * reduced on the device (the Vulkan backend's partial scan, vulkan/kernels/reduce.rs:74-139,
 * with the merge on the device too), larger k on the host over read-back logits */
int gh_read_topk(gh_backend* b, const gh_buf* logits, uint64_t vocab, uint64_t k,
                 uint32_t* idx, float* val, uint64_t* count);

/* ---- measurement helpers (no counterpart in the reference: the engine measures through
 *      its public event stream, harness/throughput.rs:64-147). HIP events recorded on the
 *      backend's stream, so they bracket exactly the kernels this backend launches. ---- */
int gh_timer_start(gh_backend* b);
/* milliseconds since gh_timer_start, after synchronizing the stream */
int gh_timer_stop(gh_backend* b, float* ms);
int gh_synchronize(gh_backend* b);
/* Attention split count (no counterpart in the reference: a test and tuning hook). Decode
 * attention splits each (row, kv head) over this many workgroups (at most one per 64-position
 * chunk); 0 restores the backend's policy (about two workgroups per CU). At most 32. Graphs
 * recorded before the call are re-recorded on their next use. */
int gh_set_attention_splits(gh_backend* b, uint32_t splits);
/* Decode attention's split merge (no counterpart in the reference: a test and tuning hook).
 * gh_create checks whether the device's dispatcher places workgroup i of a launch on XCD
 * i mod n (n = gh_xcd_count, 0 when not confirmed); if so, decode attention runs every split of
 * a (row, kv head) on one XCD and exchanges the partials through that XCD's L2 (enable = 1, the
 * default then), else through device memory (enable = 0). The results are the same bits either
 * way. Enabling without a confirmed placement fails with GH_E_UNSUPPORTED. Graphs recorded
 * before the call are re-recorded on their next use. */
int gh_set_attention_xcd_merge(gh_backend* b, int enable);
uint32_t gh_xcd_count(const gh_backend* b);

/* A plain streaming read of [offset, offset + bytes) of `src` by `workgroups` workgroups of
 * 256 threads (no counterpart in the reference: a measurement kernel). It stands for the
 * weight stream of a decode GEMV of the same size with no arithmetic, so its duration is the
 * floor of one launch of that size. `sink` (at least 4 bytes) is almost never written;
 * offset and bytes are multiples of 16. */
int gh_stream_probe(gh_backend* b, gh_encoder* enc, const gh_buf* src, uint64_t offset,
                    uint64_t bytes, const gh_buf* sink, uint32_t workgroups);

/* The backend's growable device scratch (no counterpart in the reference: a diagnostic for
 * tests): workspace bytes (split-K and attention partials, argmax partials), attention-merge
 * counter slots, and a generation number bumped whenever either is reallocated or a recorded
 * graph must be re-recorded. Any argument may be NULL. */
int gh_scratch_info(const gh_backend* b, uint64_t* workspace_bytes, uint64_t* counter_slots,
                    uint64_t* generation);

/* =====================================================================================
 * Graph driver: a C++ restatement of the caller side of the boundary — MistralGraph's pinned
 * op order for one token (family/mistral/graph/forward.rs:68-83, block.rs:17-107,
 * mlp.rs:12-61, tail.rs:22-59) and for batched prefill (graph/prefill/encode.rs:16-106,
 * prefill/layer.rs:18-122) — recorded through the ops above. It owns the engine-side
 * `Buffers{weights, scratch, logits}` (backend/buffers.rs:17-60) and one request KV.
 * ===================================================================================== */
typedef struct gh_model_config {
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
    gh_yarn yarn;
    uint32_t kv_context;   /* request KV capacity in tokens (kv_cache::alloc_shape) */
    uint32_t prefill_rows; /* prefill chunk row capacity (graph/prefill/mod.rs:20-22);
                              0: gh_prefill_rows(backend, block_count, kv_context) */
    uint32_t flags;        /* GH_MODEL_* bits */
} gh_model_config;

/* gh_model_decode_greedy launches each step's kernels directly on the stream instead of
 * replaying one captured HIP graph (same kernels, same device-resident token/position);
 * for tools that cannot trace kernels inside graphs. */
#define GH_MODEL_NO_GRAPH 1u
/* gh_model_prefill keeps no FP16 copy of the layer matrices. By default the first prefill
 * call with chunks of more than 128 rows dequantizes each Q/K/V/O/gate/up/down matrix once
 * into an FP16 copy (2 bytes per weight: 14.8 GB for the 8B shape), which the GEMMs of such
 * chunks then copy into LDS instead of dequantizing every tile; the results are the same
 * bits either way. Without the memory for the copy, the prefill dequantizes as with this
 * flag. */
#define GH_MODEL_NO_F16_WEIGHTS 2u

/* Tensor ids for gh_model_load_tensor. Per-layer ids follow backend/source.rs's canonical
 * order; global ids use layer = UINT32_MAX. */
enum gh_tensor_id {
    GH_T_ATTN_NORM = 0,
    GH_T_ATTN_Q = 1,
    GH_T_ATTN_K = 2,
    GH_T_ATTN_V = 3,
    GH_T_ATTN_OUTPUT = 4,
    GH_T_FFN_NORM = 5,
    GH_T_FFN_GATE = 6,
    GH_T_FFN_UP = 7,
    GH_T_FFN_DOWN = 8,
    GH_T_TOKEN_EMBD = 16,
    GH_T_OUTPUT_NORM = 17,
    GH_T_OUTPUT = 18
};

/* The backend's prefill chunk policy (VulkanBackend::prefill_rows, vulkan/mod.rs:65-75 with
 * profile.rs:42-58; selection.rs:95,124 sizes the request's prefill scratch with it): rows per
 * prefill batch for a model of block_count blocks and a request context. Host-only. */
uint32_t gh_prefill_rows(const gh_backend* b, uint32_t block_count, uint32_t context);

typedef struct gh_model gh_model;
int gh_model_create(gh_backend* b, const gh_model_config* cfg, gh_model** out);
void gh_model_destroy(gh_model* m);
/* GGUF bytes of one tensor (F32 norms are narrowed to F16 at load, cpu/weights.rs:151-174) */
int gh_model_load_tensor(gh_model* m, uint32_t layer, uint32_t tensor, uint32_t format,
                         const void* bytes, uint64_t len);
/* forward::token: embed, block_count blocks, tail; FP32 logits left on the device */
int gh_model_token(gh_model* m, uint32_t token, uint32_t pos);
/* prefill::prefill: tokens[0..n) at positions base.., chunked by prefill_rows */
int gh_model_prefill(gh_model* m, const uint32_t* tokens, uint32_t n, uint32_t base);
int gh_model_read_logits(gh_model* m, float* dst);
int gh_model_read_argmax(gh_model* m, uint32_t* out);
/* Greedy decode loop (generation/mod.rs:107-139 with sampling's greedy argmax): starting
 * from `token` at `pos`, runs `steps` decode steps; step i feeds the argmax of step i-1.
 * The whole step (embed .. logits .. argmax) is one replayed HIP graph with the token id and
 * position resident on the device; tokens_out[i] receives the argmax of step i. */
int gh_model_decode_greedy(gh_model* m, uint32_t token, uint32_t pos, uint32_t steps,
                           uint32_t* tokens_out);
/* read_topk over the model's logits (min(k, vocab) pairs, the order of gh_read_topk) */
int gh_model_read_topk(gh_model* m, uint64_t k, uint32_t* idx, float* val, uint64_t* count);

/* ---- host sampling (sampling.rs:1-203, restated for the driver's generation loop) ----
 * The engine samples on the host after the device reduction; these mirror its filters
 * (repeat penalty -> temperature -> top-k -> top-p -> min-p -> inverse-CDF draw, FP32,
 * sequential sums) and its xorshift64* generator, so a seed reproduces the same draws. */
typedef struct gh_sampling { /* api/request.rs:13-20 */
    float temperature;    /* <= 0: greedy argmax */
    float top_p;          /* 1: off */
    uint32_t top_k;       /* 0: off */
    float min_p;          /* 0: off */
    float repeat_penalty; /* 1: off */
    uint64_t seed;
} gh_sampling;
/* sampling::plan (sampling.rs:165-192) */
#define GH_SAMPLE_GREEDY 0
#define GH_SAMPLE_TOPK 1
#define GH_SAMPLE_FALLBACK 2
#define GH_SAMPLE_MAX_DEVICE_K 128u /* sampling::MAX_DEVICE_K */
int gh_sampling_plan(const gh_sampling* p, uint32_t* k);
/* Rng::new / Rng::next_f32 (sampling.rs:15-36): the state after seeding; a uniform in [0, 1) */
uint64_t gh_rng_seed(uint64_t seed);
float gh_rng_next_f32(uint64_t* state);
/* sampling::sample over host logits (mutated in place by the penalty) */
int gh_sample(float* logits, uint64_t vocab, const gh_sampling* p, const uint32_t* recent,
              uint64_t n_recent, uint64_t* rng, uint32_t* token);
/* sampling::sample_from_candidates: candidates sorted by (scaled logit desc, index asc) */
int gh_sample_from_candidates(const uint32_t* idx, const float* logit, uint64_t n,
                              const gh_sampling* p, uint64_t* rng, uint32_t* token);
/* generation::drive (family/mistral/generation/mod.rs:75-148): prefill `prompt` at
 * positions 0.., then up to max_tokens tokens, each from the plan's path — device argmax
 * (greedy), device top-k + host tail (temperature and 0 < top_k <= 128, no penalty), or
 * full read-back + gh_sample (otherwise); stops at `eos` (UINT32_MAX: none) or the
 * context. Each decode step replays the captured decode graph. out receives *n_out tokens. */
int gh_model_generate(gh_model* m, const uint32_t* prompt, uint32_t n_prompt, const gh_sampling* p,
                      uint32_t max_tokens, uint32_t eos, uint32_t* out, uint32_t* n_out);

/* KV cache handle of the model's request (for parity checks of the cache contents) */
int gh_model_kv(gh_model* m, gh_kv* out);
/* the FP32 residual x of the last token processed (embedding_length floats) */
int gh_model_read_x(gh_model* m, float* dst);
/* the device handle of one loaded tensor (layer = UINT32_MAX for global tensors), e.g. to
 * time a single projection on the model's own resident weights */
int gh_model_weight(gh_model* m, uint32_t layer, uint32_t tensor, gh_buf* out);

/* ---- GGUF model files (host only; no device needed until gh_gguf_load_model) ----
 * The file is mapped read-only and parsed with bounds-checked reads; every tensor span is
 * validated against the file and the other spans at open (gguf/loader/mod.rs:44-186). On a
 * failure the status is negative and gh_gguf_last_error() (thread-local) holds the message. */
typedef struct gh_gguf gh_gguf;
typedef struct gh_gguf_tensor_info {
    const char* name;     /* valid until gh_gguf_close */
    uint32_t n_dims;      /* <= 4 */
    uint32_t type;        /* ggml type id (tensor_index.rs:36-54) */
    uint64_t dims[4];     /* GGUF order: dims[0] = in (row length), dims[1] = out */
    uint64_t offset;      /* relative to the data section */
    uint64_t nbytes;      /* from the ggml block layout (TensorInfo::byte_len) */
    const void* data;     /* the tensor bytes inside the mapping */
} gh_gguf_tensor_info;

const char* gh_gguf_last_error(void);
/* GgufFile::open, gguf/loader/mod.rs:44-123 */
int gh_gguf_open(const char* path, gh_gguf** out);
void gh_gguf_close(gh_gguf* g);
int gh_gguf_info(const gh_gguf* g, uint32_t* version, uint64_t* tensor_count, uint64_t* kv_count,
                 uint64_t* data_offset);
/* GgufFile::tensors / tensor_bytes, loader/mod.rs:133-143 */
int gh_gguf_tensor(const gh_gguf* g, uint64_t index, gh_gguf_tensor_info* out);
/* TensorIndex::get, tensor_index.rs:162-170 (duplicate names: the last one) */
int gh_gguf_find(const gh_gguf* g, const char* name, uint64_t* index);
/* metadata accessors (GgufValue::as_u64 / as_f32 / as_str, loader/value.rs:24-60) */
int gh_gguf_meta_u64(const gh_gguf* g, const char* key, uint64_t* out);
int gh_gguf_meta_f64(const gh_gguf* g, const char* key, double* out);
const char* gh_gguf_meta_str(const gh_gguf* g, const char* key);
int gh_gguf_meta_array_len(const gh_gguf* g, const char* key, uint64_t* out);
/* MistralConfig::from_metadata (family/mistral/config.rs:43-125) into a model config, with the
 * request's KV capacity (1..context_length) and prefill chunk rows */
int gh_gguf_model_config(const gh_gguf* g, uint32_t kv_context, uint32_t prefill_rows,
                         gh_model_config* cfg);
/* MistralTensors::build (family/mistral/tensors.rs:40-102): every tensor present with its
 * shape and an admitted type (F32 norms, Q4_K/Q6_K matrices) */
int gh_gguf_check_model(const gh_gguf* g, const gh_model_config* cfg);
/* load_weights (cpu/weights.rs:63-135): checks first, then uploads every tensor through
 * gh_model_load_tensor in the canonical order; a missing output.weight is the tied case
 * (the token table is uploaded as the output matrix as well) */
int gh_gguf_load_model(const gh_gguf* g, const gh_model_config* cfg, gh_model* m);

#ifdef __cplusplus
}
#endif
#endif

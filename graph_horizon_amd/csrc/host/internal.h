// Host-side internals of the gfx950 backend (C++17, HIP runtime API, no device code).
#ifndef GH_HOST_INTERNAL_H
#define GH_HOST_INTERNAL_H
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/gh_backend.h"
#include "../kernels/gh_kargs.h"

enum GhKernel : int {
    K_REPACK_Q4K,
    K_REPACK_Q6K,
    K_DEQUANT_Q4K,
    K_DEQUANT_Q6K,
    K_GEMV_Q4K_R1,
    K_GEMV_Q4K_R2,
    K_GEMV_Q6K_R1,
    K_GEMV_Q6K_R2,
    K_GEMV_MIXED_R2,
    K_GEMV_SWIGLU_R1,
    K_GEMV_SWIGLU_R2,
    // RMSNorm-staging variants (same order as the seven kernels they extend)
    K_GEMV_Q4K_R1_N,
    K_GEMV_Q4K_R2_N,
    K_GEMV_Q6K_R1_N,
    K_GEMV_Q6K_R2_N,
    K_GEMV_MIXED_R2_N,
    K_GEMV_SWIGLU_R1_N,
    K_GEMV_SWIGLU_R2_N,
    K_GEMV_Q4K_R2_NW,
    K_GEMV_Q6K_R2_NW,
    K_GEMV_MIXED_R2_NW,
    K_GEMV_SWIGLU_R2_NW,
    // direct-x variants (single token, one matrix, in_dim <= 4096, no RMSNorm)
    K_GEMV_Q4K_R1_D,
    K_GEMV_Q4K_R2_D,
    K_GEMV_Q6K_R1_D,
    K_GEMV_Q6K_R2_D,
    // split-K variants (single token, one matrix, 4096 < in_dim <= 16384, no RMSNorm)
    K_GEMV_Q4K_R1_K,
    K_GEMV_Q4K_R2_K,
    K_GEMV_Q6K_R1_K,
    K_GEMV_Q6K_R2_K,
    // three-wave split-K with four-row tasks (in_dim 12288 = 192 units: one unit per lane)
    K_GEMV_Q4K_R4_K3,
    K_GEMV_Q6K_R4_K3,
    K_RMSNORM,
    K_ROPE,
    K_SILU_MUL,
    K_RESIDUAL_ADD,
    K_KV_WRITE,
    K_ARGMAX_PARTIAL,
    K_ARGMAX_FINAL,
    K_ATTN_G1,
    K_ATTN_G2,
    K_ATTN_MFMA_G4,
    K_ATTN_MFMA_G8,
    K_ATTN_MFMA_G4_S16,
    // prefill GEMM tile variants (tokens x rows per workgroup), Q4_K then Q6_K
    K_GEMM_REDUCE,
    K_GEMM_TAIL,
    K_GEMM_REDUCE_SWIGLU,
    K_GEMM3_MIXED_R128,
    K_GEMM_REDUCE_SEG,
    K_ATTN_PREFILL_G4,
    K_ATTN_PREFILL_G4_R16,
    K_GEMM3_Q4K_R128,
    K_GEMM3_Q6K_R128,
    K_GEMM3_Q4K_R96,
    K_GEMM3_Q6K_R96,
    K_TOPK_PARTIAL,
    K_TOPK_FINAL,
    K_FILL_U32,
    K_STREAM_PROBE,
    K_DEQUANT_F16_Q4K,
    K_DEQUANT_F16_Q6K,
    K_GEMM4W_Q4K_R128,
    K_GEMM4W_Q6K_R128,
    K_GEMM4W_MIXED_R128,
    K_GEMM4W_Q4K_R96,
    K_GEMM4W_Q6K_R96,
    K_GEMM3_Q4K_R128_T128,
    K_GEMM3_Q6K_R128_T128,
    K_GEMM3_Q4K_R96_T128,
    K_GEMM3_Q6K_R96_T128,
    K_GEMM3_MIXED_R128_T128,
    // decode attention, XCD-local split merge (grid (xcds, splits, pair groups))
    K_ATTN_G1_X,
    K_ATTN_G2_X,
    K_ATTN_MFMA_G4_X,
    K_ATTN_MFMA_G8_X,
    K_ATTN_MFMA_G4_S16_X,
    K_XCD_PROBE,
    K_GEMM3_SWIGLU_R96_T128,
    K_GEMM3_SWIGLU_R128_T128,
    K_GEMM3_SWIGLU_R96,
    K_GEMM4W_SWIGLU_R96,
    K_GEMM3_SWIGLU_R128,
    K_GEMM4W_SWIGLU_R128,
    K_COUNT
};

// Device-resident YaRN rotation table: (cos, sin) per (position, pair) and the query
// post-scale per position, computed on the host with Yarn::pair's formula. The backend keeps
// one for the trait's rope ops (rebuilt when their YaRN parameters change); every model owns
// its own, built once at creation for its KV context, which its recorded graphs read.
constexpr uint32_t kMaxRopePositions = 262144;  // family/mistral/version.rs:16 MAX_CONTEXT
struct GhRopeTable {
    gh_yarn yarn{};
    uint32_t positions = 0;
    void* table = nullptr;  // float2 [positions][pairs]
    void* post = nullptr;   // float [positions]
};

struct gh_encoder {
    gh_backend* b = nullptr;
    int latched = GH_OK;
};

struct gh_backend {
    int device = 0;
    uint32_t cus = 0;  // compute units of the device
    hipStream_t stream = nullptr;
    std::vector<hipModule_t> modules;
    hipFunction_t fn[K_COUNT] = {};
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    gh_encoder enc;
    bool enc_open = false;
    bool capturing = false;  // a graph capture is recording on `stream`
    std::string err;
    // growable device workspace (attention partials, argmax partials)
    void* ws = nullptr;
    size_t ws_bytes = 0;
    void* counters = nullptr;  // attention merge counters, zero between launches
    size_t counter_slots = 0;
    GhRopeTable rope;  // the trait ops' table (gh_rope_yarn, gh_rope_yarn_batched)
    uint32_t attn_splits = 0;  // gh_set_attention_splits: 0 = attention_splits' policy
    // XCDs of the device when its dispatcher was seen to place workgroup i of every probed
    // launch on XCD i mod xcds (0: not seen; decode attention then merges its splits at agent
    // scope); attn_xcd_merge: the XCD-local merge is in use (gh_set_attention_xcd_merge)
    uint32_t xcds = 0;
    bool attn_xcd_merge = false;
    void* noalloc_scratch = nullptr;  // this device's copy of the no-allocation scratch array
    // FP16 copies of weights (gh_dequant_f16 layout), by the weight's device address: the
    // warp-specialized GEMMs read a registered copy instead of dequantizing (same values).
    // Registered and dropped by their owner (a model); gh_free_buffer of a weight drops its entry.
    std::unordered_map<uint64_t, uint64_t> w16;
    uint64_t gen = 0;  // bumped whenever the workspace or rope table moves (captured graphs hold them)
};

namespace gh {
// f32::total_cmp as a signed key: the bit pattern as i32, low 31 bits flipped when negative
inline int total_key(float f) {
    int32_t b;
    std::memcpy(&b, &f, 4);
    b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
    return b;
}

int fail(gh_backend* b, int code, const std::string& msg);
// 0 when enc is b's open encoder, else a latched GH_E_STATE
int check_enc(gh_backend* b, gh_encoder* enc);
// records an op's status in the encoder (reported again by gh_submit)
int latch(gh_encoder* enc, int rc);
int check_attention(gh_backend* b, const gh_buf* out, const gh_buf* q, const gh_kv* kv,
                    uint32_t q_heads, uint32_t last_pos, uint32_t rows, uint32_t layer);
// Resolves this device's address of the no-allocation scratch array (at gh_create).
int noalloc_init(gh_backend* b);
int hip_check(gh_backend* b, hipError_t e, const char* what);
int launch(gh_backend* b, GhKernel k, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx,
           const void* args, uint32_t shmem = 0);
int ensure_workspace(gh_backend* b, size_t bytes);
// Workgroups of `block` threads and `shmem` bytes of LDS resident on the whole device at once.
uint32_t resident_wgs(gh_backend* b, GhKernel k, uint32_t block, uint32_t shmem);
// Builds (or rebuilds, for other parameters or more positions) table t for `positions`
// positions (at most kMaxRopePositions).
int ensure_rope(gh_backend* b, GhRopeTable& t, const gh_yarn* y, uint32_t positions);
void free_rope(GhRopeTable& t);
bool yarn_valid(const gh_yarn* y);
// Graph-capturable op variants used by the model driver: positions/tokens read from device.
int op_rope(gh_backend* b, const GhRopeTable& t, const gh_buf* x, uint32_t heads,
            uint32_t head_dim, uint32_t base, uint32_t rows, uint32_t role, const void* pos_ptr);
int op_kv_write(gh_backend* b, const gh_kv* kv, const gh_buf* k, const gh_buf* v,
                uint64_t k_elem_off, uint64_t v_elem_off, uint32_t vectors, const void* pos_ptr);
// Caller-provided attention scratch: split partials and merge counters (zero on entry; every
// launch leaves them zero).
struct AttnScratch {
    char* parts;
    size_t part_bytes;
    void* counters;
    size_t counter_slots;
};
// fixed: use this scratch instead of the backend's growable workspace (GH_E_RANGE when the
// launch needs more than it holds).
int op_attention(gh_backend* b, const gh_buf* out, const gh_buf* q, const gh_kv* kv,
                 uint32_t q_heads, uint32_t base, uint32_t rows, uint32_t layer,
                 const void* pos_ptr, uint32_t max_pos, const AttnScratch* fixed = nullptr);
// w (Q4_K / Q6_K) dequantized to FP16 at out16 (rows x cols x 2 bytes) in the layout the GEMMs
// read registered copies in: row r, unit u (64 weights) at out16 + (r · cols / 64 + u) · 128.
int op_dequant_f16(gh_backend* b, const gh_buf* w, uint64_t out16);
int op_embed_rows(gh_backend* b, const gh_buf* x, const gh_buf* w, const void* tokens, uint32_t rows,
                  uint32_t embd);
int op_embed(gh_backend* b, const gh_buf* x, const gh_buf* w, uint32_t token, uint32_t embd,
             const void* token_ptr);
// step_scalars / step_history: also end a replayed greedy decode step (see GhArgmaxArgs)
int op_argmax(gh_backend* b, const gh_buf* logits, uint64_t vocab, void* out, void* out2,
              void* step_scalars = nullptr, void* step_history = nullptr);
// Decode GEMVs with fused epilogues (n = 1). Segments are launched as one grid.
struct GemvSeg {
    const gh_buf* w;
    uint64_t out;
    uint32_t epi;
};
// norm: x is the FP32 residual and rmsnorm_x(norm, eps) is applied while staging it
// (in_dim <= kFusedNormMaxDim).
constexpr uint32_t kFusedNormMaxDim = 5120;
// gh_view offsets and gh_min_buffer_offset_alignment: rows are read with 16-byte loads
constexpr uint64_t kMinViewAlignment = 16;
// rope: the table the RoPE epilogues read (required when a segment has one).
int op_gemv(gh_backend* b, const GemvSeg* segs, uint32_t nseg, const gh_buf* x, uint32_t n,
            uint32_t base, const void* pos_ptr, uint32_t head_dim, const gh_buf* up,
            const gh_buf* norm = nullptr, float eps = 0.0f, const GhRopeTable* rope = nullptr);
// Epilogue of a prefill GEMM (n >= 8 tokens). epi/aux: GH_GEMM_EPI_SILU with the FP16 gate
// (out = silu_mul(gate, f16(acc))). resid != 0: the output row is folded into the FP32 residual
// x[n][out_dim] (residual_add) and, with norm != 0, its RMSNorm written to normed — the bits of
// the separate reduce, residual_add and rmsnorm_x ops (out then only holds the FP16 projection).
// rope != nullptr: the output rows (query or key heads of head_dim) are rotated at positions
// base + t as op_rope does — in the split reduce, or by op_rope after an unsplit GEMM.
struct GemmEpi {
    uint32_t epi = GH_GEMM_EPI_F16;
    uint64_t aux = 0;
    uint64_t resid = 0, norm = 0, normed = 0;
    float eps = 0.0f;
};
int op_gemm(gh_backend* b, uint64_t out, const gh_buf* a, const gh_buf* w, uint32_t n,
            const GemmEpi* e = nullptr);
bool gemm_epi_applies(uint32_t n, uint32_t out_dim, bool tail);
// SwiGLU's gate and up projections of one FP16 input (n >= 8 tokens) and silu_mul, with one
// split reduce for both GEMMs where they split K; `gate` receives the gate's FP16 output only
// where they do not. The values of op_gemm(gate), op_gemm(up) and silu_mul.
int op_gemm_swiglu(gh_backend* b, const gh_buf* out, const gh_buf* gate, const gh_buf* a, const gh_buf* wg,
                   const gh_buf* wu, uint32_t n);
// gh_matmul_batched with an epilogue (checked buffers): gate != nullptr selects the SiLU
// epilogue; resid != nullptr the residual add, and norm/normed the RMSNorm after it.
int op_matmul_epi(gh_backend* b, const gh_buf* out, const gh_buf* a, const gh_buf* w, uint32_t in_dim,
                  uint32_t out_dim, uint32_t n, const gh_buf* gate, const gh_buf* resid,
                  const gh_buf* norm = nullptr, const gh_buf* normed = nullptr, float eps = 0.0f);
bool gemm_rope_applies(uint32_t n, uint32_t out_dim, uint32_t head_dim, const GhRopeTable& rope);
// Batches of more than 128 tokens run the GEMMs in 256-token tiles, over a registered FP16 copy
// of the weights (b->w16) where there is one; 128 tokens or fewer fit the 128-token tiles of
// the dequantizing kernels exactly, where a copy's four-fold weight stream costs more. Both
// forms of a batch size share one tile and split plan, so they give the same bits.
constexpr uint32_t kGemmTallTokens = 129;
// Several projections of one FP16 input (n >= 8 tokens) in one warp-specialized launch (row
// tiles of 128, each in its matrix's format) and one split reduce that writes each matrix's
// FP16 output and applies its RoPE role (GH_GEMM_ROLE_*; rows of head_dim, positions base + t)
// — the values of separate gh_matmul_batched launches and op_rope.
struct GemmSegSpec {
    const gh_buf* w;
    const gh_buf* out;
    uint32_t role;
};
bool gemm_multi_applies(uint32_t n);
int op_gemm_multi(gh_backend* b, const gh_buf* a, const GemmSegSpec* segs, uint32_t nseg, uint32_t n,
                  const GhRopeTable* rope, uint32_t base, uint32_t head_dim);
// gh_matmul_batched then op_rope(role, positions base + t) on its output, the rotation folded
// into the split reduce when the GEMM splits K (n >= 8 tokens, out_dim a multiple of head_dim).
size_t attention_workspace(uint32_t rows, uint32_t q_heads, uint32_t splits);
uint32_t attention_splits(const gh_backend* b, uint32_t max_len, uint32_t kv_heads, uint32_t rows);
int ensure_counters(gh_backend* b, size_t slots);
}  // namespace gh

#endif

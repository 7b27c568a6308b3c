// gfx950 backend: the C ABI of include/gh_backend.h over the HIP runtime.
// Kernels come from gfx950 code objects loaded with hipModuleLoad and are launched with
// hipModuleLaunchKernel on the backend's single stream.
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "internal.h"

namespace {

struct KernelName {
    GhKernel id;
    const char* name;
};

const KernelName kKernels[] = {
    {K_REPACK_Q4K, "gh_repack_q4k"},       {K_REPACK_Q6K, "gh_repack_q6k"},
    {K_DEQUANT_Q4K, "gh_dequant_q4k"},     {K_DEQUANT_Q6K, "gh_dequant_q6k"},
    {K_GEMV_Q4K_R1, "gh_gemv_q4k_r1"},     {K_GEMV_Q4K_R2, "gh_gemv_q4k_r2"},
    {K_GEMV_Q6K_R1, "gh_gemv_q6k_r1"},     {K_GEMV_Q6K_R2, "gh_gemv_q6k_r2"},
    {K_GEMV_MIXED_R2, "gh_gemv_mixed_r2"}, {K_GEMV_SWIGLU_R1, "gh_gemv_swiglu_r1"},
    {K_GEMV_SWIGLU_R2, "gh_gemv_swiglu_r2"},
    {K_GEMV_Q4K_R1_N, "gh_gemv_q4k_r1_n"}, {K_GEMV_Q4K_R2_N, "gh_gemv_q4k_r2_n"},
    {K_GEMV_Q6K_R1_N, "gh_gemv_q6k_r1_n"}, {K_GEMV_Q6K_R2_N, "gh_gemv_q6k_r2_n"},
    {K_GEMV_MIXED_R2_N, "gh_gemv_mixed_r2_n"},
    {K_GEMV_SWIGLU_R1_N, "gh_gemv_swiglu_r1_n"}, {K_GEMV_SWIGLU_R2_N, "gh_gemv_swiglu_r2_n"},
    {K_GEMV_Q4K_R2_NW, "gh_gemv_q4k_r2_nw"},     {K_GEMV_Q6K_R2_NW, "gh_gemv_q6k_r2_nw"},
    {K_GEMV_MIXED_R2_NW, "gh_gemv_mixed_r2_nw"}, {K_GEMV_SWIGLU_R2_NW, "gh_gemv_swiglu_r2_nw"},
    {K_GEMV_Q4K_R1_D, "gh_gemv_q4k_r1_d"}, {K_GEMV_Q4K_R2_D, "gh_gemv_q4k_r2_d"},
    {K_GEMV_Q6K_R1_D, "gh_gemv_q6k_r1_d"}, {K_GEMV_Q6K_R2_D, "gh_gemv_q6k_r2_d"},
    {K_GEMV_Q4K_R1_K, "gh_gemv_q4k_r1_k"}, {K_GEMV_Q4K_R2_K, "gh_gemv_q4k_r2_k"},
    {K_GEMV_Q6K_R1_K, "gh_gemv_q6k_r1_k"}, {K_GEMV_Q6K_R2_K, "gh_gemv_q6k_r2_k"},
    {K_GEMV_Q4K_R4_K3, "gh_gemv_q4k_r4_k3"}, {K_GEMV_Q6K_R4_K3, "gh_gemv_q6k_r4_k3"},
    {K_RMSNORM, "gh_rmsnorm_x"},           {K_ROPE, "gh_rope"},
    {K_SILU_MUL, "gh_silu_mul"},           {K_RESIDUAL_ADD, "gh_residual_add"},
    {K_KV_WRITE, "gh_kv_write"},           {K_ARGMAX_PARTIAL, "gh_argmax_partial"},
    {K_ARGMAX_FINAL, "gh_argmax_final"},   {K_ATTN_G1, "gh_attn_g1"},
    {K_ATTN_G2, "gh_attn_g2"},             {K_ATTN_MFMA_G4, "gh_attn_mfma_g4"},
    {K_ATTN_MFMA_G8, "gh_attn_mfma_g8"},   {K_ATTN_MFMA_G4_S16, "gh_attn_mfma_g4_s16"},

    {K_GEMM_REDUCE, "gh_gemm_reduce"},     {K_GEMM_TAIL, "gh_gemm_tail"},
    {K_GEMM_REDUCE_SWIGLU, "gh_gemm_reduce_swiglu"},
    {K_GEMM3_MIXED_R128, "gh_gemm3_mixed_r128"},
    {K_GEMM_REDUCE_SEG, "gh_gemm_reduce_seg"},     {K_ATTN_PREFILL_G4, "gh_attn_prefill_g4"},
    {K_ATTN_PREFILL_G4_R16, "gh_attn_prefill_g4_r16"},
    {K_GEMM3_Q4K_R128, "gh_gemm3_q4k_r128"},   {K_GEMM3_Q6K_R128, "gh_gemm3_q6k_r128"},
    {K_GEMM3_Q4K_R96, "gh_gemm3_q4k_r96"},     {K_GEMM3_Q6K_R96, "gh_gemm3_q6k_r96"},
    {K_TOPK_PARTIAL, "gh_topk_partial"},       {K_TOPK_FINAL, "gh_topk_final"},
    {K_FILL_U32, "gh_fill_u32"},           {K_STREAM_PROBE, "gh_stream_probe"},
    {K_DEQUANT_F16_Q4K, "gh_dequant_f16_q4k"}, {K_DEQUANT_F16_Q6K, "gh_dequant_f16_q6k"},
    {K_GEMM4W_Q4K_R128, "gh_gemm4w_q4k_r128"}, {K_GEMM4W_Q6K_R128, "gh_gemm4w_q6k_r128"},
    {K_GEMM4W_MIXED_R128, "gh_gemm4w_mixed_r128"},
    {K_GEMM4W_Q4K_R96, "gh_gemm4w_q4k_r96"},   {K_GEMM4W_Q6K_R96, "gh_gemm4w_q6k_r96"},
    {K_GEMM3_Q4K_R128_T128, "gh_gemm3_q4k_r128_t128"}, {K_GEMM3_Q6K_R128_T128, "gh_gemm3_q6k_r128_t128"},
    {K_GEMM3_Q4K_R96_T128, "gh_gemm3_q4k_r96_t128"},   {K_GEMM3_Q6K_R96_T128, "gh_gemm3_q6k_r96_t128"},
    {K_GEMM3_MIXED_R128_T128, "gh_gemm3_mixed_r128_t128"},
    {K_ATTN_G1_X, "gh_attn_g1_x"},             {K_ATTN_G2_X, "gh_attn_g2_x"},
    {K_ATTN_MFMA_G4_X, "gh_attn_mfma_g4_x"},   {K_ATTN_MFMA_G8_X, "gh_attn_mfma_g8_x"},
    {K_ATTN_MFMA_G4_S16_X, "gh_attn_mfma_g4_s16_x"},
    {K_XCD_PROBE, "gh_xcd_probe"},
    {K_GEMM3_SWIGLU_R96_T128, "gh_gemm3_swiglu_r96_t128"}, {K_GEMM3_SWIGLU_R128_T128, "gh_gemm3_swiglu_r128_t128"},
    {K_GEMM3_SWIGLU_R96, "gh_gemm3_swiglu_r96"},           {K_GEMM4W_SWIGLU_R96, "gh_gemm4w_swiglu_r96"},
    {K_GEMM3_SWIGLU_R128, "gh_gemm3_swiglu_r128"},         {K_GEMM4W_SWIGLU_R128, "gh_gemm4w_swiglu_r128"},
};

const char* kModules[] = {"gh_quant", "gh_gemv", "gh_glue", "gh_attention", "gh_gemm"};

constexpr uint32_t kArgmaxBlocks = 256;
// argmax scratch at the front of the workspace: f32[256] values, u32[256] indices, u32 result
constexpr size_t kArgmaxBytes = 256 * 4 * 2 + 256;

std::string library_dir() {
    Dl_info info{};
    if (dladdr((void*)&gh_create, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t s = p.find_last_of('/');
        return s == std::string::npos ? std::string(".") : p.substr(0, s);
    }
    return ".";
}

inline uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

bool is_weight(const gh_buf* w) {
    return w && w->kind == GH_BUF_WEIGHT && (w->format == GH_FMT_Q4_K || w->format == GH_FMT_Q6_K);
}

bool fits(const gh_buf* buf, uint64_t bytes) { return buf && buf->addr && buf->bytes >= bytes; }

// Yarn::pair / post_scale (backend/rope.rs:60-133) evaluated on the host in FP32 with the same
// libm calls, so the device rotation table holds the reference's values.
constexpr float kPi = 3.14159265358979323846f;
float corr_dim(uint32_t rope_dim, uint32_t original_context, float rotations, float base) {
    float denom = rotations * 2.0f * kPi;
    return (float)rope_dim * std::log((float)original_context / denom) / (2.0f * std::log(base));
}
void yarn_pair(const gh_yarn* y, uint32_t pair, uint32_t position, float* c, float* s) {
    float freq_scale = 1.0f / y->factor;
    float theta_extrap =
        (float)position * std::pow(y->freq_base, -(2.0f * (float)pair) / (float)y->rope_dim);
    float theta_interp = freq_scale * theta_extrap;
    float start = std::fmax(
        std::floor(corr_dim(y->rope_dim, y->original_context, y->beta_fast, y->freq_base)), 0.0f);
    float end =
        std::fmin(std::ceil(corr_dim(y->rope_dim, y->original_context, y->beta_slow, y->freq_base)),
                  (float)(y->rope_dim - 1));
    float yv = ((float)pair - start) / std::fmax(end - start, 0.001f);
    float cl = yv < 0.0f ? 0.0f : (yv > 1.0f ? 1.0f : yv);
    float ramp = 1.0f - cl;
    float theta = theta_interp * (1.0f - ramp) + theta_extrap * ramp;
    *c = std::cos(theta) * 1.0f;
    *s = std::sin(theta) * 1.0f;
}
float yarn_post_query(const gh_yarn* y, uint32_t position) {
    float bucket = (float)(position / y->original_context);
    return std::log(bucket + 1.0f) * y->q_temperature_scale + 1.0f;
}

// IEEE binary32 -> binary16, round to nearest even (overflow to infinity, NaN stays NaN).
uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to >= 65520
    if (ax < 0x38800000u) {  // result is subnormal (or zero) in binary16
        if (ax < 0x33000000u) return (uint16_t)sign;  // below half the smallest subnormal
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - (ax >> 23);  // 14 + (112 - e) with e the f32 exponent
        const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        return (uint16_t)(sign | (q + (rem > halfway || (rem == halfway && (q & 1)))));
    }
    const uint32_t q = (ax - 0x38000000u) >> 13, rem = ax & 0x1FFFu;
    return (uint16_t)(sign | (q + (rem > 0x1000u || (rem == 0x1000u && (q & 1)))));
}

}  // namespace

namespace gh {

int fail(gh_backend* b, int code, const std::string& msg) {
    if (b) b->err = msg;
    return code;
}

int check_enc(gh_backend* b, gh_encoder* enc) {
    if (!b) return GH_E_INVALID;
    if (!enc || enc != &b->enc || !b->enc_open) return fail(b, GH_E_STATE, "no open encoder");
    return GH_OK;
}

int latch(gh_encoder* enc, int rc) {
    if (rc != GH_OK && enc && enc->latched == GH_OK) enc->latched = rc;
    return rc;
}

int hip_check(gh_backend* b, hipError_t e, const char* what) {
    if (e == hipSuccess) return GH_OK;
    return fail(b, e == hipErrorOutOfMemory ? GH_E_OOM : GH_E_HIP,
                std::string(what) + ": " + hipGetErrorString(e));
}

int launch(gh_backend* b, GhKernel k, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx,
           const void* args, uint32_t shmem) {
    if (gx == 0 || gy == 0 || gz == 0) return GH_OK;
    void* params[] = {const_cast<void*>(args)};
    return hip_check(b, hipModuleLaunchKernel(b->fn[k], gx, gy, gz, bx, 1, 1, shmem, b->stream,
                                              params, nullptr),
                     "hipModuleLaunchKernel");
}

int ensure_workspace(gh_backend* b, size_t bytes) {
    bytes += kArgmaxBytes;
    if (b->ws_bytes >= bytes) return GH_OK;
    if (b->capturing) return fail(b, GH_E_STATE, "workspace growth during graph capture");
    int rc = hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (rc) return rc;
    if (b->ws) (void)hipFree(b->ws);
    b->ws = nullptr;
    b->ws_bytes = 0;
    size_t want = std::max(bytes, (size_t)(4u << 20));
    rc = hip_check(b, hipMalloc(&b->ws, want), "hipMalloc(workspace)");
    if (rc) return rc;
    b->ws_bytes = want;
    ++b->gen;
    return GH_OK;
}

bool yarn_valid(const gh_yarn* y) {
    if (!y || y->rope_dim == 0 || y->rope_dim % 2 != 0 || y->original_context == 0) return false;
    const float v[6] = {y->freq_base, y->factor,         y->beta_fast,
                        y->beta_slow, y->log_multiplier, y->q_temperature_scale};
    for (float x : v)
        if (!std::isfinite(x) || x <= 0.0f) return false;
    return true;
}

void free_rope(GhRopeTable& t) {
    if (t.table) (void)hipFree(t.table);
    if (t.post) (void)hipFree(t.post);
    t.table = t.post = nullptr;
    t.positions = 0;
}

int ensure_rope(gh_backend* b, GhRopeTable& t, const gh_yarn* y, uint32_t positions) {
    if (positions > kMaxRopePositions)
        return fail(b, GH_E_RANGE, "rope: position beyond the table limit (262144 positions)");
    bool same = t.table && std::memcmp(&t.yarn, y, sizeof(gh_yarn)) == 0;
    if (same && t.positions >= positions) return GH_OK;
    if (b->capturing) return fail(b, GH_E_STATE, "rope table growth during graph capture");
    uint32_t n = std::min(std::max<uint32_t>(positions, 4096), kMaxRopePositions);
    if (same) n = std::min(std::max(n, t.positions * 2), kMaxRopePositions);
    const uint32_t pairs = y->rope_dim / 2;
    std::vector<float> table((size_t)n * pairs * 2), post(n);
    for (uint32_t p = 0; p < n; ++p) {
        for (uint32_t j = 0; j < pairs; ++j)
            yarn_pair(y, j, p, &table[((size_t)p * pairs + j) * 2], &table[((size_t)p * pairs + j) * 2 + 1]);
        post[p] = yarn_post_query(y, p);
    }
    int rc = hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (rc) return rc;
    free_rope(t);
    rc = hip_check(b, hipMalloc(&t.table, table.size() * 4), "hipMalloc(rope)");
    if (!rc) rc = hip_check(b, hipMalloc(&t.post, post.size() * 4), "hipMalloc(rope)");
    if (!rc) rc = hip_check(b, hipMemcpy(t.table, table.data(), table.size() * 4, hipMemcpyHostToDevice), "hipMemcpy(rope)");
    if (!rc) rc = hip_check(b, hipMemcpy(t.post, post.data(), post.size() * 4, hipMemcpyHostToDevice), "hipMemcpy(rope)");
    if (rc) {
        free_rope(t);
        return rc;
    }
    t.yarn = *y;
    t.positions = n;
    return GH_OK;
}

int op_rope(gh_backend* b, const GhRopeTable& t, const gh_buf* x, uint32_t heads,
            uint32_t head_dim, uint32_t base, uint32_t rows, uint32_t role, const void* pos_ptr) {
    if (!t.table) return fail(b, GH_E_STATE, "rope: table not built");
    GhRopeArgs a{};
    a.x = x->addr;
    a.table = (uint64_t)t.table;
    a.post = role == GH_ROPE_QUERY ? (uint64_t)t.post : 0;
    a.pos_ptr = (uint64_t)pos_ptr;
    a.heads = heads;
    a.head_dim = head_dim;
    a.pairs = t.yarn.rope_dim / 2;
    a.base = base;
    a.rows = rows;
    uint64_t total = (uint64_t)rows * heads * a.pairs;
    return launch(b, K_ROPE, ceil_div(total, 256), 1, 1, 256, &a);
}

int op_kv_write(gh_backend* b, const gh_kv* kv, const gh_buf* k, const gh_buf* v,
                uint64_t k_elem_off, uint64_t v_elem_off, uint32_t vectors, const void* pos_ptr) {
    GhKvWriteArgs a{};
    a.kc = kv->k.addr;
    a.vc = kv->v.addr;
    a.k = k->addr;
    a.v = v->addr;
    a.pos_ptr = (uint64_t)pos_ptr;
    a.k_off = k_elem_off;
    a.v_off = v_elem_off;
    a.k_count = vectors * kv->head_dim;
    a.v_count = vectors * kv->value_dim;
    a.k_stride = kv->kv_heads * kv->head_dim;
    a.v_stride = kv->kv_heads * kv->value_dim;
    return launch(b, K_KV_WRITE, ceil_div(std::max(a.k_count, a.v_count), 256), 1, 1, 256, &a);
}

// Workgroups per (row, kv head): enough that rows x kv heads x splits covers about two
// workgroups per CU, at most one per 64-position chunk and at most 32 (the merge's limit);
// longer contexts loop over chunks. (Eight-wave workgroups over 128-position chunks measured
// 35.5 vs 37.1 us at ctx 32768 but 613 vs 625 tok/s on the 8B decode: not kept.)
// gh_set_attention_splits replaces the policy's count (still capped by chunks and 32).
uint32_t attention_splits(const gh_backend* b, uint32_t max_len, uint32_t kv_heads, uint32_t rows) {
    const uint32_t chunks = ceil_div(max_len, 64);
    const uint32_t want = b->attn_splits ? b->attn_splits
                                         : ceil_div(2 * std::max(b->cus, 1u), std::max(kv_heads * rows, 1u));
    return std::max<uint32_t>(1, std::min<uint32_t>({want, chunks, 32u}));
}

size_t attention_workspace(uint32_t rows, uint32_t q_heads, uint32_t splits) {
    size_t n = (size_t)rows * q_heads * splits;
    return n * 4 * 2 + n * 128 * 4 + 1024;
}

int ensure_counters(gh_backend* b, size_t slots) {
    if (b->counter_slots >= slots) return GH_OK;
    if (b->capturing) return fail(b, GH_E_STATE, "counter growth during graph capture");
    slots = std::max<size_t>(slots, 4096);
    int rc = hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (rc) return rc;
    if (b->counters) (void)hipFree(b->counters);
    b->counters = nullptr;
    b->counter_slots = 0;
    rc = hip_check(b, hipMalloc(&b->counters, slots * 4), "hipMalloc(counters)");
    // on the (non-blocking) backend stream, so the clear is ordered before every launch
    if (!rc) rc = hip_check(b, hipMemsetAsync(b->counters, 0, slots * 4, b->stream), "hipMemsetAsync(counters)");
    if (rc) return rc;
    b->counter_slots = slots;
    ++b->gen;
    return GH_OK;
}

// Causal GQA attention for `rows` query rows at positions base + r (+ *pos_ptr);
// max_pos bounds the positions the launch can see (sizes the split grid).
constexpr uint32_t kAttnPrefillMinRows = 32;

int op_attention(gh_backend* b, const gh_buf* out, const gh_buf* q, const gh_kv* kv,
                 uint32_t q_heads, uint32_t base, uint32_t rows, uint32_t layer,
                 const void* pos_ptr, uint32_t max_pos, const AttnScratch* fixed) {
    const uint32_t group = q_heads / kv->kv_heads;
    // the XCD-local split merge when the start-up probe confirmed the dispatch rule it needs
    const bool xl = b->attn_xcd_merge && b->xcds != 0;
    GhKernel k;
    switch (group) {
        case 1: k = xl ? K_ATTN_G1_X : K_ATTN_G1; break;
        case 2: k = xl ? K_ATTN_G2_X : K_ATTN_G2; break;
        // four or eight query heads per kv head: the matrix-core decode (the K and value dims
        // are 128, which check_attention and the model enforce)
        case 4: k = xl ? K_ATTN_MFMA_G4_X : K_ATTN_MFMA_G4; break;
        case 8: k = xl ? K_ATTN_MFMA_G8_X : K_ATTN_MFMA_G8; break;
        default: return fail(b, GH_E_UNSUPPORTED, "attention: GQA group must be 1, 2, 4 or 8");
    }
    // Batched prefill on the matrix cores: 32-row query blocks x kv heads (G = 4, head 128).
    if (!pos_ptr && rows >= kAttnPrefillMinRows && group == 4 && kv->head_dim == 128 &&
        kv->value_dim == 128) {
        GhAttnArgs a{};
        a.q = q->addr;
        a.kc = kv->k.addr;
        a.vc = kv->v.addr;
        a.out = out->addr;
        a.key_dim = kv->head_dim;
        a.value_dim = kv->value_dim;
        a.kv_heads = kv->kv_heads;
        a.q_heads = q_heads;
        a.layer = layer;
        a.context = kv->context;
        a.base = base;
        a.rows = rows;
        a.scale = 1.0f / std::sqrt((float)kv->head_dim);
        // 32 query rows per workgroup (K/V tiles shared by twice the rows of 16-row blocks;
        // 248 VGPRs keep two workgroups resident per CU), 16 when 32-row blocks would leave
        // CUs without a workgroup
        if ((uint64_t)ceil_div(rows, 32) * kv->kv_heads < b->cus)
            return launch(b, K_ATTN_PREFILL_G4_R16, ceil_div(rows, 16), kv->kv_heads, 1, 256, &a);
        return launch(b, K_ATTN_PREFILL_G4, ceil_div(rows, 32), kv->kv_heads, 1, 256, &a);
    }
    // decode reads a layer's K/V through 32-bit buffer ranges
    if (((uint64_t)kv->context + 2048) * kv->kv_heads * kv->head_dim * 2 >= (1ull << 31))
        return fail(b, GH_E_UNSUPPORTED, "attention: a layer's K or V cache of 2 GiB or more");
    const uint32_t splits = attention_splits(b, max_pos + 1, kv->kv_heads, rows);
    // the merge of a launch of at most 16 splits reads 16 slots (same bits, half the loads)
    if (k == K_ATTN_MFMA_G4 && splits <= 16) k = K_ATTN_MFMA_G4_S16;
    if (k == K_ATTN_MFMA_G4_X && splits <= 16) k = K_ATTN_MFMA_G4_S16_X;
    // the kernels take the head counts and the launch's rows as 16-bit fields
    if (q_heads > 0xFFFFu || kv->kv_heads > 0xFFFFu)
        return fail(b, GH_E_UNSUPPORTED, "attention: more than 65535 heads");
    char* ws = nullptr;
    void* counters = nullptr;
    uint32_t group_rows = rows;
    int rc = GH_OK;
    if (fixed) {
        if (attention_workspace(rows, q_heads, splits) > fixed->part_bytes ||
            (size_t)rows * kv->kv_heads > fixed->counter_slots)
            return fail(b, GH_E_RANGE, "attention: launch needs more scratch than the caller's");
        ws = fixed->parts;
        counters = fixed->counters;
    } else {
        // bound the partials: rows in groups that fit a 256 MiB workspace
        const size_t per_row = attention_workspace(1, q_heads, splits);
        group_rows = (uint32_t)std::max<size_t>(1, ((size_t)256 << 20) / per_row);
        group_rows = std::min({group_rows, rows, 0xFFFFu});
        rc = ensure_workspace(b, attention_workspace(group_rows, q_heads, splits));
        if (!rc) rc = ensure_counters(b, (size_t)group_rows * kv->kv_heads);
        if (rc) return rc;
        ws = (char*)b->ws + kArgmaxBytes;
        counters = b->counters;
    }
    for (uint32_t r0 = 0; r0 < rows; r0 += group_rows) {
        const uint32_t nr = std::min(group_rows, rows - r0);
        const size_t n = (size_t)nr * q_heads * splits;
        GhAttnArgs a{};
        a.q = q->addr + (uint64_t)r0 * q_heads * kv->head_dim * 2;
        a.kc = kv->k.addr;
        a.vc = kv->v.addr;
        a.out = out->addr + (uint64_t)r0 * q_heads * kv->value_dim * 2;
        a.part_m = (uint64_t)ws;
        a.part_l = (uint64_t)(ws + n * 4);
        a.part_acc = (uint64_t)(ws + n * 8);
        a.pos_ptr = (uint64_t)pos_ptr;
        a.counters = (uint64_t)counters;
        a.key_dim = kv->head_dim;
        a.value_dim = kv->value_dim;
        a.kv_heads = kv->kv_heads;
        a.q_heads = q_heads;
        a.layer = layer;
        a.context = kv->context;
        a.base = base + r0;
        a.rows = nr;
        a.splits = splits;
        a.scale = 1.0f / std::sqrt((float)kv->head_dim);
        // leading scalar parameters (preloaded into SGPRs), then the full arguments
        uint32_t heads = q_heads | kv->kv_heads << 16, shape = nr | (xl ? b->xcds : 0u) << 16;
        void* params[] = {&a.q, &a.kc, &a.vc, &a.pos_ptr, &a.layer, &a.context, &heads, &shape, &a};
        // XL: workgroup (x, split, z) serves the (row, kv head) pair z·xcds + x, so all splits of
        // a pair share workgroup ids modulo xcds, i.e. one XCD
        const uint32_t gx = xl ? b->xcds : splits, gy = xl ? splits : kv->kv_heads,
                       gz = xl ? ceil_div(nr * kv->kv_heads, b->xcds) : nr;
        rc = hip_check(b, hipModuleLaunchKernel(b->fn[k], gx, gy, gz, 256, 1, 1, 0, b->stream, params, nullptr),
                       "hipModuleLaunchKernel");
        if (rc) return rc;
    }
    return GH_OK;
}

int check_attention(gh_backend* b, const gh_buf* out, const gh_buf* q, const gh_kv* kv,
                    uint32_t q_heads, uint32_t last_pos, uint32_t rows, uint32_t layer) {
    if (!kv || kv->scheme != GH_KV_F16) return fail(b, GH_E_UNSUPPORTED, "attention: only the f16 KV scheme");
    if (kv->head_dim != 128 || kv->value_dim != 128) return fail(b, GH_E_UNSUPPORTED, "attention: head_dim 128 only");
    if (kv->kv_heads == 0 || q_heads % kv->kv_heads) return fail(b, GH_E_INVALID, "attention: q_heads not a multiple of kv_heads");
    if (layer >= kv->block_count || last_pos >= kv->context) return fail(b, GH_E_RANGE, "attention: position beyond context");
    const uint64_t cache = (uint64_t)kv->block_count * kv->context * kv->kv_heads * 128 * 2;
    if (!fits(&kv->k, cache) || !fits(&kv->v, cache)) return fail(b, GH_E_RANGE, "attention: cache too small");
    if (!fits(q, (uint64_t)rows * q_heads * 256) || !fits(out, (uint64_t)rows * q_heads * 256))
        return fail(b, GH_E_RANGE, "attention: buffer too small");
    return GH_OK;
}

int op_embed(gh_backend* b, const gh_buf* x, const gh_buf* w, uint32_t token, uint32_t embd,
             const void* token_ptr) {
    GhDequantArgs a{};
    a.w = w->addr;
    a.out = x->addr;
    a.row_ptr = (uint64_t)token_ptr;
    a.wrows = w->rows;
    a.nb = embd / 256;
    a.row0 = token;
    a.rows = 1;
    return launch(b, w->format == GH_FMT_Q4_K ? K_DEQUANT_Q4K : K_DEQUANT_Q6K,
                  ceil_div(embd, 256), 1, 1, 256, &a);
}

// Embedding rows of a token list already on the device (u32[rows]): one launch for a whole
// prefill chunk, row r of x = dequantized row tokens[r] (the same values as op_embed per row).
int op_embed_rows(gh_backend* b, const gh_buf* x, const gh_buf* w, const void* tokens, uint32_t rows,
                  uint32_t embd) {
    if (!is_weight(w) || w->cols != embd) return fail(b, GH_E_UNSUPPORTED, "embed: token_embd must be a Q4_K/Q6_K weight of width embd");
    if (!fits(x, (uint64_t)rows * embd * 4)) return fail(b, GH_E_RANGE, "embed: x too small");
    GhDequantArgs a{};
    a.w = w->addr;
    a.out = x->addr;
    a.row_list = (uint64_t)tokens;
    a.wrows = w->rows;
    a.nb = embd / 256;
    a.rows = rows;
    return launch(b, w->format == GH_FMT_Q4_K ? K_DEQUANT_Q4K : K_DEQUANT_Q6K,
                  (uint32_t)ceil_div((uint64_t)rows * embd, (uint64_t)256), 1, 1, 256, &a);
}

int op_argmax(gh_backend* b, const gh_buf* logits, uint64_t vocab, void* out, void* out2,
              void* step_scalars, void* step_history) {
    int rc = ensure_workspace(b, 0);
    if (rc) return rc;
    GhArgmaxArgs a{};
    a.logits = logits->addr;
    a.part_v = (uint64_t)b->ws;
    a.part_i = (uint64_t)((char*)b->ws + 1024);
    a.out = out ? (uint64_t)out : (uint64_t)((char*)b->ws + 2048);
    a.out2 = (uint64_t)out2;
    a.step_scalars = (uint64_t)step_scalars;
    a.step_history = (uint64_t)step_history;
    a.n = (uint32_t)vocab;
    a.blocks = std::min<uint32_t>(kArgmaxBlocks, ceil_div(vocab, 256));
    rc = launch(b, K_ARGMAX_PARTIAL, a.blocks, 1, 1, 256, &a);
    if (!rc) rc = launch(b, K_ARGMAX_FINAL, 1, 1, 1, 256, &a);
    return rc;
}

// Rows per wavefront task: two from 4096 rows, one below (more tasks to fill the machine).
static uint32_t gemv_rows(uint64_t total_rows) { return total_rows >= 4096 ? 2 : 1; }

uint32_t resident_wgs(gh_backend* b, GhKernel k, uint32_t block, uint32_t shmem) {
    int n = 0;
    if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, b->fn[k], (int)block, shmem) != hipSuccess || n < 1)
        n = 1;
    return (uint32_t)n * b->cus;
}

int op_gemv(gh_backend* b, const GemvSeg* segs, uint32_t nseg, const gh_buf* x, uint32_t n,
            uint32_t base, const void* pos_ptr, uint32_t head_dim, const gh_buf* up,
            const gh_buf* norm, float eps, const GhRopeTable* rt) {
    if (nseg == 0 || nseg > 3) return fail(b, GH_E_INVALID, "gemv: 1..3 segments");
    GhGemvArgs a{};
    const uint32_t in_dim = segs[0].w->cols;
    bool mixed = false, rope = false, swiglu = false;
    uint64_t total_rows = 0;
    for (uint32_t i = 0; i < nseg; ++i) {
        const gh_buf* w = segs[i].w;
        if (!is_weight(w) || w->cols != in_dim) return fail(b, GH_E_INVALID, "gemv: segment shape");
        mixed |= w->format != segs[0].w->format;
        rope |= segs[i].epi == GH_EPI_ROPE || segs[i].epi == GH_EPI_ROPE_CACHE;
        swiglu |= segs[i].epi == GH_EPI_SWIGLU;
        total_rows += w->rows;
    }
    if (n > 1)
        for (uint32_t i = 0; i < nseg; ++i)
            if (segs[i].epi != GH_EPI_F16 && segs[i].epi != GH_EPI_F32)
                return fail(b, GH_E_INVALID, "gemv: fused epilogues are single-token");
    uint32_t r = gemv_rows(total_rows);
    if (rope || mixed) r = 2;  // RoPE needs row pairs; the mixed kernel is compiled for R = 2
    if (norm) r = std::min<uint32_t>(r, 2);  // the RMSNorm variants exist for R = 1, 2
    GhKernel k;
    if (swiglu) {
        if (nseg != 1 || !up || up->format != GH_FMT_Q4_K || segs[0].w->format != GH_FMT_Q4_K ||
            up->rows != segs[0].w->rows || up->cols != in_dim)
            return fail(b, GH_E_INVALID, "gemv: SwiGLU needs Q4_K gate/up of one shape");
        k = r == 2 ? K_GEMV_SWIGLU_R2 : K_GEMV_SWIGLU_R1;
        a.aux = up->addr;
    } else if (mixed) {
        k = K_GEMV_MIXED_R2;
    } else if (segs[0].w->format == GH_FMT_Q4_K) {
        k = r == 2 ? K_GEMV_Q4K_R2 : K_GEMV_Q4K_R1;
    } else {
        k = r == 2 ? K_GEMV_Q6K_R2 : K_GEMV_Q6K_R1;
    }
    const bool direct = !norm && n == 1 && nseg == 1 && !swiglu && in_dim <= 4096;
    // direct launches of 8192 rows or more take one-row tasks (more waves in flight: 12288x4096
    // Q4_K measured 6.84 us against 7.21 us with two-row tasks; 4096x4096 stays at two rows,
    // 4.01 us against 4.16 us with one-row tasks)
    if (direct && total_rows >= 8192 && (k == K_GEMV_Q4K_R2 || k == K_GEMV_Q6K_R2)) {
        k = k == K_GEMV_Q4K_R2 ? K_GEMV_Q4K_R1 : K_GEMV_Q6K_R1;
        r = 1;
    }
    if (direct) {
        switch (k) {
            case K_GEMV_Q4K_R1: k = K_GEMV_Q4K_R1_D; break;
            case K_GEMV_Q4K_R2: k = K_GEMV_Q4K_R2_D; break;
            case K_GEMV_Q6K_R1: k = K_GEMV_Q6K_R1_D; break;
            case K_GEMV_Q6K_R2: k = K_GEMV_Q6K_R2_D; break;
            default: break;
        }
    }
    const bool splitk = !norm && n == 1 && nseg == 1 && !swiglu && in_dim > 4096 && in_dim <= 16384;
    // in_dim 12288 (192 units) splits over three waves, one unit per lane, four rows per task
    // (the 8B FFN down: 1,024 tasks, one round at three waves per SIMD). Measured on the 8B
    // decode: 607 tok/s, against 599 with two-row tasks and 596 with the four-wave kernels.
    // (Four-row tasks for in_dim 16384, four waves, measured neutral on the 14B decode: 374.2
    // vs 374.0 tok/s.)
    uint32_t block = 256;
    if (splitk && in_dim / 64 == 192 && r >= 2) {
        r = 4;
        k = segs[0].w->format == GH_FMT_Q4_K ? K_GEMV_Q4K_R4_K3 : K_GEMV_Q6K_R4_K3;
        block = 192;
    } else if (splitk) {
        switch (k) {
            case K_GEMV_Q4K_R1: k = K_GEMV_Q4K_R1_K; break;
            case K_GEMV_Q4K_R2: k = K_GEMV_Q4K_R2_K; break;
            case K_GEMV_Q6K_R1: k = K_GEMV_Q6K_R1_K; break;
            case K_GEMV_Q6K_R2: k = K_GEMV_Q6K_R2_K; break;
            default: break;
        }
    }
    if (norm) {
        switch (k) {
            case K_GEMV_Q4K_R1: k = K_GEMV_Q4K_R1_N; break;
            case K_GEMV_Q4K_R2: k = K_GEMV_Q4K_R2_N; break;
            case K_GEMV_Q6K_R1: k = K_GEMV_Q6K_R1_N; break;
            case K_GEMV_Q6K_R2: k = K_GEMV_Q6K_R2_N; break;
            case K_GEMV_MIXED_R2: k = K_GEMV_MIXED_R2_N; break;
            case K_GEMV_SWIGLU_R1: k = K_GEMV_SWIGLU_R1_N; break;
            case K_GEMV_SWIGLU_R2: k = K_GEMV_SWIGLU_R2_N; break;
            default: return fail(b, GH_E_UNSUPPORTED, "gemv: no RMSNorm variant");
        }
        // rows of 65-128 units: both chunks of a task requested at once (same bits)
        const uint32_t units = in_dim / 64;
        if (units > 64 && units <= 128) {
            switch (k) {
                case K_GEMV_Q4K_R2_N: k = K_GEMV_Q4K_R2_NW; break;
                case K_GEMV_Q6K_R2_N: k = K_GEMV_Q6K_R2_NW; break;
                case K_GEMV_MIXED_R2_N: k = K_GEMV_MIXED_R2_NW; break;
                case K_GEMV_SWIGLU_R2_N: k = K_GEMV_SWIGLU_R2_NW; break;
                default: break;
            }
        }
    }
    uint32_t task = 0;
    for (uint32_t i = 0; i < nseg; ++i) {
        a.seg[i].w = segs[i].w->addr;
        a.seg[i].out = segs[i].out;
        a.seg[i].rows = segs[i].w->rows;
        a.seg[i].fmt = segs[i].w->format;
        a.seg[i].epi = segs[i].epi;
        a.seg[i].task0 = task;
        task += ceil_div(segs[i].w->rows, r);
    }
    a.x = x->addr;
    if (norm) {
        if (n != 1) return fail(b, GH_E_INVALID, "gemv: fused norm is single-token");
        if (norm->format != GH_FMT_F16 || norm->bytes < (uint64_t)in_dim * 2 || in_dim % 8 || in_dim > kFusedNormMaxDim)
            return fail(b, GH_E_INVALID, "gemv: fused norm needs an F16[in_dim] weight and in_dim <= 5120");
        a.norm_w = norm->addr;
        a.eps = eps;
    }
    if (rope && (!rt || !rt->table)) return fail(b, GH_E_STATE, "gemv: RoPE table not built");
    a.table = rt ? (uint64_t)rt->table : 0;
    a.post = rt ? (uint64_t)rt->post : 0;
    a.pos_ptr = (uint64_t)pos_ptr;
    a.in_dim = in_dim;
    a.nseg = nseg;
    a.n = n;
    a.base = base;
    a.pairs = rt ? rt->yarn.rope_dim / 2 : 0;
    a.head_dim = head_dim;
    a.tasks = task;
    if (in_dim / 64 > 256) return fail(b, GH_E_UNSUPPORTED, "gemv: in_dim above 16384");
    // x staged once per workgroup in LDS (144 B per 64-weight unit; both layouts if mixed);
    // the persistent grid (at most what is resident at once) loops its waves over the tasks.
    // + the normalized FP16 row and 16 bytes of reduction scratch when RMSNorm is fused
    uint32_t shmem = (in_dim / 64) * 144 * (mixed ? 2 : 1) + (norm ? in_dim * 2 + 16 : 0);
    if (direct || splitk) shmem = 0;
    if (direct) block = 64 * GH_DIRECT_WAVES;
    const uint32_t cap = resident_wgs(b, k, block, shmem);
    // split-K: one task per workgroup (its waves share it); otherwise one per wave
    const uint32_t want = splitk ? task : ceil_div(task, block / 64);
    a.groups = std::max<uint32_t>(1, std::min<uint32_t>(want, cap));
    // the kernels' leading scalar parameters (preloaded into SGPRs), then the full arguments
    void* params[] = {&a.x, &a.seg[0].w, &a.norm_w, &a.in_dim, &a.seg[0].rows, &a.tasks, &a.groups, &a};
    return hip_check(b, hipModuleLaunchKernel(b->fn[k], a.groups, 1, 1, block, 1, 1, shmem, b->stream, params, nullptr),
                     "hipModuleLaunchKernel");
}


}  // namespace gh

using namespace gh;

extern "C" {

// The XCD count when the dispatcher places workgroup i of a launch on XCD i mod n, else 0.
// Four launches record each workgroup's XCD (gh_xcd_probe): a 1-D grid of 16384 workgroups
// (more than the device holds at once; n = the XCDs seen), then grids of the XCD-local
// attention's form (n, splits, groups), whose workgroups must share the XCD of their x.
uint32_t probe_xcds(gh_backend* b) {
    constexpr uint32_t kWgs = 16384;
    void* d = nullptr;
    if (hipMalloc(&d, kWgs * 4) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    std::vector<uint32_t> h(kWgs);
    uint32_t n = 0;
    bool ok = true;
    const uint32_t shapes[4][3] = {{kWgs, 1, 1}, {0, 9, 1}, {0, 32, 4}, {0, 3, 7}};
    for (int pass = 0; pass < 4 && ok; ++pass) {
        const uint32_t gx = pass ? n : shapes[0][0], gy = shapes[pass][1], gz = shapes[pass][2];
        const uint32_t total = gx * gy * gz;
        uint64_t out = (uint64_t)d;
        uint32_t px = gx, py = gy;
        void* params[] = {&out, &px, &py};
        ok = hipModuleLaunchKernel(b->fn[K_XCD_PROBE], gx, gy, gz, 64, 1, 1, 0, b->stream, params, nullptr) ==
                 hipSuccess &&
             hipMemcpyAsync(h.data(), d, (size_t)total * 4, hipMemcpyDeviceToHost, b->stream) == hipSuccess &&
             hipStreamSynchronize(b->stream) == hipSuccess;
        if (!ok) break;
        if (pass == 0) {
            std::vector<uint32_t> seen;
            for (uint32_t i = 0; i < total && seen.size() <= 16; ++i)
                if (std::find(seen.begin(), seen.end(), h[i]) == seen.end()) seen.push_back(h[i]);
            n = (uint32_t)seen.size();
            ok = n >= 1 && n <= 16;
        }
        // distinct XCDs for x = 0 .. n-1, and every workgroup on the XCD of its x
        for (uint32_t i = 0; ok && i < n; ++i)
            for (uint32_t j = 0; ok && j < i; ++j) ok = h[i] != h[j];
        for (uint32_t i = 0; ok && i < total; ++i) ok = h[i] == h[i % gx % n];
    }
    (void)hipGetLastError();
    (void)hipFree(d);
    return ok ? n : 0;
}

int gh_create(const gh_config* cfg, gh_backend** out) {
    if (!out) return GH_E_INVALID;
    *out = nullptr;
    int dev = cfg ? cfg->device : 0;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= dev || dev < 0) return GH_E_NO_DEVICE;
    hipDeviceProp_t prop{};
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return GH_E_NO_DEVICE;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return GH_E_NO_DEVICE;
    if (hipSetDevice(dev) != hipSuccess) return GH_E_NO_DEVICE;
    auto* b = new gh_backend();
    b->device = dev;
    b->cus = (uint32_t)std::max(1, prop.multiProcessorCount);
    b->enc.b = b;
    int rc = hip_check(b, hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking), "hipStreamCreate");
    if (!rc) rc = hip_check(b, hipEventCreate(&b->ev_start), "hipEventCreate");
    if (!rc) rc = hip_check(b, hipEventCreate(&b->ev_stop), "hipEventCreate");
    std::string dir = cfg && cfg->code_object_path ? std::string(cfg->code_object_path) : library_dir();
    for (const char* m : kModules) {
        if (rc) break;
        hipModule_t mod = nullptr;
        std::string path = dir + "/" + m + "_gfx950.co";
        if (hipModuleLoad(&mod, path.c_str()) != hipSuccess) {
            rc = fail(b, GH_E_MODULE, "hipModuleLoad failed: " + path);
            break;
        }
        b->modules.push_back(mod);
    }
    for (const KernelName& kn : kKernels) {
        if (rc) break;
        hipFunction_t f = nullptr;
        for (hipModule_t mod : b->modules)
            if (hipModuleGetFunction(&f, mod, kn.name) == hipSuccess) break;
        if (!f) rc = fail(b, GH_E_MODULE, std::string("kernel not found: ") + kn.name);
        b->fn[kn.id] = f;
    }
    // the lookups in modules that do not hold a kernel leave hipErrorNotFound as the thread's
    // last error, which another HIP user in the process (a framework that checks
    // hipGetLastError after its own calls) would take for its own failure
    (void)hipGetLastError();
    if (!rc) rc = ensure_workspace(b, 0);
    if (!rc) rc = noalloc_init(b);
    if (!rc) {
        b->xcds = probe_xcds(b);
        b->attn_xcd_merge = b->xcds != 0;
    }
    if (rc) {
        gh_destroy(b);
        return rc;
    }
    *out = b;
    return GH_OK;
}

void gh_destroy(gh_backend* b) {
    if (!b) return;
    if (b->stream) (void)hipStreamSynchronize(b->stream);
    if (b->ws) (void)hipFree(b->ws);
    if (b->counters) (void)hipFree(b->counters);
    free_rope(b->rope);
    for (hipModule_t m : b->modules) (void)hipModuleUnload(m);
    if (b->ev_start) (void)hipEventDestroy(b->ev_start);
    if (b->ev_stop) (void)hipEventDestroy(b->ev_stop);
    if (b->stream) (void)hipStreamDestroy(b->stream);
    delete b;
}

const char* gh_last_error(const gh_backend* b) { return b ? b->err.c_str() : "no backend"; }

int gh_alloc_buffer(gh_backend* b, uint64_t bytes, gh_buf* out) {
    if (!b || !out || bytes == 0) return fail(b, GH_E_INVALID, "alloc: zero size");
    void* p = nullptr;
    int rc = hip_check(b, hipMalloc(&p, bytes), "hipMalloc");
    if (rc) return rc;
    *out = gh_buf{(uint64_t)p, bytes, GH_FMT_F16, GH_BUF_ALLOC, 0, 0};
    return GH_OK;
}

int gh_free_buffer(gh_backend* b, gh_buf* buf) {
    if (!b || !buf) return GH_E_INVALID;
    if (buf->kind != GH_BUF_ALLOC && buf->kind != GH_BUF_WEIGHT)
        return fail(b, GH_E_INVALID, "free_buffer: a view never owns its storage");
    int rc = hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (!rc) rc = hip_check(b, hipFree((void*)buf->addr), "hipFree");
    if (buf->kind == GH_BUF_WEIGHT) b->w16.erase(buf->addr);  // its FP16 copy no longer applies
    *buf = gh_buf{};
    return rc;
}

int gh_view(gh_backend* b, const gh_buf* buf, uint64_t off, uint64_t len, gh_buf* out) {
    if (!b || !buf || !out) return GH_E_INVALID;
    if (buf->kind == GH_BUF_WEIGHT) return fail(b, GH_E_INVALID, "view of a packed weight");
    if (off > buf->bytes || len > buf->bytes - off) return fail(b, GH_E_RANGE, "view beyond buffer");
    if (off % kMinViewAlignment) return fail(b, GH_E_INVALID, "view offset not 16-byte aligned");
    *out = gh_buf{buf->addr + off, len, buf->format, GH_BUF_VIEW, 0, 0};
    return GH_OK;
}

// The kernels read activation rows with 16-byte vector loads and LDS DMA, so views start on
// 16-byte boundaries (every Mistral row stride is a multiple of 512 bytes).
uint64_t gh_min_buffer_offset_alignment(const gh_backend*) { return kMinViewAlignment; }

int gh_upload(gh_backend* b, const gh_buf* dst, uint64_t off, const void* src, uint64_t len) {
    if (!b || !dst || (!src && len)) return GH_E_INVALID;
    if (off > dst->bytes || len > dst->bytes - off) return fail(b, GH_E_RANGE, "upload beyond buffer");
    if (len == 0) return GH_OK;
    int rc = hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (rc) return rc;
    return hip_check(b, hipMemcpy((void*)(dst->addr + off), src, len, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

int gh_download(gh_backend* b, const gh_buf* src, uint64_t off, void* dst, uint64_t len) {
    if (!b || !src || (!dst && len)) return GH_E_INVALID;
    if (off > src->bytes || len > src->bytes - off) return fail(b, GH_E_RANGE, "download beyond buffer");
    if (len == 0) return GH_OK;
    int rc = hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (rc) return rc;
    return hip_check(b, hipMemcpy(dst, (const void*)(src->addr + off), len, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

int gh_load_weight(gh_backend* b, uint32_t format, const void* bytes, uint64_t len,
                   uint32_t in_dim, uint32_t out_dim, gh_buf* out) {
    if (!b || !bytes || !out || in_dim == 0 || out_dim == 0) return fail(b, GH_E_INVALID, "load_weight: bad argument");
    *out = gh_buf{};
    if (format == GH_FMT_F32 || format == GH_FMT_F16) {
        const uint64_t n = (uint64_t)in_dim * out_dim;
        if (len != n * (format == GH_FMT_F32 ? 4 : 2)) return fail(b, GH_E_INVALID, "load_weight: length mismatch");
        std::vector<uint16_t> h(n);
        if (format == GH_FMT_F32) {
            // cpu/weights.rs:151-174: F32 norms are narrowed RNE to F16 at load
            const float* f = (const float*)bytes;
            for (uint64_t i = 0; i < n; ++i) h[i] = f32_to_f16_rne(f[i]);
        } else {
            std::memcpy(h.data(), bytes, len);
        }
        gh_buf buf;
        int rc = gh_alloc_buffer(b, n * 2, &buf);
        if (rc) return rc;
        rc = gh_upload(b, &buf, 0, h.data(), n * 2);
        if (rc) {
            gh_free_buffer(b, &buf);
            return rc;
        }
        buf.format = GH_FMT_F16;
        buf.rows = out_dim;
        buf.cols = in_dim;
        *out = buf;
        return GH_OK;
    }
    if (format != GH_FMT_Q4_K && format != GH_FMT_Q6_K)
        return fail(b, GH_E_UNSUPPORTED, "load_weight: format outside the Q4_K_M profile");
    if (in_dim % 256 != 0) return fail(b, GH_E_INVALID, "load_weight: in_dim not a multiple of 256");
    const uint64_t bl = format == GH_FMT_Q4_K ? 144 : 210;
    const uint64_t nb = in_dim / 256;
    if (len % bl != 0 || len != (uint64_t)out_dim * nb * bl)
        return fail(b, GH_E_INVALID, "load_weight: malformed quantized weight (not whole blocks of the shape)");
    void* staging = nullptr;
    void* dst = nullptr;
    int rc = hip_check(b, hipMalloc(&staging, len), "hipMalloc(staging)");
    if (!rc) rc = hip_check(b, hipMalloc(&dst, len), "hipMalloc(weight)");
    if (!rc) rc = hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (!rc) rc = hip_check(b, hipMemcpy(staging, bytes, len, hipMemcpyHostToDevice), "hipMemcpy(weight)");
    if (!rc) {
        GhRepackArgs a{(uint64_t)staging, (uint64_t)dst, out_dim, (uint32_t)nb};
        uint64_t threads = format == GH_FMT_Q4_K ? (uint64_t)out_dim * nb * 9 : len;
        rc = launch(b, format == GH_FMT_Q4_K ? K_REPACK_Q4K : K_REPACK_Q6K, ceil_div(threads, 256), 1, 1, 256, &a);
    }
    if (!rc) rc = hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (staging) (void)hipFree(staging);
    if (rc) {
        if (dst) (void)hipFree(dst);
        return rc;
    }
    *out = gh_buf{(uint64_t)dst, len, format, GH_BUF_WEIGHT, out_dim, in_dim};
    return GH_OK;
}

int gh_dequant_rows(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* w,
                    uint32_t row0, uint32_t rows) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (!is_weight(w)) return latch(enc, fail(b, GH_E_INVALID, "dequant: not a quantized weight"));
    if ((uint64_t)row0 + rows > w->rows) return latch(enc, fail(b, GH_E_RANGE, "dequant: rows beyond weight"));
    if (!fits(out, (uint64_t)rows * w->cols * 4)) return latch(enc, fail(b, GH_E_RANGE, "dequant: output too small"));
    GhDequantArgs a{};
    a.w = w->addr;
    a.out = out->addr;
    a.wrows = w->rows;
    a.nb = w->cols / 256;
    a.row0 = row0;
    a.rows = rows;
    return latch(enc, launch(b, w->format == GH_FMT_Q4_K ? K_DEQUANT_Q4K : K_DEQUANT_Q6K,
                             ceil_div((uint64_t)rows * w->cols, 256), 1, 1, 256, &a));
}

int gh_begin(gh_backend* b, gh_encoder** enc) {
    if (!b || !enc) return GH_E_INVALID;
    if (b->enc_open) return fail(b, GH_E_STATE, "begin: encoder already open");
    b->enc_open = true;
    b->enc.latched = GH_OK;
    *enc = &b->enc;
    return GH_OK;
}

int gh_submit(gh_backend* b, gh_encoder* enc) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    b->enc_open = false;
    rc = hip_check(b, hipStreamSynchronize(b->stream), "submit");
    return enc->latched != GH_OK ? enc->latched : rc;
}

void gh_no_barrier(gh_backend*) {}

int gh_kv_write(gh_backend* b, gh_encoder* enc, const gh_kv* kv, const gh_buf* k,
                const gh_buf* v, uint64_t k_payload_offset, uint64_t v_payload_offset,
                uint64_t, uint64_t, uint32_t vectors) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (!kv || !k || !v) return latch(enc, fail(b, GH_E_INVALID, "kv_write: null"));
    if (kv->scheme != GH_KV_F16) return latch(enc, fail(b, GH_E_UNSUPPORTED, "kv_write: only the f16 scheme"));
    const uint64_t kb = (uint64_t)vectors * kv->head_dim * 2, vb = (uint64_t)vectors * kv->value_dim * 2;
    if (!fits(k, kb) || !fits(v, vb) || k_payload_offset % 2 || v_payload_offset % 2 ||
        k_payload_offset > kv->k.bytes || kb > kv->k.bytes - k_payload_offset ||
        v_payload_offset > kv->v.bytes || vb > kv->v.bytes - v_payload_offset)
        return latch(enc, fail(b, GH_E_RANGE, "kv_write: beyond cache"));
    return latch(enc, op_kv_write(b, kv, k, v, k_payload_offset / 2, v_payload_offset / 2, vectors, nullptr));
}

int gh_embed(gh_backend* b, gh_encoder* enc, const gh_buf* x, const gh_buf* w, uint32_t token,
             uint32_t embd) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (!is_weight(w) || w->cols != embd) return latch(enc, fail(b, GH_E_UNSUPPORTED, "embed: token_embd must be a Q4_K/Q6_K weight of width embd"));
    if (token >= w->rows) return latch(enc, fail(b, GH_E_RANGE, "embed: token beyond vocabulary"));
    if (!fits(x, (uint64_t)embd * 4)) return latch(enc, fail(b, GH_E_RANGE, "embed: x too small"));
    return latch(enc, op_embed(b, x, w, token, embd, nullptr));
}

}  // extern "C"

namespace gh {

// Matrix-core GEMM for n >= kGemmMinTokens: the warp-specialized kernels (512-thread
// workgroups of 256 tokens, or 128 below 256 tokens, x 128 or 96 rows), over FP16 weight
// copies where registered; K splits over the units when the tiles alone would leave CUs idle.
constexpr uint32_t kGemmMinTokens = 8;
constexpr uint32_t kGemmTailMaxRows = 8192;  // gh_gemm_tail: two 16-value items per thread

// The launch plan of one GEMM: kernel, row and token tiles, and K splits (every split
// non-empty); w16 is the registered FP16 copy of w that the kernel reads instead (0: none).
struct GemmPlan {
    GhKernel k;
    uint32_t tr, tt, splits;
    uint64_t w16;
};

// Threads per workgroup of a prefill GEMM kernel: the dequantizing 256-token tiles and the
// 128-row 128-token tiles run eight consumer and four producer waves, every other form eight
// waves.
static uint32_t gemm_block(GhKernel k) {
    switch (k) {
        case K_GEMM3_Q4K_R96:
        case K_GEMM3_Q6K_R96:
        case K_GEMM3_Q4K_R128:
        case K_GEMM3_Q6K_R128:
        case K_GEMM3_MIXED_R128:
        case K_GEMM3_Q4K_R128_T128:
        case K_GEMM3_Q6K_R128_T128:
        case K_GEMM3_MIXED_R128_T128: return 768;
        default: return 512;
    }
}

static GemmPlan plan_gemm(gh_backend* b, const gh_buf* w, uint32_t n) {
    const uint32_t rows = w->rows, units = w->cols / 64;
    // Batches of 128 tokens or fewer take 128-token tiles (kGemmTallTokens).
    const bool tall = n >= kGemmTallTokens;
    // splits: at most 16, and at least 8 units of 64 k per split (12 in the 128-token tiles,
    // where a workgroup's fixed costs weigh more: 4096 x 4096 at 128 tokens in 96-row tiles x 5
    // splits 22.2 us against 26.0 in 128-row tiles x 8 splits of 8 units)
    const uint32_t min_units = tall ? 8u : 12u;
    auto clamp_splits = [&](uint32_t s) {
        return std::max<uint32_t>(1, std::min<uint32_t>({s, std::max<uint32_t>(1, units / min_units), 16u}));
    };
    const bool q4 = w->format == GH_FMT_Q4_K;
    // Row height (measured at 512 tokens on the 8B and 14B shapes): one workgroup per CU,
    // s = CUs / tiles splits (clamped as above), and the height whose tiles x splits fill the
    // CUs' last wave better — 96 rows for 12288 x 4096 (256 tiles against 192 of 128 rows),
    // 128 rows otherwise. Narrow outputs (<= 1024 rows) take 96 rows with two workgroups per
    // CU and up to 16 splits: their few units per split leave latency for a second to hide.
    const uint32_t tt = ceil_div(n, tall ? 256u : 128u), cus = b->cus;
    // a registered FP16 copy of w: the same sums with the weights copied, not dequantized
    const auto copy = b->w16.find(w->addr);
    const uint64_t w16 = copy == b->w16.end() || !tall ? 0 : copy->second;
    auto fill = [&](uint32_t br) {
        const uint32_t t = ceil_div(rows, br) * tt, s = clamp_splits(std::max<uint32_t>(1, cus / t));
        const uint64_t ts = (uint64_t)t * s;
        return (double)ts / ((double)cus * (double)ceil_div(ts, cus));
    };
    const bool narrow = rows <= 1024;
    const uint32_t br = narrow || fill(96) > fill(128) ? 96u : 128u;
    GhKernel k = br == 96 ? (q4 ? K_GEMM3_Q4K_R96 : K_GEMM3_Q6K_R96) : (q4 ? K_GEMM3_Q4K_R128 : K_GEMM3_Q6K_R128);
    if (!tall)
        k = br == 96 ? (q4 ? K_GEMM3_Q4K_R96_T128 : K_GEMM3_Q6K_R96_T128)
                     : (q4 ? K_GEMM3_Q4K_R128_T128 : K_GEMM3_Q6K_R128_T128);
    if (w16)
        k = br == 96 ? (q4 ? K_GEMM4W_Q4K_R96 : K_GEMM4W_Q6K_R96) : (q4 ? K_GEMM4W_Q4K_R128 : K_GEMM4W_Q6K_R128);
    const uint32_t tr = ceil_div(rows, br), tiles = tr * tt;
    const uint32_t slots = narrow ? resident_wgs(b, k, gemm_block(k), 0) : cus;
    uint32_t splits = clamp_splits(std::max<uint32_t>(1, slots / tiles));
    // the kernels give split z the units [z per, min(units, (z + 1) per)), per = whole blocks
    // (gh_gemm_split_units): shrink splits to ceil(units / per) until every split is non-empty
    for (;;) {
        const uint32_t per = gh_gemm_split_units(units, splits), s = ceil_div(units, per);
        if (s == splits) break;
        splits = s;
    }
    return GemmPlan{k, tr, tt, splits, w16};
}

// The GEMM kernel of plan p alone; with p.splits > 1 its FP32 partials [splits][n][rows] go to
// `part` (which holds p.splits * n * rows floats).
static int gemm_kernel(gh_backend* b, const GemmPlan& p, uint64_t out, uint64_t part, const gh_buf* a,
                       const gh_buf* w, uint32_t n, uint32_t epi = GH_GEMM_EPI_F16, uint64_t aux = 0) {
    GhGemmArgs ga{};
    ga.x = a->addr;
    ga.w = p.w16 ? p.w16 : w->addr;
    ga.out = out;
    ga.part = part;
    ga.in_dim = w->cols;
    ga.rows = w->rows;
    ga.n = n;
    ga.splits = p.splits;
    ga.epi = epi;
    ga.aux = aux;
    return launch(b, p.k, p.tr, p.tt, p.splits, gemm_block(p.k), &ga);
}

// One GEMM launch over its plan's tiles and K splits; with splits > 1 the kernel writes FP32
// partials to the workspace and gh_gemm_reduce sums them in split order. `e` adds the SiLU
// epilogue (in the GEMM or the reduce) or replaces the reduce by gh_gemm_tail (residual add
// and RMSNorm of each output row).
int op_gemm(gh_backend* b, uint64_t out, const gh_buf* a, const gh_buf* w, uint32_t n, const GemmEpi* e) {
    const GemmPlan p = plan_gemm(b, w, n);
    const bool tail = e && e->resid;
    const uint32_t epi = e && !tail ? e->epi : GH_GEMM_EPI_F16;
    const uint64_t aux = e && !tail ? e->aux : 0;
    uint64_t part = 0;
    if (p.splits > 1) {
        int rc = ensure_workspace(b, (size_t)p.splits * n * w->rows * 4);
        if (rc) return rc;
        part = (uint64_t)((char*)b->ws + kArgmaxBytes);
    }
    int rc = gemm_kernel(b, p, out, part, a, w, n, epi, aux);
    if (rc) return rc;
    GhGemmArgs ga{};
    ga.out = out;
    ga.part = part;
    ga.rows = w->rows;
    ga.n = n;
    ga.splits = p.splits;
    if (tail) {
        ga.aux = e->resid;
        ga.norm = e->norm;
        ga.normed = e->normed;
        ga.eps = e->eps;
        return launch(b, K_GEMM_TAIL, n, 1, 1, 1024, &ga);
    }
    if (p.splits == 1) return GH_OK;
    ga.epi = epi;
    ga.aux = aux;
    const uint64_t total = (uint64_t)n * w->rows;
    return launch(b, K_GEMM_REDUCE, (uint32_t)std::min<uint64_t>(ceil_div(total, (uint64_t)256), 4096), 1, 1,
                  256, &ga);
}

// SwiGLU's two projections of one input: out = silu_mul(f16(x wg^T), f16(x wu^T)). Where the
// GEMMs split K, both write their partials and one reduce (gh_gemm_reduce_swiglu) rounds each
// sum to FP16 and applies silu_mul; otherwise the up GEMM applies it in its epilogue to the
// gate's FP16 output in `gate`. The values of op_gemm(gate), op_gemm(up) and silu_mul.
int op_gemm_swiglu(gh_backend* b, const gh_buf* out, const gh_buf* gate, const gh_buf* a, const gh_buf* wg,
                   const gh_buf* wu, uint32_t n) {
    if (!is_weight(wg) || !is_weight(wu) || wg->rows != wu->rows || wg->cols != wu->cols)
        return fail(b, GH_E_INVALID, "gemm swiglu: gate and up of one shape");
    if (n < kGemmMinTokens) return fail(b, GH_E_UNSUPPORTED, "gemm swiglu: GEMM path only");
    const uint64_t cells = (uint64_t)n * wg->rows;
    if (!fits(a, (uint64_t)n * wg->cols * 2) || !fits(out, cells * 2) || !fits(gate, cells * 2))
        return fail(b, GH_E_RANGE, "gemm swiglu: buffer too small");
    // 8-128 tokens, Q4_K gate and up whose row pairs fill at most one wave of workgroups: one
    // launch of 96-row tiles (48 gate rows + the same 48 up rows) or, where those would be more
    // than the CUs, 128-row tiles (64 + 64, eight consumers), K unsplit, silu_mul in the
    // epilogue — no FP32 partials or split reduce (8B 128 x 4096 -> 2 x 12288: 256 tiles of
    // 96; 14B 128 x 5120 -> 2 x 16384: 256 tiles of 128)
    const bool pair96 = ceil_div(wg->rows, 48u) <= b->cus;
    const uint32_t pair_tiles = ceil_div(wg->rows, pair96 ? 48u : 64u);
    if (n < kGemmTallTokens && wg->format == GH_FMT_Q4_K && wu->format == GH_FMT_Q4_K && pair_tiles <= b->cus) {
        GhGemmArgs ga{};
        ga.x = a->addr;
        ga.w = wg->addr;
        ga.aux = wu->addr;
        ga.out = out->addr;
        ga.in_dim = wg->cols;
        ga.rows = wg->rows;
        ga.n = n;
        ga.splits = 1;
        return launch(b, pair96 ? K_GEMM3_SWIGLU_R96_T128 : K_GEMM3_SWIGLU_R128_T128, pair_tiles, ceil_div(n, 128u),
                      1, pair96 ? 512 : 768, &ga);
    }
    // Longer chunks whose separate GEMMs run K unsplit: the same pairs in 256-token tiles of the
    // separate launches' height (96 rows: 8B at 256-1024 tokens; 128 rows where the fill rule
    // picks them: 8B at 2048, 14B), so each sum is the separate launch's, over the FP16 copies
    // when both weights have one (8B 512-token prefill 11.73 -> 11.56-11.65 ms, same box; 96-row
    // pairs where the separate launches take 128 rows measured 34.6 -> 36.4 ms at 2048)
    const GemmPlan pg = plan_gemm(b, wg, n), pu = plan_gemm(b, wu, n);
    const bool r96 = pg.k == K_GEMM4W_Q4K_R96 || pg.k == K_GEMM3_Q4K_R96;
    const bool r128 = pg.k == K_GEMM4W_Q4K_R128 || pg.k == K_GEMM3_Q4K_R128;
    // Where the separate launches split K (8B at 129-255 tokens: 128 tiles x 2 splits and a
    // split reduce), 96-row pairs unsplit instead when they fill the CUs in one pass, at least
    // half of them: the 128-token tiles' trade, in 256-token tiles
    const uint32_t tt = ceil_div(n, 256u), p96 = ceil_div(wg->rows, 48u) * tt, p128 = ceil_div(wg->rows, 64u) * tt;
    const bool fits96 = p96 <= b->cus && 2 * p96 >= b->cus, fits128 = p128 <= b->cus && 2 * p128 >= b->cus;
    const bool split_pairs = pg.splits > 1 && (fits96 || fits128);  // 128-row pairs: 14B, 256 tiles
    if (n >= kGemmTallTokens && wg->format == GH_FMT_Q4_K && wu->format == GH_FMT_Q4_K &&
        ((pg.splits == 1 && pu.splits == 1 && (r96 || r128) && pu.k == pg.k) || split_pairs)) {
        const auto cg = b->w16.find(wg->addr), cu = b->w16.find(wu->addr);
        const bool copies = cg != b->w16.end() && cu != b->w16.end();
        GhGemmArgs ga{};
        ga.x = a->addr;
        ga.w = copies ? cg->second : wg->addr;
        ga.aux = copies ? cu->second : wu->addr;
        ga.out = out->addr;
        ga.in_dim = wg->cols;
        ga.rows = wg->rows;
        ga.n = n;
        ga.splits = 1;
        const bool p96t = split_pairs ? fits96 : r96;
        const GhKernel k = p96t ? (copies ? K_GEMM4W_SWIGLU_R96 : K_GEMM3_SWIGLU_R96)
                                : (copies ? K_GEMM4W_SWIGLU_R128 : K_GEMM3_SWIGLU_R128);
        return launch(b, k, ceil_div(wg->rows, p96t ? 48u : 64u), tt, 1, copies ? 512 : 768, &ga);
    }
    if (pg.splits == 1 || pu.splits != pg.splits || wg->rows % 4) {
        GemmEpi e;
        e.epi = GH_GEMM_EPI_SILU;
        e.aux = gate->addr;
        int rc = op_gemm(b, gate->addr, a, wg, n);
        return rc ? rc : op_gemm(b, out->addr, a, wu, n, &e);
    }
    const size_t half = (size_t)pg.splits * cells * 4;
    int rc = ensure_workspace(b, 2 * half);
    if (rc) return rc;
    const uint64_t part = (uint64_t)((char*)b->ws + kArgmaxBytes);
    rc = gemm_kernel(b, pg, 0, part, a, wg, n);
    if (!rc) rc = gemm_kernel(b, pu, 0, part + half, a, wu, n);
    if (rc) return rc;
    GhGemmArgs ga{};
    ga.out = out->addr;
    ga.part = part;
    ga.rows = wg->rows;
    ga.n = n;
    ga.splits = pg.splits;
    return launch(b, K_GEMM_REDUCE_SWIGLU, (uint32_t)std::min<uint64_t>(ceil_div(cells / 4, (uint64_t)256), 4096), 1,
                  1, 256, &ga);
}

// The SiLU epilogue and the tail apply to every GEMM (n >= kGemmMinTokens).
bool gemm_epi_applies(uint32_t n, uint32_t out_dim, bool tail) {
    return n >= kGemmMinTokens && (!tail || (out_dim % 4 == 0 && out_dim <= kGemmTailMaxRows));
}

int op_matmul_epi(gh_backend* b, const gh_buf* out, const gh_buf* a, const gh_buf* w, uint32_t in_dim,
                  uint32_t out_dim, uint32_t n, const gh_buf* gate, const gh_buf* resid,
                  const gh_buf* norm, const gh_buf* normed, float eps) {
    const bool tail = resid != nullptr;
    if ((gate != nullptr) == tail || (norm != nullptr) != (normed != nullptr) || (norm && !tail))
        return fail(b, GH_E_INVALID, "matmul epilogue: SiLU, or residual (+ norm)");
    if (!gemm_epi_applies(n, out_dim, tail)) return fail(b, GH_E_UNSUPPORTED, "matmul epilogue: GEMM path only");
    if (!is_weight(w)) return fail(b, GH_E_UNSUPPORTED, "matmul: weight must be Q4_K or Q6_K");
    if (w->cols != in_dim || w->rows != out_dim) return fail(b, GH_E_INVALID, "matmul: weight shape mismatch");
    const uint64_t cells = (uint64_t)n * out_dim;
    if (!fits(a, (uint64_t)n * in_dim * 2) || !fits(out, cells * 2) || (gate && !fits(gate, cells * 2)) ||
        (tail && !fits(resid, cells * 4)) || (norm && (!fits(norm, (uint64_t)out_dim * 2) || !fits(normed, cells * 2))))
        return fail(b, GH_E_RANGE, "matmul epilogue: buffer too small");
    GemmEpi e;
    if (gate) {
        e.epi = GH_GEMM_EPI_SILU;
        e.aux = gate->addr;
    } else {
        e.resid = resid->addr;
        e.norm = norm ? norm->addr : 0;
        e.normed = normed ? normed->addr : 0;
        e.eps = eps;
    }
    return op_gemm(b, out->addr, a, w, n, &e);
}

bool gemm_multi_applies(uint32_t n) { return n >= kGemmMinTokens; }

int op_gemm_multi(gh_backend* b, const gh_buf* a, const GemmSegSpec* segs, uint32_t nseg, uint32_t n,
                  const GhRopeTable* rope, uint32_t base, uint32_t head_dim) {
    constexpr uint32_t BR = 128;
    if (nseg == 0 || nseg > 3 || !gemm_multi_applies(n)) return fail(b, GH_E_UNSUPPORTED, "gemm multi: 1..3 matrices, n >= 8");
    const uint32_t in_dim = segs[0].w->cols;
    GhGemmArgs ga{};
    uint32_t tiles = 0, total = 0;
    bool any_rope = false;
    for (uint32_t i = 0; i < nseg; ++i) {
        const gh_buf* w = segs[i].w;
        if (!is_weight(w) || w->cols != in_dim || w->rows % 2) return fail(b, GH_E_INVALID, "gemm multi: matrix shape");
        if (!fits(segs[i].out, (uint64_t)n * w->rows * 2)) return fail(b, GH_E_RANGE, "gemm multi: output too small");
        if (segs[i].role > GH_GEMM_ROLE_ROPE_KEY) return fail(b, GH_E_INVALID, "gemm multi: role");
        if (segs[i].role) {
            any_rope = true;
            if (!rope || !gemm_rope_applies(n, w->rows, head_dim, *rope) || (uint64_t)base + n > rope->positions)
                return fail(b, GH_E_UNSUPPORTED, "gemm multi: RoPE over whole heads, positions in the table");
        }
        ga.seg[i] = GhGemmSeg{w->addr, segs[i].out->addr, w->rows, w->format, tiles, total, segs[i].role, 0};
        tiles += ceil_div(w->rows, BR);
        total += w->rows;
    }
    if (!fits(a, (uint64_t)n * in_dim * 2)) return fail(b, GH_E_RANGE, "gemm multi: input too small");
    // 256-token tiles above 128 tokens, 128-token tiles below (kGemmTallTokens); FP16 copies
    // registered for every matrix: the launch copies the weights instead of dequantizing them
    const bool tall = n >= kGemmTallTokens;
    bool copies = tall;
    for (uint32_t i = 0; i < nseg; ++i) copies = copies && b->w16.count(segs[i].w->addr);
    const uint32_t tt = ceil_div(n, tall ? 256u : 128u), units = in_dim / 64;
    // splits: the CUs over the tiles, at most 16 and at least 8 units per split (12 in the
    // 128-token tiles, as op_gemm), none empty
    const uint32_t min_units = tall ? 8u : 12u;
    uint32_t splits =
        std::max<uint32_t>(1, std::min<uint32_t>({b->cus / (tiles * tt), std::max<uint32_t>(1, units / min_units), 16u}));
    for (;;) {
        const uint32_t per = gh_gemm_split_units(units, splits), s = ceil_div(units, per);
        if (s == splits) break;
        splits = s;
    }
    if (copies)
        for (uint32_t i = 0; i < nseg; ++i) ga.seg[i].w = b->w16.at(segs[i].w->addr);
    ga.x = a->addr;
    ga.in_dim = in_dim;
    ga.rows = total;
    ga.n = n;
    ga.splits = splits;
    ga.nseg = nseg;
    if (any_rope) {
        ga.table = (uint64_t)rope->table;
        ga.post = (uint64_t)rope->post;
        ga.base = base;
        ga.head_dim = head_dim;
        ga.pairs = rope->yarn.rope_dim / 2;
    } else {
        ga.head_dim = 2;  // unused (no role): a nonzero divisor
    }
    if (splits > 1) {
        int rc = ensure_workspace(b, (size_t)splits * n * total * 4);
        if (rc) return rc;
        ga.part = (uint64_t)((char*)b->ws + kArgmaxBytes);
    }
    const GhKernel k = copies ? K_GEMM4W_MIXED_R128 : tall ? K_GEMM3_MIXED_R128 : K_GEMM3_MIXED_R128_T128;
    int rc = launch(b, k, tiles, tt, splits, gemm_block(k), &ga);
    if (rc) return rc;
    if (splits > 1) {
        const uint64_t npairs = (uint64_t)n * total / 2;
        return launch(b, K_GEMM_REDUCE_SEG, (uint32_t)std::min<uint64_t>(ceil_div(npairs, (uint64_t)256), 4096), 1, 1,
                      256, &ga);
    }
    for (uint32_t i = 0; i < nseg && !rc; ++i)
        if (segs[i].role)
            rc = op_rope(b, *rope, segs[i].out, segs[i].w->rows / head_dim, head_dim, base, n,
                         segs[i].role == GH_GEMM_ROLE_ROPE_QUERY ? GH_ROPE_QUERY : GH_ROPE_KEY, nullptr);
    return rc;
}

int op_dequant_f16(gh_backend* b, const gh_buf* w, uint64_t out16) {
    if (!is_weight(w)) return fail(b, GH_E_UNSUPPORTED, "dequant f16: weight must be Q4_K or Q6_K");
    GhGemmArgs ga{};
    ga.w = w->addr;
    ga.out = out16;
    ga.in_dim = w->cols;
    ga.rows = w->rows;
    const uint64_t threads = (uint64_t)w->rows * (w->cols / 64) * 2;
    return launch(b, w->format == GH_FMT_Q4_K ? K_DEQUANT_F16_Q4K : K_DEQUANT_F16_Q6K, ceil_div(threads, 256), 1, 1,
                  256, &ga);
}

bool gemm_rope_applies(uint32_t n, uint32_t out_dim, uint32_t head_dim, const GhRopeTable& rope) {
    return n >= kGemmMinTokens && head_dim && head_dim % 2 == 0 && out_dim % head_dim == 0 && rope.table &&
           rope.yarn.rope_dim <= head_dim;
}

}  // namespace gh

extern "C" {

static int gemv_launch(gh_backend* b, const gh_buf* out, const gh_buf* a, const gh_buf* w,
                       uint32_t in_dim, uint32_t out_dim, uint32_t n, bool f32) {
    if (!is_weight(w)) return fail(b, GH_E_UNSUPPORTED, "matmul: weight must be Q4_K or Q6_K");
    if (w->cols != in_dim || w->rows != out_dim) return fail(b, GH_E_INVALID, "matmul: weight shape mismatch");
    if (!fits(a, (uint64_t)n * in_dim * 2) || !fits(out, (uint64_t)n * out_dim * (f32 ? 4 : 2)))
        return fail(b, GH_E_RANGE, "matmul: buffer too small");
    if (!f32 && n >= kGemmMinTokens) return op_gemm(b, out->addr, a, w, n);
    GemvSeg seg{w, out->addr, f32 ? (uint32_t)GH_EPI_F32 : (uint32_t)GH_EPI_F16};
    return op_gemv(b, &seg, 1, a, n, 0, nullptr, 0, nullptr);
}

int gh_matmul(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* a,
              const gh_buf* w, uint32_t in_dim, uint32_t out_dim) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    return latch(enc, gemv_launch(b, out, a, w, in_dim, out_dim, 1, false));
}

int gh_matmul_batched(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* a,
                      const gh_buf* w, uint32_t in_dim, uint32_t out_dim, uint32_t n) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (n == 0) return latch(enc, fail(b, GH_E_INVALID, "matmul_batched: n == 0"));
    return latch(enc, gemv_launch(b, out, a, w, in_dim, out_dim, n, false));
}

int gh_logits(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* x,
              const gh_buf* w, uint32_t in_dim, uint32_t out_dim) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    return latch(enc, gemv_launch(b, out, x, w, in_dim, out_dim, 1, true));
}

int gh_rmsnorm_x(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* x,
                 const gh_buf* w, uint32_t dim, float eps, uint32_t rows) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (dim == 0 || !fits(x, (uint64_t)rows * dim * 4) || !fits(out, (uint64_t)rows * dim * 2) || !fits(w, (uint64_t)dim * 2))
        return latch(enc, fail(b, GH_E_RANGE, "rmsnorm_x: buffer too small"));
    if (dim % 4) return latch(enc, fail(b, GH_E_INVALID, "rmsnorm_x: dim must be a multiple of 4"));
    GhRmsnormArgs a{out->addr, x->addr, w->addr, dim, rows, eps, 0};
    return latch(enc, launch(b, K_RMSNORM, rows, 1, 1, 256, &a));
}

int gh_rope_yarn(gh_backend* b, gh_encoder* enc, const gh_buf* x, uint32_t heads,
                 uint32_t head_dim, uint32_t pos, const gh_yarn* yarn, uint32_t role) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (!yarn_valid(yarn) || role > 1 || yarn->rope_dim > head_dim)
        return latch(enc, fail(b, GH_E_INVALID, "rope: invalid YaRN parameters"));
    if (!fits(x, (uint64_t)heads * head_dim * 2)) return latch(enc, fail(b, GH_E_RANGE, "rope: buffer too small"));
    if (pos >= kMaxRopePositions) return latch(enc, fail(b, GH_E_RANGE, "rope: position beyond the table limit"));
    rc = ensure_rope(b, b->rope, yarn, pos + 1);
    if (rc) return latch(enc, rc);
    return latch(enc, op_rope(b, b->rope, x, heads, head_dim, pos, 1, role, nullptr));
}

int gh_rope_yarn_batched(gh_backend* b, gh_encoder* enc, const gh_buf* q, const gh_buf* k,
                         uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim, uint32_t base,
                         uint32_t rows, const gh_yarn* yarn) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (rows == 0) return latch(enc, fail(b, GH_E_INVALID, "rope: empty batch"));
    if (!yarn_valid(yarn) || yarn->rope_dim > head_dim) return latch(enc, fail(b, GH_E_INVALID, "rope: invalid YaRN parameters"));
    if ((uint64_t)base + rows > 0xFFFFFFFFull) return latch(enc, fail(b, GH_E_RANGE, "rope: position overflow"));
    if (!fits(q, (uint64_t)rows * q_heads * head_dim * 2) || !fits(k, (uint64_t)rows * kv_heads * head_dim * 2))
        return latch(enc, fail(b, GH_E_RANGE, "rope: buffer too small"));
    rc = ensure_rope(b, b->rope, yarn, base + rows);
    if (!rc) rc = op_rope(b, b->rope, q, q_heads, head_dim, base, rows, GH_ROPE_QUERY, nullptr);
    if (!rc) rc = op_rope(b, b->rope, k, kv_heads, head_dim, base, rows, GH_ROPE_KEY, nullptr);
    return latch(enc, rc);
}

int gh_silu_mul(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* gate,
                const gh_buf* up, uint32_t n) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (!fits(out, (uint64_t)n * 2) || !fits(gate, (uint64_t)n * 2) || !fits(up, (uint64_t)n * 2))
        return latch(enc, fail(b, GH_E_RANGE, "silu_mul: buffer too small"));
    GhEltArgs a{out->addr, gate->addr, up->addr, n, 0};
    return latch(enc, launch(b, K_SILU_MUL, ceil_div(n, 256), 1, 1, 256, &a));
}

int gh_residual_add(gh_backend* b, gh_encoder* enc, const gh_buf* x, const gh_buf* y,
                    uint32_t n) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (!fits(x, (uint64_t)n * 4) || !fits(y, (uint64_t)n * 2))
        return latch(enc, fail(b, GH_E_RANGE, "residual_add: buffer too small"));
    GhEltArgs a{x->addr, 0, y->addr, n, 0};
    return latch(enc, launch(b, K_RESIDUAL_ADD, ceil_div(n, 256), 1, 1, 256, &a));
}


int gh_attention_decode(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* q,
                        const gh_kv* kv, uint32_t q_heads, uint32_t pos, uint32_t layer) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    rc = check_attention(b, out, q, kv, q_heads, pos, 1, layer);
    if (!rc) rc = op_attention(b, out, q, kv, q_heads, pos, 1, layer, nullptr, pos);
    return latch(enc, rc);
}

int gh_attention_prefill(gh_backend* b, gh_encoder* enc, const gh_buf* out, const gh_buf* q,
                         const gh_kv* kv, uint32_t q_heads, uint32_t base, uint32_t n,
                         uint32_t layer) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (n == 0) return latch(enc, fail(b, GH_E_INVALID, "attention_prefill: n == 0"));
    rc = check_attention(b, out, q, kv, q_heads, base + n - 1, n, layer);
    if (!rc) rc = op_attention(b, out, q, kv, q_heads, base, n, layer, nullptr, base + n - 1);
    return latch(enc, rc);
}

int gh_read_logits(gh_backend* b, const gh_buf* logits, uint64_t vocab, float* dst) {
    if (!b || !logits) return GH_E_INVALID;
    if (!fits(logits, vocab * 4)) return fail(b, GH_E_RANGE, "read_logits: buffer smaller than vocab");
    return gh_download(b, logits, 0, dst, vocab * 4);
}

int gh_read_argmax(gh_backend* b, const gh_buf* logits, uint64_t vocab, uint32_t* out) {
    if (!b || !logits || !out) return GH_E_INVALID;
    if (vocab == 0) return fail(b, GH_E_INVALID, "read_argmax on empty logits");
    if (!fits(logits, vocab * 4)) return fail(b, GH_E_RANGE, "read_argmax: buffer smaller than vocab");
    int rc = op_argmax(b, logits, vocab, nullptr, nullptr);
    if (rc) return rc;
    rc = hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
    if (rc) return rc;
    return hip_check(b, hipMemcpy(out, (char*)b->ws + 2048, 4, hipMemcpyDeviceToHost), "hipMemcpy argmax");
}

// read_topk: k <= 128 on the device (gh_topk_partial over stripes of at most kTopkChunk
// logits per step, at most 128 stripes, then gh_topk_final; 8 k bytes come back), larger k
// on the host over the read-back logits. Both give exactly the reference's selection and
// order (cpu/readback.rs:59-69): (logit desc by f32 total order, index asc).
constexpr uint64_t kTopkDeviceMax = 128, kTopkChunk = 2048, kTopkStripes = 128;

int gh_read_topk(gh_backend* b, const gh_buf* logits, uint64_t vocab, uint64_t k, uint32_t* idx,
                 float* val, uint64_t* count) {
    if (!b || !logits || !count) return GH_E_INVALID;
    if (vocab == 0) return fail(b, GH_E_INVALID, "read_topk on empty logits");
    if (vocab > 0xFFFFFFFFull) return fail(b, GH_E_UNSUPPORTED, "read_topk: vocab beyond 32-bit indices");
    if (!fits(logits, vocab * 4)) return fail(b, GH_E_RANGE, "read_topk: buffer smaller than vocab");
    k = std::min<uint64_t>(k, vocab);
    *count = 0;
    if (k == 0) return GH_OK;
    if (k <= kTopkDeviceMax) {
        uint32_t width = 1;
        while (width < k) width <<= 1;
        // stripes of kTopkChunk logits, widened (in whole chunks) to keep at most 128 stripes
        const uint64_t chunks = (vocab + kTopkChunk - 1) / kTopkChunk;
        const uint64_t per = kTopkChunk * ((chunks + kTopkStripes - 1) / kTopkStripes);
        GhTopkArgs a{};
        a.logits = logits->addr;
        a.n = (uint32_t)vocab;
        a.per = (uint32_t)std::min<uint64_t>(per, 0xFFFFFFFFull);
        a.stripes = (uint32_t)((vocab + per - 1) / per);
        a.width = width;
        a.k = (uint32_t)k;
        const size_t part_bytes = (size_t)a.stripes * width * 8;
        int rc = ensure_workspace(b, part_bytes + 8 * k);
        if (rc) return rc;
        char* ws = (char*)b->ws + kArgmaxBytes;
        a.part = (uint64_t)ws;
        a.out = (uint64_t)(ws + part_bytes);
        rc = launch(b, K_TOPK_PARTIAL, a.stripes, 1, 1, 512, &a);
        if (!rc) rc = launch(b, K_TOPK_FINAL, 1, 1, 1, 1024, &a);
        if (!rc) rc = hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
        std::vector<uint32_t> pairs(2 * k);
        if (!rc) rc = hip_check(b, hipMemcpy(pairs.data(), ws + part_bytes, 8 * k, hipMemcpyDeviceToHost),
                                "hipMemcpy topk");
        if (rc) return rc;
        for (uint64_t i = 0; i < k; ++i) {
            if (idx) idx[i] = pairs[i];
            if (val) std::memcpy(&val[i], &pairs[k + i], 4);
        }
        *count = k;
        return GH_OK;
    }
    std::vector<float> l(vocab);
    int rc = gh_read_logits(b, logits, vocab, l.data());
    if (rc) return rc;
    std::vector<uint32_t> cand(vocab);
    for (uint64_t i = 0; i < vocab; ++i) cand[i] = (uint32_t)i;
    auto order = [&](uint32_t x, uint32_t y) {
        int kx = total_key(l[x]), ky = total_key(l[y]);
        return kx != ky ? kx > ky : x < y;
    };
    std::partial_sort(cand.begin(), cand.begin() + (ptrdiff_t)k, cand.end(), order);
    for (uint64_t i = 0; i < k; ++i) {
        if (idx) idx[i] = cand[i];
        if (val) val[i] = l[cand[i]];
    }
    *count = k;
    return GH_OK;
}

int gh_timer_start(gh_backend* b) {
    if (!b) return GH_E_INVALID;
    return hip_check(b, hipEventRecord(b->ev_start, b->stream), "hipEventRecord");
}

int gh_timer_stop(gh_backend* b, float* ms) {
    if (!b || !ms) return GH_E_INVALID;
    int rc = hip_check(b, hipEventRecord(b->ev_stop, b->stream), "hipEventRecord");
    if (!rc) rc = hip_check(b, hipEventSynchronize(b->ev_stop), "hipEventSynchronize");
    if (!rc) rc = hip_check(b, hipEventElapsedTime(ms, b->ev_start, b->ev_stop), "hipEventElapsedTime");
    return rc;
}

int gh_synchronize(gh_backend* b) {
    if (!b) return GH_E_INVALID;
    return hip_check(b, hipStreamSynchronize(b->stream), "hipStreamSynchronize");
}

int gh_set_attention_xcd_merge(gh_backend* b, int enable) {
    if (!b) return GH_E_INVALID;
    if (enable && !b->xcds)
        return fail(b, GH_E_UNSUPPORTED, "attention: the device's workgroup-to-XCD placement was not confirmed");
    b->attn_xcd_merge = enable != 0;
    ++b->gen;  // recorded decode graphs hold the other kernel
    return GH_OK;
}

uint32_t gh_xcd_count(const gh_backend* b) { return b ? b->xcds : 0; }

int gh_set_attention_splits(gh_backend* b, uint32_t splits) {
    if (!b) return GH_E_INVALID;
    if (splits > 32) return fail(b, GH_E_INVALID, "attention splits: at most 32");
    b->attn_splits = splits;
    ++b->gen;  // recorded graphs hold the old grid
    return GH_OK;
}

int gh_stream_probe(gh_backend* b, gh_encoder* enc, const gh_buf* src, uint64_t offset, uint64_t bytes,
                    const gh_buf* sink, uint32_t workgroups) {
    int rc = check_enc(b, enc);
    if (rc) return rc;
    if (!src || !sink) return latch(enc, fail(b, GH_E_INVALID, "stream probe: null"));
    if (offset % 16 || bytes % 16 || bytes == 0 || bytes / 16 > 0xFFFFFFFFull || workgroups == 0 ||
        workgroups > 65535)
        return latch(enc, fail(b, GH_E_INVALID, "stream probe: 16-byte multiples, 1..65535 workgroups"));
    if (offset > src->bytes || bytes > src->bytes - offset || !fits(sink, 4))
        return latch(enc, fail(b, GH_E_RANGE, "stream probe: beyond buffer"));
    GhEltArgs e{sink->addr, src->addr + offset, 0, (uint32_t)(bytes / 16), workgroups};
    return latch(enc, launch(b, K_STREAM_PROBE, workgroups, 1, 1, 256, &e));
}

int gh_scratch_info(const gh_backend* b, uint64_t* workspace_bytes, uint64_t* counter_slots,
                    uint64_t* generation) {
    if (!b) return GH_E_INVALID;
    if (workspace_bytes) *workspace_bytes = b->ws_bytes;
    if (counter_slots) *counter_slots = b->counter_slots;
    if (generation) *generation = b->gen;
    return GH_OK;
}

}  // extern "C"

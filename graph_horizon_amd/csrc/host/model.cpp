// Graph driver: MistralGraph's op order recorded through the backend ops.
//   decode  — forward::token (family/mistral/graph/forward.rs:68-83), block::record
//             (block.rs:17-107), mlp::record (mlp.rs:12-61), tail::record (tail.rs:11-59);
//   prefill — prefill::prefill / record_batch (graph/prefill/encode.rs:16-106) and
//             prefill::layer::record (prefill/layer.rs:18-122).
// The greedy loop replays a captured HIP graph per token (one graph per range of positions):
// the token id and position live in device memory, the step ends with an on-device argmax that
// becomes the next step's input.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <array>
#include <cstring>
#include <vector>

#include "internal.h"

using namespace gh;

namespace {
constexpr uint32_t kNoLayer = 0xFFFFFFFFu;

// Decode steps run from graphs captured per position range: each range's attention launch is
// sized for the range's last position (one split per 64-position chunk, at most 32), so a step
// at a short position of a long cache does not launch the idle splits of the whole context
// (at most a fifth of a range's splits idle from 256 positions on). Ranges end at these
// positions and at the cache's context (from 2048 positions the split count is 32 anyway; a
// forced split count, gh_set_attention_splits, keeps one range over the whole context).
constexpr uint32_t kStepRangeEnds[] = {64, 128, 192, 256, 320, 384, 512, 640, 768, 1024, 1280, 1536, 2048};
constexpr uint32_t kStepRanges = sizeof(kStepRangeEnds) / sizeof(kStepRangeEnds[0]) + 1;

struct StepGraph {
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph = nullptr;
    uint64_t gen = 0;  // backend generation the graph was captured against
};

struct Scratch {  // backend/buffers.rs:17-29, sized for `rows` token rows
    gh_buf x, normed, q, k, v, attn, proj, gate, up, act, ffn_out;
};
}  // namespace

struct gh_model {
    gh_backend* b = nullptr;
    gh_model_config cfg{};
    std::vector<std::array<gh_buf, 9>> layers;
    gh_buf token_embd{}, output_norm{}, output{};
    Scratch dec{}, pre{};
    gh_buf logits{};
    gh_buf scalars{};  // u32[4]: position, token, argmax, spare
    gh_buf history{};  // u32[kv_context]
    gh_buf prompt{};   // u32[kv_context]: the token ids of a prefill call, for the batched embed
    gh_kv kv{};
    GhRopeTable rope;  // this model's YaRN table for positions 0 .. kv_context - 1
    std::vector<gh_buf> owned;
    std::array<StepGraph, kStepRanges> steps{};  // decode step graphs by position range
    uint32_t step_len = 0;  // positions the decode step being recorded serves (0: the context)
    uint32_t last_rows = 0;  // rows of the most recent pass (for read_x)
    bool last_prefill = false;
    // FP16 copies of the layer matrices for the prefill GEMMs (registered in b->w16), made
    // before the first prefill chunk of more than 128 rows (kGemmTallTokens); empty until then (and
    // left unregistered during shorter chunks, whose GEMMs dequantize)
    std::vector<std::pair<uint64_t, gh_buf>> w16;  // (weight address, copy)
    // the copies did not fit (or crowded out a prefill's workspace): the prefill dequantizes
    // from then on, until the weights are reloaded
    bool w16_failed = false;
};

namespace {

int alloc(gh_model* m, uint64_t bytes, gh_buf* out) {
    int rc = gh_alloc_buffer(m->b, std::max<uint64_t>(bytes, 256), out);
    if (!rc) m->owned.push_back(*out);
    return rc;
}

// Register the copies for this prefill call, or withdraw them (shorter chunks dequantize).
void set_w16(gh_model* m, bool on) {
    for (auto& [addr, copy] : m->w16) {
        if (on)
            m->b->w16[addr] = copy.addr;
        else
            m->b->w16.erase(addr);
    }
}

void free_w16(gh_model* m) {
    for (auto& [addr, copy] : m->w16) {
        m->b->w16.erase(addr);
        gh_free_buffer(m->b, &copy);
    }
    m->w16.clear();
}

constexpr uint32_t kCopiedTensors[] = {GH_T_ATTN_Q, GH_T_ATTN_K, GH_T_ATTN_V, GH_T_ATTN_OUTPUT,
                                       GH_T_FFN_GATE, GH_T_FFN_UP, GH_T_FFN_DOWN};

// Device memory a prefill chunk of `rows` rows may still claim after the copies are made: the
// GEMMs' split-K partials (at most one FP32 value per output and split, 32 splits bounded by
// the CU count) and the attention partials, with 1 GiB beside them for the rest.
uint64_t prefill_headroom(const gh_model* m, uint32_t rows) {
    const gh_model_config& c = m->cfg;
    const uint64_t widest = std::max<uint64_t>(c.feed_forward_length, (uint64_t)c.head_count * c.key_length);
    const uint64_t split_k = (uint64_t)rows * widest * 4 * 8;
    return split_k + ((uint64_t)256 << 20) + ((uint64_t)1 << 30);
}

// Dequantize every layer matrix once into an FP16 copy and register it, so that the prefill
// GEMMs copy weight tiles into LDS instead of dequantizing them per tile (the same FP16 values:
// identical results). 2 bytes per weight: 13.1 GB for the 8B shape, 24.3 GB for the 14B one, of
// 288 GB. The copies are made only when the device has room for them and for a prefill chunk's
// workspace beside them; otherwise (or when an allocation fails) the model records the failure
// and its prefills keep dequantizing (nothing is registered) without trying again.
int ensure_w16(gh_model* m) {
    if ((m->cfg.flags & GH_MODEL_NO_F16_WEIGHTS) || m->w16_failed || !m->w16.empty()) return GH_OK;
    uint64_t need = prefill_headroom(m, m->cfg.prefill_rows);
    for (auto& l : m->layers)
        for (uint32_t t : kCopiedTensors) need += (uint64_t)l[t].rows * l[t].cols * 2;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess || free_b < need) {
        (void)hipGetLastError();
        m->w16_failed = true;
        return GH_OK;
    }
    for (auto& l : m->layers)
        for (uint32_t t : kCopiedTensors) {
            const gh_buf& w = l[t];
            gh_buf copy{};
            if (gh_alloc_buffer(m->b, (uint64_t)w.rows * w.cols * 2, &copy) != GH_OK) {
                free_w16(m);
                m->b->err.clear();
                m->w16_failed = true;
                return GH_OK;
            }
            int rc = op_dequant_f16(m->b, &w, copy.addr);
            if (rc) {
                gh_free_buffer(m->b, &copy);
                free_w16(m);
                return rc;
            }
            m->w16.emplace_back(w.addr, copy);
            m->b->w16[w.addr] = copy.addr;
        }
    return GH_OK;
}

int latch_rc(gh_encoder* enc, int rc) {
    if (rc != GH_OK && enc && enc->latched == GH_OK) enc->latched = rc;
    return rc;
}

int alloc_scratch(gh_model* m, uint32_t rows, Scratch* s) {
    const gh_model_config& c = m->cfg;
    const uint64_t d = c.embedding_length, ffn = c.feed_forward_length;
    const uint64_t qw = (uint64_t)c.head_count * c.key_length, kw = (uint64_t)c.kv_head_count * c.key_length;
    const uint64_t vw = (uint64_t)c.kv_head_count * c.value_length, aw = (uint64_t)c.head_count * c.value_length;
    int rc = alloc(m, rows * d * 4, &s->x);
    if (!rc) rc = alloc(m, rows * d * 2, &s->normed);
    if (!rc) rc = alloc(m, rows * qw * 2, &s->q);
    if (!rc) rc = alloc(m, rows * kw * 2, &s->k);
    if (!rc) rc = alloc(m, rows * vw * 2, &s->v);
    if (!rc) rc = alloc(m, rows * aw * 2, &s->attn);
    if (!rc) rc = alloc(m, rows * d * 2, &s->proj);
    if (!rc) rc = alloc(m, rows * ffn * 2, &s->gate);
    if (!rc) rc = alloc(m, rows * ffn * 2, &s->up);
    if (!rc) rc = alloc(m, rows * ffn * 2, &s->act);
    if (!rc) rc = alloc(m, rows * d * 2, &s->ffn_out);
    return rc;
}

// One decode layer (rows == 1) with the glue fused into the GEMV epilogues:
//   rmsnorm → [Q, K, V GEMVs + RoPE(Q) + RoPE(K)→K cache + V→V cache] → attention →
//   [O GEMV + residual] → rmsnorm → [gate/up GEMVs + SwiGLU] → [down GEMV + residual].
// Same values as the op-by-op recording below: each epilogue applies the reference op to
// the FP16-rounded projection (block.rs:17-107, mlp.rs:12-61).
int layer_decode_fused(gh_model* m, gh_encoder* enc, const Scratch& s, uint32_t li,
                       uint32_t base, const void* pos_ptr) {
    gh_backend* b = m->b;
    const gh_model_config& c = m->cfg;
    const auto& w = m->layers[li];
    const uint64_t kv_row_k = (uint64_t)c.kv_head_count * c.key_length;
    const uint64_t kv_row_v = (uint64_t)c.kv_head_count * c.value_length;
    const uint64_t kbase = m->kv.k.addr + (uint64_t)li * m->kv.context * kv_row_k * 2;
    const uint64_t vbase = m->kv.v.addr + (uint64_t)li * m->kv.context * kv_row_v * 2;
    // RMSNorm fused into the QKV and gate/up launches' staging of x (up to kFusedNormMaxDim)
    const bool fuse_norm = c.embedding_length <= kFusedNormMaxDim;
    auto normed = [&](const gh_buf* nw, const gh_buf** x_in, const gh_buf** norm_w) {
        if (fuse_norm) {
            *x_in = &s.x;
            *norm_w = nw;
            return 0;
        }
        *x_in = &s.normed;
        *norm_w = nullptr;
        return gh_rmsnorm_x(b, enc, &s.normed, &s.x, nw, c.embedding_length, c.rms_epsilon, 1);
    };
    const GemvSeg qkv[3] = {{&w[GH_T_ATTN_Q], s.q.addr, GH_EPI_ROPE},
                            {&w[GH_T_ATTN_K], kbase, GH_EPI_ROPE_CACHE},
                            {&w[GH_T_ATTN_V], vbase, GH_EPI_CACHE}};
    const gh_buf *xin = nullptr, *nw = nullptr;
    int rc = normed(&w[GH_T_ATTN_NORM], &xin, &nw);
    if (!rc) rc = op_gemv(b, qkv, 3, xin, 1, base, pos_ptr, c.key_length, nullptr, nw, c.rms_epsilon, &m->rope);
    const uint32_t max_pos = pos_ptr ? (m->step_len ? m->step_len : m->kv.context) - 1 : base;
    if (!rc) rc = op_attention(b, &s.attn, &s.q, &m->kv, c.head_count, base, 1, li, pos_ptr, max_pos);
    const GemvSeg o{&w[GH_T_ATTN_OUTPUT], s.x.addr, GH_EPI_RESID};
    if (!rc) rc = op_gemv(b, &o, 1, &s.attn, 1, 0, nullptr, 0, nullptr);
    const GemvSeg gu{&w[GH_T_FFN_GATE], s.act.addr, GH_EPI_SWIGLU};
    if (!rc) rc = normed(&w[GH_T_FFN_NORM], &xin, &nw);
    if (!rc) rc = op_gemv(b, &gu, 1, xin, 1, 0, nullptr, 0, &w[GH_T_FFN_UP], nw, c.rms_epsilon);
    const GemvSeg dn{&w[GH_T_FFN_DOWN], s.x.addr, GH_EPI_RESID};
    if (!rc) rc = op_gemv(b, &dn, 1, &s.act, 1, 0, nullptr, 0, nullptr);
    return latch_rc(enc, rc);
}

bool fusable(const gh_model* m, uint32_t li) {
    const auto& w = m->layers[li];
    return w[GH_T_FFN_GATE].format == GH_FMT_Q4_K && w[GH_T_FFN_UP].format == GH_FMT_Q4_K &&
           m->cfg.head_count * m->cfg.value_length == w[GH_T_ATTN_OUTPUT].cols;
}

// One transformer layer over `rows` packed rows at absolute positions base + r
// (+ *pos_ptr when the position lives on the device). With `normed` (prefill), the GEMM path's
// epilogues carry the glue: the O and down projections' output rows go straight into the
// residual and the following RMSNorm (gh_gemm_tail), silu_mul is applied in the gate and up
// projections' shared split reduce (or the up projection's epilogue); *normed on return says
// the next layer's attention norm is already in s.normed. The values are those of the
// separate ops below.
int layer(gh_model* m, gh_encoder* enc, const Scratch& s, uint32_t li, uint32_t base,
          uint32_t rows, const void* pos_ptr, bool* normed = nullptr) {
    if (rows == 1 && fusable(m, li)) return layer_decode_fused(m, enc, s, li, base, pos_ptr);
    gh_backend* b = m->b;
    const gh_model_config& c = m->cfg;
    const auto& w = m->layers[li];
    const uint32_t d = c.embedding_length, ffn = c.feed_forward_length;
    const uint32_t qw = c.head_count * c.key_length, kw = c.kv_head_count * c.key_length;
    const uint32_t vw = c.kv_head_count * c.value_length, aw = c.head_count * c.value_length;
    const bool fuse = normed != nullptr;
    int rc = GH_OK;
    if (!(fuse && *normed)) rc = gh_rmsnorm_x(b, enc, &s.normed, &s.x, &w[GH_T_ATTN_NORM], d, c.rms_epsilon, rows);
    if (fuse) *normed = false;
    gh_no_barrier(b);
    // kv_cache::append_batch (kv_cache/mod.rs:133-177): payload offsets of (layer, base)
    const uint64_t per_pos_k = (uint64_t)c.kv_head_count * c.key_length;
    const uint64_t per_pos_v = (uint64_t)c.kv_head_count * c.value_length;
    const uint64_t koff = ((uint64_t)li * m->kv.context + base) * per_pos_k;
    const uint64_t voff = ((uint64_t)li * m->kv.context + base) * per_pos_v;
    if (fuse) {
        // The cache rows of positions base .. base + rows - 1 ([position][kv_heads][dim]) are the
        // K/V projections' output layout: the GEMMs write there and RoPE rotates K in place —
        // the bytes of projecting, rotating and append_batch's copy.
        gh_buf kd{}, vd{};
        if (!rc) rc = gh_view(b, &m->kv.k, koff * 2, (uint64_t)rows * kw * 2, &kd);
        if (!rc) rc = gh_view(b, &m->kv.v, voff * 2, (uint64_t)rows * vw * 2, &vd);
        if (gemm_multi_applies(rows)) {
            // the three projections in one launch and one split reduce
            const GemmSegSpec qkv[3] = {{&w[GH_T_ATTN_Q], &s.q, GH_GEMM_ROLE_ROPE_QUERY},
                                        {&w[GH_T_ATTN_K], &kd, GH_GEMM_ROLE_ROPE_KEY},
                                        {&w[GH_T_ATTN_V], &vd, GH_GEMM_ROLE_PLAIN}};
            if (!rc) rc = op_gemm_multi(b, &s.normed, qkv, 3, rows, &m->rope, base, c.key_length);
        } else {
            // chunks of fewer than 8 rows (the GEMV): rope_yarn_batched (prefill/layer.rs:79-89)
            // on the Q rows and, in place, on the K cache rows
            if (!rc) rc = gh_matmul_batched(b, enc, &s.q, &s.normed, &w[GH_T_ATTN_Q], d, qw, rows);
            if (!rc) rc = gh_matmul_batched(b, enc, &kd, &s.normed, &w[GH_T_ATTN_K], d, kw, rows);
            if (!rc) rc = gh_matmul_batched(b, enc, &vd, &s.normed, &w[GH_T_ATTN_V], d, vw, rows);
            if (!rc) rc = op_rope(b, m->rope, &s.q, c.head_count, c.key_length, base, rows, GH_ROPE_QUERY, nullptr);
            if (!rc) rc = op_rope(b, m->rope, &kd, c.kv_head_count, c.key_length, base, rows, GH_ROPE_KEY, nullptr);
        }
    } else {
        if (!rc) rc = gh_matmul_batched(b, enc, &s.q, &s.normed, &w[GH_T_ATTN_Q], d, qw, rows);
        if (!rc) rc = gh_matmul_batched(b, enc, &s.k, &s.normed, &w[GH_T_ATTN_K], d, kw, rows);
        if (!rc) rc = gh_matmul_batched(b, enc, &s.v, &s.normed, &w[GH_T_ATTN_V], d, vw, rows);
        // rope_yarn (block.rs:147-166) / rope_yarn_batched (prefill/layer.rs:79-89)
        if (!rc) rc = op_rope(b, m->rope, &s.q, c.head_count, c.key_length, base, rows, GH_ROPE_QUERY, pos_ptr);
        if (!rc) rc = op_rope(b, m->rope, &s.k, c.kv_head_count, c.key_length, base, rows, GH_ROPE_KEY, pos_ptr);
        if (!rc) rc = op_kv_write(b, &m->kv, &s.k, &s.v, koff, voff, rows * c.kv_head_count, pos_ptr);
    }
    const uint32_t max_pos = pos_ptr ? (m->step_len ? m->step_len : m->kv.context) - 1 : base + rows - 1;
    if (!rc) rc = op_attention(b, &s.attn, &s.q, &m->kv, c.head_count, base, rows, li, pos_ptr, max_pos);
    if (fuse && gemm_epi_applies(rows, d, true)) {
        // out-projection, residual add and mlp::record's norm in one GEMM + tail
        if (!rc) rc = op_matmul_epi(b, &s.proj, &s.attn, &w[GH_T_ATTN_OUTPUT], aw, d, rows, nullptr, &s.x,
                                    &w[GH_T_FFN_NORM], &s.normed, c.rms_epsilon);
    } else {
        if (!rc) rc = gh_matmul_batched(b, enc, &s.proj, &s.attn, &w[GH_T_ATTN_OUTPUT], aw, d, rows);
        if (!rc) rc = gh_residual_add(b, enc, &s.x, &s.proj, d * rows);
        // mlp::record
        if (!rc) rc = gh_rmsnorm_x(b, enc, &s.normed, &s.x, &w[GH_T_FFN_NORM], d, c.rms_epsilon, rows);
    }
    gh_no_barrier(b);
    if (fuse && gemm_epi_applies(rows, ffn, false)) {
        // gate, up and silu_mul: where the GEMMs split K, one reduce for both
        if (!rc) rc = op_gemm_swiglu(b, &s.act, &s.gate, &s.normed, &w[GH_T_FFN_GATE], &w[GH_T_FFN_UP], rows);
    } else {
        if (!rc) rc = gh_matmul_batched(b, enc, &s.gate, &s.normed, &w[GH_T_FFN_GATE], d, ffn, rows);
        if (!rc) rc = gh_matmul_batched(b, enc, &s.up, &s.normed, &w[GH_T_FFN_UP], d, ffn, rows);
        if (!rc) rc = gh_silu_mul(b, enc, &s.act, &s.gate, &s.up, ffn * rows);
    }
    if (fuse && gemm_epi_applies(rows, d, true)) {
        // down projection and residual add, with the next layer's attention norm when there is one
        const bool next = li + 1 < c.block_count;
        const gh_buf* nw = next ? &m->layers[li + 1][GH_T_ATTN_NORM] : nullptr;
        if (!rc) rc = op_matmul_epi(b, &s.ffn_out, &s.act, &w[GH_T_FFN_DOWN], ffn, d, rows, nullptr, &s.x, nw,
                                    next ? &s.normed : nullptr, c.rms_epsilon);
        if (!rc) *normed = next;
    } else {
        if (!rc) rc = gh_matmul_batched(b, enc, &s.ffn_out, &s.act, &w[GH_T_FFN_DOWN], ffn, d, rows);
        if (!rc) rc = gh_residual_add(b, enc, &s.x, &s.ffn_out, d * rows);
    }
    return latch_rc(enc, rc);
}

// tail::record_buffers (tail.rs:22-59): output_norm then FP32 logits (dedicated or tied).
// output_norm is fused into the logits launch's staging of x.
int tail(gh_model* m, gh_encoder* enc, const gh_buf* xrow, const gh_buf* normed_row) {
    const gh_model_config& c = m->cfg;
    const gh_buf* out = m->output.addr ? &m->output : &m->token_embd;
    const bool quant = out->format == GH_FMT_Q4_K || out->format == GH_FMT_Q6_K;
    if (!quant || out->cols != c.embedding_length || out->rows != c.vocab_size ||
        c.embedding_length > kFusedNormMaxDim) {
        int rc = gh_rmsnorm_x(m->b, enc, normed_row, xrow, &m->output_norm, c.embedding_length,
                              c.rms_epsilon, 1);
        if (!rc) rc = gh_logits(m->b, enc, &m->logits, normed_row, out, c.embedding_length, c.vocab_size);
        return rc;
    }
    const GemvSeg lg{out, m->logits.addr, GH_EPI_F32};
    return latch_rc(enc, op_gemv(m->b, &lg, 1, xrow, 1, 0, nullptr, 0, nullptr, &m->output_norm,
                                 c.rms_epsilon));
}

bool weights_ready(const gh_model* m) {
    if (!m->token_embd.addr || !m->output_norm.addr) return false;
    for (const auto& l : m->layers)
        for (const gh_buf& w : l)
            if (!w.addr) return false;
    return true;
}

// Record one decode step reading token and position from m->scalars (graph-capturable).
int record_step(gh_model* m, gh_encoder* enc) {
    const gh_model_config& c = m->cfg;
    const void* pos_ptr = (const void*)m->scalars.addr;
    const void* tok_ptr = (const void*)(m->scalars.addr + 4);
    int rc = op_embed(m->b, &m->dec.x, &m->token_embd, 0, c.embedding_length, tok_ptr);
    for (uint32_t li = 0; li < c.block_count && !rc; ++li) rc = layer(m, enc, m->dec, li, 0, 1, pos_ptr);
    if (!rc) rc = tail(m, enc, &m->dec.x, &m->dec.normed);
    // the argmax's final pass also stores it in history[pos] and advances (token, pos)
    if (!rc) rc = op_argmax(m->b, &m->logits, c.vocab_size, (void*)(m->scalars.addr + 8), nullptr,
                            (void*)m->scalars.addr, (void*)m->history.addr);
    return rc;
}

// End (exclusive) of decode position range k; the range of position pos.
uint32_t step_range_end(const gh_model* m, uint32_t k) {
    const uint32_t ctx = m->kv.context;
    if (m->b->attn_splits || k + 1 >= kStepRanges) return ctx;
    return std::min(kStepRangeEnds[k], ctx);
}

uint32_t step_range(const gh_model* m, uint32_t pos) {
    uint32_t k = 0;
    while (k + 1 < kStepRanges && pos >= step_range_end(m, k)) ++k;
    return k;
}

void destroy_steps(gh_model* m) {
    for (StepGraph& g : m->steps) {
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
        if (g.graph) (void)hipGraphDestroy(g.graph);
        g = StepGraph{};
    }
}

// The step graph of position range k, captured on first use and again after the backend's
// workspace or RoPE table moved.
int ensure_step(gh_model* m, uint32_t k) {
    gh_backend* b = m->b;
    StepGraph& sg = m->steps[k];
    if (sg.exec && sg.gen != b->gen) {
        (void)hipGraphExecDestroy(sg.exec);
        (void)hipGraphDestroy(sg.graph);
        sg = StepGraph{};
    }
    if (sg.exec) return GH_OK;
    // size the attention partials and merge counters for the whole context's split count in
    // force now (gh_set_attention_splits may have raised it since gh_model_create), so that no
    // range's capture grows them (which would move the workspace under the other ranges'
    // graphs): nothing may grow while the capture records
    const uint32_t splits = attention_splits(b, m->kv.context, m->cfg.kv_head_count, 1);
    int rc = ensure_workspace(b, attention_workspace(1, m->cfg.head_count, splits));
    if (!rc) rc = ensure_counters(b, m->cfg.kv_head_count);
    if (rc) return rc;
    gh_encoder* enc = nullptr;
    rc = gh_begin(b, &enc);
    if (rc) return rc;
    rc = hip_check(b, hipStreamBeginCapture(b->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    if (!rc) {
        b->capturing = true;
        m->step_len = step_range_end(m, k);
        int rec = record_step(m, enc);
        m->step_len = 0;
        b->capturing = false;
        hipGraph_t g = nullptr;
        int end = hip_check(b, hipStreamEndCapture(b->stream, &g), "hipStreamEndCapture");
        rc = rec ? rec : end;
        if (!rc) rc = hip_check(b, hipGraphInstantiate(&sg.exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
        if (rc && g) (void)hipGraphDestroy(g);
        else sg.graph = g;
        sg.gen = b->gen;
    }
    b->enc_open = false;
    return rc;
}

// Runs `steps` decode steps from (token, pos): the step graphs of the positions' ranges
// replayed, or with GH_MODEL_NO_GRAPH the same kernels launched on the stream. Each step leaves
// its logits, its argmax in history[pos] and the next (token, pos) in m->scalars, from which
// the next step (in the same graph or the next range's) continues.
int run_steps(gh_model* m, uint32_t token, uint32_t pos, uint32_t steps) {
    gh_backend* b = m->b;
    const uint32_t init[4] = {pos, token, 0, 0};
    int rc = GH_OK;
    if (m->cfg.flags & GH_MODEL_NO_GRAPH) {
        rc = gh_upload(b, &m->scalars, 0, init, sizeof(init));
        gh_encoder* enc = nullptr;
        if (!rc) rc = gh_begin(b, &enc);
        for (uint32_t i = 0; i < steps && !rc; ++i) {
            m->step_len = step_range_end(m, step_range(m, pos + i));  // the graph's split grid
            rc = record_step(m, enc);
        }
        m->step_len = 0;
        if (enc) {
            int rs = gh_submit(b, enc);
            rc = rc ? rc : rs;
        }
        m->last_rows = 1;
        m->last_prefill = false;
        return rc;
    }
    // every range the steps cross is captured before the first replay; a capture that grew the
    // workspace (which moves it) leaves the ranges captured before it stale, so they are
    // captured again (the second pass grows nothing: every capture sizes for the context)
    const uint32_t k0 = step_range(m, pos), k1 = step_range(m, pos + steps - 1);
    for (int pass = 0; pass < 2 && !rc; ++pass)
        for (uint32_t k = k0; k <= k1 && !rc; ++k) rc = ensure_step(m, k);
    for (uint32_t k = k0; k <= k1 && !rc; ++k)
        if (m->steps[k].gen != b->gen) rc = fail(b, GH_E_STATE, "decode: step graphs kept moving");
    if (!rc) rc = gh_upload(b, &m->scalars, 0, init, sizeof(init));
    for (uint32_t i = 0; i < steps && !rc; ++i)
        rc = hip_check(b, hipGraphLaunch(m->steps[step_range(m, pos + i)].exec, b->stream), "hipGraphLaunch");
    m->last_rows = 1;
    m->last_prefill = false;
    return rc;
}

// The chunks of one gh_model_prefill call (prefill::prefill, encode.rs:16-106) over the
// prompt ids already on the device: embed, the layers, and the tail on the last chunk's last
// row.
int prefill_chunks(gh_model* m, uint32_t n, uint32_t base) {
    const gh_model_config& c = m->cfg;
    const uint32_t cap = c.prefill_rows;
    const uint64_t d = c.embedding_length;
    for (uint32_t off = 0; off < n; off += cap) {
        const uint32_t rows = std::min(cap, n - off);
        gh_encoder* enc = nullptr;
        int rc = gh_begin(m->b, &enc);
        if (rc) return rc;
        rc = latch_rc(enc, op_embed_rows(m->b, &m->pre.x, &m->token_embd, (const void*)(m->prompt.addr + (uint64_t)off * 4),
                                         rows, c.embedding_length));
        bool normed = false;
        for (uint32_t li = 0; li < c.block_count && !rc; ++li)
            rc = layer(m, enc, m->pre, li, base + off, rows, nullptr, &normed);
        if (!rc && off + rows == n) {  // the tail belongs to the last chunk's last row
            gh_buf xr, nr;
            rc = gh_view(m->b, &m->pre.x, (rows - 1) * d * 4, d * 4, &xr);
            if (!rc) rc = gh_view(m->b, &m->pre.normed, (rows - 1) * d * 2, d * 2, &nr);
            if (!rc) rc = tail(m, enc, &xr, &nr);
        }
        int rs = gh_submit(m->b, enc);
        if (rc || rs) return rc ? rc : rs;
        m->last_rows = rows;
        m->last_prefill = true;
    }
    return GH_OK;
}

}  // namespace

extern "C" {

uint32_t gh_prefill_rows(const gh_backend* b, uint32_t block_count, uint32_t context) {
    (void)b;
    (void)block_count;
    // One policy for every depth: 2048-row chunks. Measured on the 8B shape (34 blocks):
    // 2048-token prompts 38.7K tok/s in one chunk vs 29.3K in 512-row chunks; 8192-token
    // prompts 35.6K tok/s vs 36.4K with 4096-row chunks and 24.2K with 512 (each chunk
    // streams every weight once, and the MFMA GEMM's efficiency grows with the rows). The
    // scratch for 2048 rows is ~245 MB on the 8B shape. Capped by the context.
    return std::max<uint32_t>(1, std::min<uint32_t>(2048, context));
}

int gh_model_create(gh_backend* b, const gh_model_config* cfg, gh_model** out) {
    if (!b || !cfg || !out) return GH_E_INVALID;
    *out = nullptr;
    gh_model_config c = *cfg;
    if (c.prefill_rows == 0) c.prefill_rows = gh_prefill_rows(b, c.block_count, c.kv_context);
    if (c.block_count == 0 || c.embedding_length % 256 || c.feed_forward_length % 256 ||
        c.head_count == 0 || c.kv_head_count == 0 || c.head_count % c.kv_head_count ||
        c.key_length != 128 || c.value_length != 128 || c.vocab_size == 0 || c.kv_context == 0 ||
        c.prefill_rows == 0 || (c.head_count * c.value_length) % 256 || !yarn_valid(&c.yarn) ||
        c.yarn.rope_dim > c.key_length)
        return fail(b, GH_E_INVALID, "model: unsupported shape");
    auto* m = new gh_model();
    m->b = b;
    m->cfg = c;
    m->layers.assign(c.block_count, std::array<gh_buf, 9>{});
    m->kv.scheme = GH_KV_F16;
    m->kv.block_count = c.block_count;
    m->kv.context = c.kv_context;
    m->kv.kv_heads = c.kv_head_count;
    m->kv.head_dim = c.key_length;
    m->kv.value_dim = c.value_length;
    // kv_cache::alloc_shape (kv_cache/mod.rs:70-114); layout::buffer_bytes (f16)
    const uint64_t kv_bytes = (uint64_t)c.block_count * c.kv_context * c.kv_head_count * c.key_length * 2;
    int rc = alloc(m, kv_bytes, &m->kv.k);
    if (!rc) rc = alloc(m, kv_bytes, &m->kv.v);
    if (!rc) rc = alloc_scratch(m, 1, &m->dec);
    if (!rc) rc = alloc_scratch(m, c.prefill_rows, &m->pre);
    if (!rc) rc = alloc(m, (uint64_t)c.vocab_size * 4, &m->logits);
    if (!rc) rc = alloc(m, 16, &m->scalars);
    if (!rc) rc = alloc(m, (uint64_t)c.kv_context * 4, &m->history);
    if (!rc) rc = alloc(m, (uint64_t)c.kv_context * 4, &m->prompt);
    if (!rc) rc = ensure_rope(b, m->rope, &c.yarn, c.kv_context);
    // partials for a decode step and for one prefill chunk
    const uint32_t dsplits = attention_splits(b, c.kv_context, c.kv_head_count, 1);
    if (!rc) rc = ensure_workspace(b, attention_workspace(1, c.head_count, dsplits));
    if (!rc) rc = ensure_counters(b, c.kv_head_count);
    if (rc) {
        gh_model_destroy(m);
        return rc;
    }
    *out = m;
    return GH_OK;
}

void gh_model_destroy(gh_model* m) {
    if (!m) return;
    free_w16(m);
    destroy_steps(m);
    for (gh_buf& buf : m->owned) gh_free_buffer(m->b, &buf);
    for (auto& l : m->layers)
        for (gh_buf& w : l)
            if (w.addr) gh_free_buffer(m->b, &w);
    for (gh_buf* w : {&m->token_embd, &m->output_norm, &m->output})
        if (w->addr) gh_free_buffer(m->b, w);
    (void)hipStreamSynchronize(m->b->stream);
    free_rope(m->rope);
    delete m;
}

int gh_model_load_tensor(gh_model* m, uint32_t layer_index, uint32_t tensor, uint32_t format,
                         const void* bytes, uint64_t len) {
    if (!m) return GH_E_INVALID;
    const gh_model_config& c = m->cfg;
    uint32_t in = 0, out = 0;
    gh_buf* slot = nullptr;
    const bool norm = tensor == GH_T_ATTN_NORM || tensor == GH_T_FFN_NORM || tensor == GH_T_OUTPUT_NORM;
    if (layer_index == kNoLayer) {
        switch (tensor) {
            case GH_T_TOKEN_EMBD: in = c.embedding_length; out = c.vocab_size; slot = &m->token_embd; break;
            case GH_T_OUTPUT_NORM: in = c.embedding_length; out = 1; slot = &m->output_norm; break;
            case GH_T_OUTPUT: in = c.embedding_length; out = c.vocab_size; slot = &m->output; break;
            default: return fail(m->b, GH_E_INVALID, "model: unknown global tensor");
        }
    } else {
        if (layer_index >= c.block_count || tensor > GH_T_FFN_DOWN) return fail(m->b, GH_E_INVALID, "model: unknown layer tensor");
        const uint32_t d = c.embedding_length;
        switch (tensor) {
            case GH_T_ATTN_NORM: case GH_T_FFN_NORM: in = d; out = 1; break;
            case GH_T_ATTN_Q: in = d; out = c.head_count * c.key_length; break;
            case GH_T_ATTN_K: in = d; out = c.kv_head_count * c.key_length; break;
            case GH_T_ATTN_V: in = d; out = c.kv_head_count * c.value_length; break;
            case GH_T_ATTN_OUTPUT: in = c.head_count * c.value_length; out = d; break;
            case GH_T_FFN_GATE: case GH_T_FFN_UP: in = d; out = c.feed_forward_length; break;
            case GH_T_FFN_DOWN: in = c.feed_forward_length; out = d; break;
        }
        slot = &m->layers[layer_index][tensor];
    }
    if (norm != (format == GH_FMT_F32 || format == GH_FMT_F16))
        return fail(m->b, GH_E_UNSUPPORTED, "model: norms are F32/F16, matrices Q4_K/Q6_K");
    free_w16(m);  // made again from the new weights by the next long prefill
    m->w16_failed = false;
    if (slot->addr) gh_free_buffer(m->b, slot);
    destroy_steps(m);
    return gh_load_weight(m->b, format, bytes, len, in, out, slot);
}

int gh_model_token(gh_model* m, uint32_t token, uint32_t pos) {
    if (!m) return GH_E_INVALID;
    const gh_model_config& c = m->cfg;
    if (!weights_ready(m)) return fail(m->b, GH_E_STATE, "model: weights not loaded");
    if (pos >= c.context_length || pos >= m->kv.context) return fail(m->b, GH_E_RANGE, "model: position beyond context");
    if (token >= c.vocab_size) return fail(m->b, GH_E_RANGE, "model: token beyond vocabulary");
    gh_encoder* enc = nullptr;
    int rc = gh_begin(m->b, &enc);
    if (rc) return rc;
    rc = gh_embed(m->b, enc, &m->dec.x, &m->token_embd, token, c.embedding_length);
    for (uint32_t li = 0; li < c.block_count && !rc; ++li) rc = layer(m, enc, m->dec, li, pos, 1, nullptr);
    if (!rc) rc = tail(m, enc, &m->dec.x, &m->dec.normed);
    int rs = gh_submit(m->b, enc);
    m->last_rows = 1;
    m->last_prefill = false;
    return rc ? rc : rs;
}

int gh_model_prefill(gh_model* m, const uint32_t* tokens, uint32_t n, uint32_t base) {
    if (!m || !tokens) return GH_E_INVALID;
    const gh_model_config& c = m->cfg;
    if (n == 0) return fail(m->b, GH_E_INVALID, "model: empty prompt");
    if (!weights_ready(m)) return fail(m->b, GH_E_STATE, "model: weights not loaded");
    if ((uint64_t)base + n > m->kv.context || (uint64_t)base + n > c.context_length)
        return fail(m->b, GH_E_RANGE, "model: prompt beyond context");
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] >= c.vocab_size) return fail(m->b, GH_E_RANGE, "model: token beyond vocabulary");
    const uint32_t cap = c.prefill_rows;
    // the chunk's embedding rows in one launch from the token ids on the device (the values
    // of embed per row, encode.rs:16-106, without a launch per token)
    int urc = gh_upload(m->b, &m->prompt, 0, tokens, (uint64_t)n * 4);
    const bool copies = std::min(cap, n) >= kGemmTallTokens;
    if (!urc && copies) urc = ensure_w16(m);
    if (urc) return urc;
    set_w16(m, copies);
    int rc = prefill_chunks(m, n, base);
    if (rc == GH_E_OOM && copies && !m->w16.empty()) {
        // the copies crowded out this prefill's workspace: drop them for good and run the
        // prompt again dequantizing (every chunk rewrites the same cache rows)
        free_w16(m);
        m->w16_failed = true;
        m->b->err.clear();
        rc = prefill_chunks(m, n, base);
    }
    return rc;
}

int gh_model_read_logits(gh_model* m, float* dst) {
    if (!m || !dst) return GH_E_INVALID;
    return gh_read_logits(m->b, &m->logits, m->cfg.vocab_size, dst);
}

int gh_model_read_argmax(gh_model* m, uint32_t* out) {
    if (!m || !out) return GH_E_INVALID;
    return gh_read_argmax(m->b, &m->logits, m->cfg.vocab_size, out);
}

int gh_model_decode_greedy(gh_model* m, uint32_t token, uint32_t pos, uint32_t steps,
                           uint32_t* tokens_out) {
    if (!m || (steps && !tokens_out)) return GH_E_INVALID;
    const gh_model_config& c = m->cfg;
    if (!weights_ready(m)) return fail(m->b, GH_E_STATE, "model: weights not loaded");
    if (token >= c.vocab_size) return fail(m->b, GH_E_RANGE, "model: token beyond vocabulary");
    if ((uint64_t)pos + steps > m->kv.context || (uint64_t)pos + steps > c.context_length)
        return fail(m->b, GH_E_RANGE, "model: decode beyond context");
    if (steps == 0) return GH_OK;
    int rc = run_steps(m, token, pos, steps);
    if (!rc) rc = gh_download(m->b, &m->history, (uint64_t)pos * 4, tokens_out, (uint64_t)steps * 4);
    return rc;
}

int gh_model_read_topk(gh_model* m, uint64_t k, uint32_t* idx, float* val, uint64_t* count) {
    if (!m) return GH_E_INVALID;
    return gh_read_topk(m->b, &m->logits, m->cfg.vocab_size, k, idx, val, count);
}

int gh_model_generate(gh_model* m, const uint32_t* prompt, uint32_t n_prompt, const gh_sampling* p,
                      uint32_t max_tokens, uint32_t eos, uint32_t* out, uint32_t* n_out) {
    if (!m || !prompt || !p || !n_out || (max_tokens && !out)) return GH_E_INVALID;
    *n_out = 0;
    const gh_model_config& c = m->cfg;
    const uint64_t context = std::min<uint64_t>(c.context_length, m->kv.context);
    if (n_prompt == 0) return fail(m->b, GH_E_INVALID, "generate: empty prompt");
    if (n_prompt > context) return fail(m->b, GH_E_RANGE, "generate: prompt beyond context");
    int rc = gh_model_prefill(m, prompt, n_prompt, 0);
    if (rc) return rc;
    uint32_t k = 0;
    const int path = gh_sampling_plan(p, &k);
    uint64_t rng = gh_rng_seed(p->seed);
    std::vector<uint32_t> recent(prompt, prompt + n_prompt);
    std::vector<uint32_t> idx;
    std::vector<float> val;
    uint32_t produced = 0;
    while (produced < max_tokens && n_prompt + produced < context) {
        uint32_t token = 0;
        if (path == GH_SAMPLE_GREEDY) {
            rc = gh_model_read_argmax(m, &token);
        } else if (path == GH_SAMPLE_TOPK) {
            // the raw top-k (read_topk's order), scaled by 1/temperature, straight into the
            // shared tail (generation/mod.rs:113-120)
            idx.resize(k);
            val.resize(k);
            uint64_t cnt = 0;
            rc = gh_model_read_topk(m, k, idx.data(), val.data(), &cnt);
            const float inv = 1.0f / p->temperature;
            for (uint64_t i = 0; i < cnt; ++i) val[i] *= inv;
            if (!rc) rc = gh_sample_from_candidates(idx.data(), val.data(), cnt, p, &rng, &token);
        } else {
            val.resize(c.vocab_size);
            rc = gh_model_read_logits(m, val.data());
            if (!rc) rc = gh_sample(val.data(), c.vocab_size, p, recent.data(), recent.size(), &rng, &token);
        }
        if (rc) return rc;
        if (token == eos) break;
        out[produced++] = token;
        *n_out = produced;
        recent.push_back(token);
        if (produced < max_tokens && n_prompt + produced < context) {
            rc = run_steps(m, token, n_prompt + produced - 1, 1);
            if (rc) return rc;
        }
    }
    return GH_OK;
}

int gh_model_kv(gh_model* m, gh_kv* out) {
    if (!m || !out) return GH_E_INVALID;
    *out = m->kv;
    return GH_OK;
}

int gh_model_read_x(gh_model* m, float* dst) {
    if (!m || !dst) return GH_E_INVALID;
    const uint64_t d = m->cfg.embedding_length;
    const gh_buf& x = m->last_prefill ? m->pre.x : m->dec.x;
    const uint64_t off = m->last_prefill ? (uint64_t)(m->last_rows - 1) * d * 4 : 0;
    return gh_download(m->b, &x, off, dst, d * 4);
}

int gh_model_weight(gh_model* m, uint32_t layer_index, uint32_t tensor, gh_buf* out) {
    if (!m || !out) return GH_E_INVALID;
    const gh_buf* w = nullptr;
    if (layer_index == kNoLayer) {
        if (tensor == GH_T_TOKEN_EMBD) w = &m->token_embd;
        else if (tensor == GH_T_OUTPUT_NORM) w = &m->output_norm;
        else if (tensor == GH_T_OUTPUT) w = &m->output;
    } else if (layer_index < m->cfg.block_count && tensor <= GH_T_FFN_DOWN) {
        w = &m->layers[layer_index][tensor];
    }
    if (!w || !w->addr) return fail(m->b, GH_E_INVALID, "model: no such tensor loaded");
    *out = *w;
    return GH_OK;
}

}  // extern "C"

// gh_oracle graph restatement (test infrastructure): the pinned Ministral op order and FP16
// rounding boundaries of family/mistral/graph/{forward,block,mlp,tail}.rs and
// graph/prefill/{encode,layer}.rs, executed over host buffers with the oracle's ops.
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "gh_oracle.h"
#include "internal.h"

using namespace gho;

struct gho_model {
    gho_model_cfg cfg;
    gho_tensor token_embd, output_norm, output;
    std::vector<gho_tensor> layers;
    uint32_t kv_context;
    std::vector<uint16_t> kc, vc;  // [layer][kv_context][kv_heads][head_dim]
    std::vector<float> logits;
    std::vector<float> last_x;
    // Op trace (the shape-recorder protocol of family/mistral/graph/shape.rs:120-360): each op
    // records the name of the tensor it was handed (looked up by address, so a wiring mistake
    // shows up as the wrong name), or its op name when it takes no tensor.
    bool tracing = false;
    std::vector<std::string> trace;
    std::map<const void*, std::string> names;
    std::string joined;
    int plant = GHO_PLANT_NONE;  // a planted mistake (tests of the checks' power only)
};

namespace {
const uint16_t* f16p(const gho_tensor& t) { return (const uint16_t*)t.bytes; }

void rec(gho_model* m, const std::string& op) {
    if (m->tracing) m->trace.push_back(op);
}
void rec(gho_model* m, const gho_tensor& t) {
    if (!m->tracing) return;
    auto it = m->names.find(t.bytes);
    m->trace.push_back(it == m->names.end() ? std::string("?") : it->second);
}

// kv_cache::append_batch (kv_cache/mod.rs:133-177) + kv_write_f16 (attention/write.rs:50-63).
void kv_append(gho_model* m, size_t layer, size_t pos, const uint16_t* k, const uint16_t* v,
               size_t rows) {
    const auto& c = m->cfg;
    size_t elems = rows * c.kv_head_count * c.key_length;
    size_t off = gho_kv_payload_offset(layer, pos, c.kv_head_count, c.key_length, m->kv_context) / 2;
    std::memcpy(m->kc.data() + off, k, elems * 2);
    size_t voff =
        gho_kv_payload_offset(layer, pos, c.kv_head_count, c.value_length, m->kv_context) / 2;
    std::memcpy(m->vc.data() + voff, v, rows * c.kv_head_count * c.value_length * 2);
}

// One layer for `rows` packed tokens at absolute positions base.. (prefill/layer.rs:18-122);
// rows == 1 is block::record (block.rs:17-107) with matmul_batched(n=1) == matmul.
void layer_rows(gho_model* m, size_t li, size_t base, size_t rows, std::vector<float>& x) {
    const auto& c = m->cfg;
    const gho_tensor* t = &m->layers[li * GHO_LAYER_TENSORS];
    size_t d = c.embedding_length, ffn = c.feed_forward_length;
    size_t qw = c.head_count * c.key_length, kw = c.kv_head_count * c.key_length;
    size_t vw = c.kv_head_count * c.value_length, aw = c.head_count * c.value_length;
    std::vector<uint16_t> normed(rows * d), q(rows * qw), k(rows * kw), v(rows * vw);
    std::vector<uint16_t> attn(rows * aw), proj(rows * d);
    rec(m, t[GHO_ATTN_NORM]);
    gho_rmsnorm_x(normed.data(), x.data(), f16p(t[GHO_ATTN_NORM]), d, c.rms_epsilon, rows);
    rec(m, t[GHO_ATTN_Q]);
    gho_matmul_batched(t[GHO_ATTN_Q].format, q.data(), normed.data(), t[GHO_ATTN_Q].bytes, d, qw, rows);
    rec(m, t[GHO_ATTN_K]);
    gho_matmul_batched(t[GHO_ATTN_K].format, k.data(), normed.data(), t[GHO_ATTN_K].bytes, d, kw, rows);
    rec(m, t[GHO_ATTN_V]);
    gho_matmul_batched(t[GHO_ATTN_V].format, v.data(), normed.data(), t[GHO_ATTN_V].bytes, d, vw, rows);
    // rope_yarn_batched default (contract.rs:187-246): per row, Q then K at base + row.
    rec(m, rows == 1 ? "rope_q" : "rope_batched");
    if (rows == 1) rec(m, "rope_k");
    // the role only selects the post-scale (rope.rs:84-100), so a planted role swap is
    // exactly a post-scale mistake
    const int q_role = m->plant == GHO_PLANT_NO_POST_SCALE_ON_Q ? 1 : 0;
    const int k_role = m->plant == GHO_PLANT_POST_SCALE_ON_K ? 0 : 1;
    for (size_t r = 0; r < rows; ++r) {
        gho_rope_yarn(q.data() + r * qw, c.head_count, c.key_length, base + r, &c.yarn, q_role);
        gho_rope_yarn(k.data() + r * kw, c.kv_head_count, c.key_length, base + r, &c.yarn, k_role);
    }
    rec(m, "kv_write");
    kv_append(m, li, base, k.data(), v.data(), rows);
    rec(m, rows == 1 ? "attention" : "attention_prefill");
    if (rows == 1)
        gho_attention_decode(attn.data(), q.data(), m->kc.data(), m->vc.data(), c.key_length,
                             c.value_length, c.kv_head_count, c.head_count, base, li, m->kv_context);
    else
        gho_attention_prefill(attn.data(), q.data(), m->kc.data(), m->vc.data(), c.key_length,
                              c.value_length, c.kv_head_count, c.head_count, base, rows, li,
                              m->kv_context);
    rec(m, t[GHO_ATTN_OUTPUT]);
    gho_matmul_batched(t[GHO_ATTN_OUTPUT].format, proj.data(), attn.data(),
                       t[GHO_ATTN_OUTPUT].bytes, aw, d, rows);
    rec(m, "residual");
    gho_residual_add(x.data(), proj.data(), d * rows);
    // mlp::record (mlp.rs:12-61)
    std::vector<uint16_t> gate(rows * ffn), up(rows * ffn), act(rows * ffn), ffn_out(rows * d);
    rec(m, t[GHO_FFN_NORM]);
    gho_rmsnorm_x(normed.data(), x.data(), f16p(t[GHO_FFN_NORM]), d, c.rms_epsilon, rows);
    rec(m, t[GHO_FFN_GATE]);
    gho_matmul_batched(t[GHO_FFN_GATE].format, gate.data(), normed.data(), t[GHO_FFN_GATE].bytes, d, ffn, rows);
    rec(m, t[GHO_FFN_UP]);
    gho_matmul_batched(t[GHO_FFN_UP].format, up.data(), normed.data(), t[GHO_FFN_UP].bytes, d, ffn, rows);
    rec(m, "silu_mul");
    gho_silu_mul(act.data(), gate.data(), up.data(), ffn * rows);
    rec(m, t[GHO_FFN_DOWN]);
    gho_matmul_batched(t[GHO_FFN_DOWN].format, ffn_out.data(), act.data(), t[GHO_FFN_DOWN].bytes, ffn, d, rows);
    rec(m, "residual");
    gho_residual_add(x.data(), ffn_out.data(), d * rows);
}

// tail::record_buffers (tail.rs:22-59): output_norm then FP32 logits (dedicated or tied).
void tail(gho_model* m, const float* xrow) {
    const auto& c = m->cfg;
    size_t d = c.embedding_length;
    std::vector<uint16_t> normed(d);
    rec(m, m->output_norm);
    gho_rmsnorm_x(normed.data(), xrow, f16p(m->output_norm), d, c.rms_epsilon, 1);
    const gho_tensor& out = m->output.bytes ? m->output : m->token_embd;
    if (m->tracing) {
        rec(m, out);
        m->trace.back() = "logits:" + m->trace.back();
    }
    gho_logits(out.format, m->logits.data(), normed.data(), out.bytes, d, c.vocab_size);
}
}  // namespace

extern "C" {
gho_model* gho_model_create(const gho_model_cfg* cfg, const gho_tensor* token_embd,
                            const gho_tensor* output_norm, const gho_tensor* output,
                            const gho_tensor* layers, uint32_t kv_context) {
    auto* m = new gho_model();
    m->cfg = *cfg;
    m->token_embd = *token_embd;
    m->output_norm = *output_norm;
    m->output = output ? *output : gho_tensor{nullptr, 0};
    m->layers.assign(layers, layers + (size_t)cfg->block_count * GHO_LAYER_TENSORS);
    m->kv_context = kv_context;
    size_t kv = (size_t)cfg->block_count * kv_context * cfg->kv_head_count;
    m->kc.assign(kv * cfg->key_length, 0);
    m->vc.assign(kv * cfg->value_length, 0);
    m->logits.assign(cfg->vocab_size, 0.0f);
    // the reference shape recorder's tensor names (graph/shape.rs:57-120)
    static const char* kLayerNames[GHO_LAYER_TENSORS] = {"attn_norm", "q", "k", "v", "attn_out",
                                                         "ffn_norm", "gate", "up", "down"};
    for (size_t li = 0; li < cfg->block_count; ++li)
        for (size_t ti = 0; ti < GHO_LAYER_TENSORS; ++ti)
            m->names[m->layers[li * GHO_LAYER_TENSORS + ti].bytes] =
                "l" + std::to_string(li) + "." + kLayerNames[ti];
    m->names[m->token_embd.bytes] = "token_embd";
    m->names[m->output_norm.bytes] = "output_norm";
    if (m->output.bytes) m->names[m->output.bytes] = "output";
    return m;
}

void gho_model_destroy(gho_model* m) { delete m; }

// forward::token (forward.rs:68-83).
int gho_model_token(gho_model* m, uint32_t token, uint32_t pos) {
    const auto& c = m->cfg;
    if (pos >= c.context_length || pos >= m->kv_context) return -1;
    if (token >= c.vocab_size) return -1;
    std::vector<float> x(c.embedding_length);
    rec(m, "begin");
    rec(m, "embed");
    gho_embed(x.data(), m->token_embd.format, m->token_embd.bytes, token, c.embedding_length);
    for (size_t li = 0; li < c.block_count; ++li) layer_rows(m, li, pos, 1, x);
    tail(m, x.data());
    rec(m, "submit");
    m->last_x = x;
    return 0;
}

// prefill::prefill + record_batch (prefill/encode.rs:16-106): chunks of row_capacity rows;
// the tail runs only on the last chunk's last row.
int gho_model_prefill(gho_model* m, const uint32_t* tokens, uint32_t n, uint32_t base,
                      uint32_t row_capacity) {
    const auto& c = m->cfg;
    if (n == 0 || row_capacity == 0) return -1;
    if ((size_t)base + n > m->kv_context) return -1;
    size_t d = c.embedding_length;
    for (uint32_t off = 0; off < n; off += row_capacity) {
        uint32_t rows = std::min(row_capacity, n - off);
        std::vector<float> x(rows * d);
        for (uint32_t r = 0; r < rows; ++r) {
            if (tokens[off + r] >= c.vocab_size) return -1;
            gho_embed(x.data() + r * d, m->token_embd.format, m->token_embd.bytes, tokens[off + r], d);
        }
        for (size_t li = 0; li < c.block_count; ++li) layer_rows(m, li, base + off, rows, x);
        if (off + rows == n) {
            tail(m, x.data() + (rows - 1) * d);
            m->last_x.assign(x.begin() + (rows - 1) * d, x.begin() + rows * d);
        }
    }
    return 0;
}

const float* gho_model_logits(const gho_model* m) { return m->logits.data(); }
const uint16_t* gho_model_kv(const gho_model* m, int role) {
    return role == 0 ? m->kc.data() : m->vc.data();
}
const float* gho_model_x(const gho_model* m) { return m->last_x.data(); }

int gho_model_load_kv(gho_model* m, const uint16_t* k, const uint16_t* v, uint32_t src_context,
                      uint32_t positions) {
    const auto& c = m->cfg;
    if (positions > src_context || positions > m->kv_context) return -1;
    const size_t kr = (size_t)c.kv_head_count * c.key_length, vr = (size_t)c.kv_head_count * c.value_length;
    for (size_t l = 0; l < c.block_count; ++l) {
        std::memcpy(m->kc.data() + l * m->kv_context * kr, k + l * src_context * kr, positions * kr * 2);
        std::memcpy(m->vc.data() + l * m->kv_context * vr, v + l * src_context * vr, positions * vr * 2);
    }
    return 0;
}

void gho_model_set_trace(gho_model* m, int on) {
    m->tracing = on != 0;
    m->trace.clear();
}

int gho_model_set_plant(gho_model* m, int plant) {
    if (plant < GHO_PLANT_NONE || plant > GHO_PLANT_NO_POST_SCALE_ON_Q) return -1;
    m->plant = plant;
    return 0;
}

const char* gho_model_trace(gho_model* m) {
    m->joined.clear();
    for (const std::string& op : m->trace) m->joined += op + "\n";
    return m->joined.c_str();
}
}

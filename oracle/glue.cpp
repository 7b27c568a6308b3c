// gh_oracle elementwise glue, YaRN RoPE, read-back reductions and KV layout (test
// infrastructure). Restates backend/cpu/kernels/elementwise/*.rs, backend/rope.rs,
// backend/cpu/readback.rs and kv_cache/layout.rs (f16 scheme).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "gh_oracle.h"
#include "internal.h"

using namespace gho;

namespace {
constexpr float kPi = 3.14159265358979323846f;  // std::f32::consts::PI

// Yarn::validate, rope.rs:37-57.
bool yarn_valid(const gho_yarn* y) {
    if (y->rope_dim == 0 || y->rope_dim % 2 != 0) return false;
    if (y->original_context == 0) return false;
    const float v[6] = {y->freq_base, y->factor,         y->beta_fast,
                        y->beta_slow, y->log_multiplier, y->q_temperature_scale};
    for (float x : v)
        if (!std::isfinite(x) || x <= 0.0f) return false;
    return true;
}

// corr_dim, rope.rs:124-127.
float corr_dim(uint32_t rope_dim, uint32_t original_context, float rotations, float base) {
    float denom = rotations * 2.0f * kPi;
    return (float)rope_dim * std::log((float)original_context / denom) / (2.0f * std::log(base));
}

// yarn_ramp, rope.rs:130-133 (f32::clamp(0, 1)).
float yarn_ramp(float low, float high, size_t pair) {
    float y = ((float)pair - low) / std::fmax(high - low, 0.001f);
    float c = y < 0.0f ? 0.0f : (y > 1.0f ? 1.0f : y);
    return 1.0f - c;
}

// f32::total_cmp key (IEEE 754 totalOrder), used by the top-k comparator.
int32_t total_key(float f) {
    int32_t b;
    std::memcpy(&b, &f, 4);
    b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
    return b;
}
}  // namespace

extern "C" {

// rmsnorm_x, normalization.rs:12-40: sequential Σx², inverse = 1/sqrt(Σx²/dim + eps),
// out = (x * inverse) * w, narrowed to FP16.
void gho_rmsnorm_x(uint16_t* out, const float* x, const uint16_t* w16, size_t dim, float eps,
                   size_t rows) {
    std::vector<float> w(dim);
    f16_slice_to_f32(w16, w.data(), dim);
    std::vector<float> values(rows * dim);
    for_units(rows * dim, dim, [&](size_t row0, size_t start, size_t end) {
        for (size_t r = 0; r < (end - start) / dim; ++r) {
            const float* in = x + (row0 + r) * dim;
            float* o = values.data() + start + r * dim;
            float sum = 0.0f;
            for (size_t i = 0; i < dim; ++i) sum += in[i] * in[i];
            float inverse = 1.0f / std::sqrt(sum / (float)dim + eps);
            for (size_t i = 0; i < dim; ++i) o[i] = in[i] * inverse * w[i];
        }
    });
    f32_slice_to_f16(values.data(), out, values.size());
}

// silu_mul, activation.rs:16-29: out = f16( f16(g / (1 + exp(-g))) * u ).
void gho_silu_mul(uint16_t* out, const uint16_t* gate, const uint16_t* up, size_t n) {
    std::vector<float> values(n);
    for (size_t i = 0; i < n; ++i) {
        float g = f16_to_f32(gate[i]);
        float silu = g / (1.0f + std::exp(-g));
        values[i] = f16_to_f32(f32_to_f16(silu)) * f16_to_f32(up[i]);
    }
    f32_slice_to_f16(values.data(), out, n);
}

// residual_add, residual.rs:12-22: x[i] += f32(y[i]) over the first n elements.
void gho_residual_add(float* x, const uint16_t* y, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] += f16_to_f32(y[i]);
}

// embed, embedding.rs:12-24: dequantize row `token` into the FP32 residual.
int gho_embed(float* x, uint32_t format, const uint8_t* token_embd, size_t token, size_t embd) {
    return dequant_row(format, token_embd, token, embd, x);
}

// Yarn::pair, rope.rs:60-81.
int gho_yarn_pair(const gho_yarn* y, int role, size_t pair, size_t position, float* cos_out,
                  float* sin_out) {
    (void)role;  // role_scale is 1.0 for both roles (rope.rs:84-89)
    if (!yarn_valid(y) || pair >= y->rope_dim / 2) return -1;
    float freq_scale = 1.0f / y->factor;
    float theta_extrap =
        (float)position * std::pow(y->freq_base, -(2.0f * (float)pair) / (float)y->rope_dim);
    float theta_interp = freq_scale * theta_extrap;
    float start, end;
    gho_yarn_correction_dims(y, &start, &end);
    float ramp = yarn_ramp(start, end, pair);
    float theta = theta_interp * (1.0f - ramp) + theta_extrap * ramp;
    *cos_out = std::cos(theta) * 1.0f;
    *sin_out = std::sin(theta) * 1.0f;
    return 0;
}

// Yarn::post_scale, rope.rs:91-99.
float gho_yarn_post_scale(const gho_yarn* y, int role, size_t position) {
    if (role != 0) return 1.0f;
    float bucket = (float)(position / y->original_context);
    return std::log(bucket + 1.0f) * y->q_temperature_scale + 1.0f;
}

// Yarn::correction_dims, rope.rs:102-120.
void gho_yarn_correction_dims(const gho_yarn* y, float* start, float* end) {
    *start = std::fmax(
        std::floor(corr_dim(y->rope_dim, y->original_context, y->beta_fast, y->freq_base)), 0.0f);
    *end = std::fmin(
        std::ceil(corr_dim(y->rope_dim, y->original_context, y->beta_slow, y->freq_base)),
        (float)(y->rope_dim - 1));
}

// rope_yarn, cpu/kernels/elementwise/rope.rs:14-39: adjacent pairs, post-scale per role.
int gho_rope_yarn(uint16_t* x, size_t heads, size_t head_dim, size_t pos, const gho_yarn* y,
                  int role) {
    if (!yarn_valid(y)) return -1;
    size_t half = y->rope_dim / 2;
    std::vector<float> values(heads * head_dim);
    f16_slice_to_f32(x, values.data(), values.size());
    float scale = gho_yarn_post_scale(y, role, pos);
    for (size_t head = 0; head < heads; ++head) {
        size_t base = head * head_dim;
        for (size_t pair = 0; pair < half; ++pair) {
            float c, s;
            if (gho_yarn_pair(y, role, pair, pos, &c, &s) != 0) return -1;
            size_t first = base + pair * 2;
            float a = values[first], b = values[first + 1];
            values[first] = (a * c - b * s) * scale;
            values[first + 1] = (a * s + b * c) * scale;
        }
    }
    f32_slice_to_f16(values.data(), x, values.size());
    return 0;
}

// argmax_f32, readback.rs:45-55: strict `>`, lowest index wins; NaN never wins.
uint32_t gho_argmax(const float* l, size_t vocab) {
    size_t best = 0;
    float best_val = -INFINITY;
    for (size_t i = 0; i < vocab; ++i) {
        if (l[i] > best_val) {
            best_val = l[i];
            best = i;
        }
    }
    return (uint32_t)best;
}

// topk_f32, readback.rs:59-69: total order (logit desc by total_cmp, index asc).
size_t gho_topk(const float* l, size_t vocab, size_t k, uint32_t* idx, float* val) {
    std::vector<uint32_t> cand(vocab);
    for (size_t i = 0; i < vocab; ++i) cand[i] = (uint32_t)i;
    auto order = [&](uint32_t a, uint32_t b) {
        int32_t ka = total_key(l[a]), kb = total_key(l[b]);
        if (ka != kb) return ka > kb;
        return a < b;
    };
    k = std::min(k, vocab);
    if (k == 0) return 0;
    std::partial_sort(cand.begin(), cand.begin() + (ptrdiff_t)k, cand.end(), order);
    for (size_t i = 0; i < k; ++i) {
        idx[i] = cand[i];
        val[i] = l[cand[i]];
    }
    return k;
}

// layout::payload_offset / buffer_bytes, kv_cache/layout.rs:22-89, f16: 2 bytes/element.
uint64_t gho_kv_payload_offset(size_t layer, size_t pos, size_t kv_heads, size_t head_dim,
                               size_t context) {
    return (uint64_t)((layer * context + pos) * kv_heads) * (uint64_t)(head_dim * 2);
}
uint64_t gho_kv_buffer_bytes(size_t block_count, size_t context, size_t kv_heads,
                             size_t head_dim) {
    return (uint64_t)(block_count * context * kv_heads) * (uint64_t)(head_dim * 2);
}
}

// gh_oracle causal GQA attention over an FP16 KV cache (test infrastructure).
// Restates backend/cpu/kernels/attention/{mod,simd,paired}.rs for the f16 scheme: the
// three-pass softmax (max, exp/sum, weighted V) with the AVX2+F16C inner loops
// (simd.rs:37-262) the reference runs on x86_64 hosts with avx2+fma+f16c.
#include <immintrin.h>

#include <cmath>
#include <vector>

#include "gh_oracle.h"
#include "internal.h"

namespace gho {
namespace {

__attribute__((target("avx2"))) inline float hsum256(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s);
}

// dot_f16_x4_avx2 (simd.rs:147-186) with G queries; G=1 is dot_f16_avx2 (simd.rs:37-61),
// G=2 is dot_f16_x2_avx2 (simd.rs:101-138). Per-query order is identical for every G.
template <int G>
__attribute__((target("avx2,fma,f16c"))) inline void dot_gx(const float* const* q,
                                                            const uint16_t* k, size_t hd,
                                                            float* s) {
    __m256 acc[G];
    for (int g = 0; g < G; ++g) acc[g] = _mm256_setzero_ps();
    size_t d = 0;
    for (; d + 8 <= hd; d += 8) {
        __m256 kf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(k + d)));
        for (int g = 0; g < G; ++g) acc[g] = _mm256_fmadd_ps(_mm256_loadu_ps(q[g] + d), kf, acc[g]);
    }
    for (int g = 0; g < G; ++g) s[g] = hsum256(acc[g]);
    for (; d < hd; ++d) {
        float kf = f16_to_f32(k[d]);
        for (int g = 0; g < G; ++g) s[g] += q[g][d] * kf;
    }
}

// axpy_f16_x4_avx2 (simd.rs:225-262) with G outputs; G=1 axpy_f16_avx2 (simd.rs:67-92),
// G=2 axpy_f16_x2_avx2 (simd.rs:191-219).
template <int G>
__attribute__((target("avx2,fma,f16c"))) inline void axpy_gx(float* const* out, const float* w,
                                                             const uint16_t* v, size_t hd) {
    __m256 wv[G];
    for (int g = 0; g < G; ++g) wv[g] = _mm256_set1_ps(w[g]);
    size_t d = 0;
    for (; d + 8 <= hd; d += 8) {
        __m256 vf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(v + d)));
        for (int g = 0; g < G; ++g) {
            __m256 o = _mm256_loadu_ps(out[g] + d);
            _mm256_storeu_ps(out[g] + d, _mm256_fmadd_ps(wv[g], vf, o));
        }
    }
    for (; d < hd; ++d) {
        float vf = f16_to_f32(v[d]);
        for (int g = 0; g < G; ++g) out[g][d] += w[g] * vf;
    }
}

// attend / attend_pair / attend_quad (mod.rs:220-396): G query heads sharing kv head kvh.
template <int G>
void attend_g(const float* const* q, const uint16_t* kc, const uint16_t* vc, size_t key_dim,
              size_t value_dim, size_t kv_heads, size_t kvh, size_t layer, size_t context,
              float scale, float* const* out, std::vector<float>* scores, size_t len) {
    float m[G];
    for (int g = 0; g < G; ++g) m[g] = -INFINITY;
    for (size_t t = 0; t < len; ++t) {
        size_t kbase = ((layer * context + t) * kv_heads + kvh) * key_dim;
        float s[G];
        dot_gx<G>(q, kc + kbase, key_dim, s);
        for (int g = 0; g < G; ++g) {
            float sc = s[g] * scale;
            scores[g][t] = sc;
            m[g] = std::fmax(m[g], sc);  // f32::max (IEEE maxNum)
        }
    }
    float denom[G];
    for (int g = 0; g < G; ++g) denom[g] = 0.0f;
    for (size_t t = 0; t < len; ++t) {
        for (int g = 0; g < G; ++g) {
            float e = std::exp(scores[g][t] - m[g]);
            scores[g][t] = e;
            denom[g] += e;
        }
    }
    for (size_t t = 0; t < len; ++t) {
        size_t vbase = ((layer * context + t) * kv_heads + kvh) * value_dim;
        float w[G];
        for (int g = 0; g < G; ++g) w[g] = scores[g][t] / denom[g];
        axpy_gx<G>(out, w, vc + vbase, value_dim);
    }
}

// One (row, kv_head) unit of attention_decode_f16 / attention_prefill_f16 (mod.rs:486-570,
// mod.rs:628-720): groups of four, then pair, then single, each head's passes in fixed order.
void attend_unit(const float* qrow, const uint16_t* kc, const uint16_t* vc, size_t key_dim,
                 size_t value_dim, size_t kv_heads, size_t q_heads, size_t kvh, size_t layer,
                 size_t context, float scale, float* group_out, std::vector<float>* scores,
                 size_t len) {
    size_t group = q_heads / kv_heads;
    size_t gh = 0;
    while (gh + 3 < group) {
        size_t h0 = kvh * group + gh;
        const float* q[4] = {qrow + h0 * key_dim, qrow + (h0 + 1) * key_dim,
                             qrow + (h0 + 2) * key_dim, qrow + (h0 + 3) * key_dim};
        float* o[4] = {group_out + gh * value_dim, group_out + (gh + 1) * value_dim,
                       group_out + (gh + 2) * value_dim, group_out + (gh + 3) * value_dim};
        attend_g<4>(q, kc, vc, key_dim, value_dim, kv_heads, kvh, layer, context, scale, o,
                    scores, len);
        gh += 4;
    }
    while (gh + 1 < group) {
        size_t h0 = kvh * group + gh;
        const float* q[2] = {qrow + h0 * key_dim, qrow + (h0 + 1) * key_dim};
        float* o[2] = {group_out + gh * value_dim, group_out + (gh + 1) * value_dim};
        attend_g<2>(q, kc, vc, key_dim, value_dim, kv_heads, kvh, layer, context, scale, o,
                    scores, len);
        gh += 2;
    }
    if (gh < group) {
        size_t h = kvh * group + gh;
        const float* q[1] = {qrow + h * key_dim};
        float* o[1] = {group_out + gh * value_dim};
        attend_g<1>(q, kc, vc, key_dim, value_dim, kv_heads, kvh, layer, context, scale, o,
                    scores, len);
    }
}

}  // namespace
}  // namespace gho

using namespace gho;

extern "C" {

// attention_decode_f16, mod.rs:458-574: units are kv heads (stride group*value_dim).
void gho_attention_decode(uint16_t* out, const uint16_t* q16, const uint16_t* kc,
                          const uint16_t* vc, size_t key_dim, size_t value_dim, size_t kv_heads,
                          size_t q_heads, size_t pos, size_t layer, size_t context) {
    std::vector<float> q(q_heads * key_dim);
    f16_slice_to_f32(q16, q.data(), q.size());
    float scale = 1.0f / std::sqrt((float)key_dim);
    size_t group = q_heads / kv_heads;
    size_t unit = group * value_dim;
    std::vector<float> o(q_heads * value_dim, 0.0f);
    for_units(o.size(), unit, [&](size_t k0, size_t start, size_t end) {
        std::vector<float> scores[4];
        for (auto& s : scores) s.assign(pos + 1, 0.0f);
        for (size_t j = 0; j < (end - start) / unit; ++j) {
            size_t kvh = k0 + j;
            attend_unit(q.data(), kc, vc, key_dim, value_dim, kv_heads, q_heads, kvh, layer,
                        context, scale, o.data() + start + j * unit, scores, pos + 1);
        }
    });
    f32_slice_to_f16(o.data(), out, o.size());
}

// attention_prefill_f16, mod.rs:582-725. The paired AVX2 route (paired.rs:8-78) is asserted
// byte-identical to per-row decode by the reference (mod.rs:738-814), and the generic route
// calls the same `attend` family per (row, kv_head); both equal decode at pos = base + i.
void gho_attention_prefill(uint16_t* out, const uint16_t* q16, const uint16_t* kc,
                           const uint16_t* vc, size_t key_dim, size_t value_dim, size_t kv_heads,
                           size_t q_heads, size_t base, size_t n, size_t layer, size_t context) {
    std::vector<float> q(n * q_heads * key_dim);
    f16_slice_to_f32(q16, q.data(), q.size());
    float scale = 1.0f / std::sqrt((float)key_dim);
    size_t group = q_heads / kv_heads;
    size_t unit = group * value_dim;
    std::vector<float> o(n * q_heads * value_dim, 0.0f);
    for_units(o.size(), unit, [&](size_t u0, size_t start, size_t end) {
        size_t units = (end - start) / unit;
        if (units == 0) return;
        size_t max_pos = base + (u0 + units - 1) / kv_heads;
        std::vector<float> scores[4];
        for (auto& s : scores) s.assign(max_pos + 1, 0.0f);
        for (size_t j = 0; j < units; ++j) {
            size_t ui = u0 + j;
            size_t i = ui / kv_heads;
            size_t kvh = ui % kv_heads;
            size_t pos = base + i;
            attend_unit(q.data() + i * q_heads * key_dim, kc, vc, key_dim, value_dim, kv_heads,
                        q_heads, kvh, layer, context, scale, o.data() + start + j * unit, scores,
                        pos + 1);
        }
    });
    f32_slice_to_f16(o.data(), out, o.size());
}

// The serial scalar three-pass reference of the reference's parity test (mod.rs:876-913):
// scalar dot in d order, max, exp/sum, scalar weighted V. head_dim = key_dim = value_dim.
void gho_attention_decode_serial(uint16_t* out, const uint16_t* q16, const uint16_t* kc,
                                 const uint16_t* vc, size_t head_dim, size_t kv_heads,
                                 size_t q_heads, size_t pos, size_t layer, size_t context) {
    float scale = 1.0f / std::sqrt((float)head_dim);
    size_t group = q_heads / kv_heads;
    std::vector<float> expected(q_heads * head_dim, 0.0f);
    std::vector<float> scores(pos + 1);
    for (size_t h = 0; h < q_heads; ++h) {
        size_t kvh = h / group;
        size_t qbase = h * head_dim;
        float m = -INFINITY;
        for (size_t t = 0; t <= pos; ++t) {
            size_t kbase = ((layer * context + t) * kv_heads + kvh) * head_dim;
            float s = 0.0f;
            for (size_t d = 0; d < head_dim; ++d) s += f16_to_f32(q16[qbase + d]) * f16_to_f32(kc[kbase + d]);
            s *= scale;
            scores[t] = s;
            m = std::fmax(m, s);
        }
        float denom = 0.0f;
        for (size_t t = 0; t <= pos; ++t) {
            scores[t] = std::exp(scores[t] - m);
            denom += scores[t];
        }
        for (size_t t = 0; t <= pos; ++t) {
            float w = scores[t] / denom;
            size_t kbase = ((layer * context + t) * kv_heads + kvh) * head_dim;
            for (size_t d = 0; d < head_dim; ++d) expected[qbase + d] += w * f16_to_f32(vc[kbase + d]);
        }
    }
    f32_slice_to_f16(expected.data(), out, expected.size());
}
}

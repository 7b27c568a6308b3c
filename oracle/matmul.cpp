// gh_oracle fused Q4_K / Q6_K GEMV and batched GEMM (test infrastructure).
// Restates backend/cpu/kernels/matmul/{mod,q4k,q4k_simd,q6k,q6k_simd}.rs. On x86_64 with
// AVX2+FMA the reference executes the *_avx2 variants (q4k.rs:38-49, q6k.rs:67-77); they are
// restated here with the same intrinsics in the same order, so the FP32 results are the
// reference's bits on the same inputs.
#include <immintrin.h>

#include <cstring>
#include <vector>

#include "gh_oracle.h"
#include "internal.h"

namespace gho {

static inline float f16_at(const uint8_t* b) {
    return f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
}

// hsum256, q4k_simd.rs:321-331: (lo+hi) then two hadds.
__attribute__((target("avx2"))) static inline float hsum256(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s);
}

// row_dot_q4k_scalar, q4k.rs:58-96: per-sub-block partial, then acc += partial.
float row_dot_q4k_scalar(const float* a, const uint8_t* bytes, size_t row, size_t in_dim) {
    size_t nb = in_dim / 256;
    size_t base = row * nb * 144;
    float acc = 0.0f;
    for (size_t s = 0; s < nb; ++s) {
        const uint8_t* blk = bytes + base + s * 144;
        float d = f16_at(blk);
        float dmin = f16_at(blk + 2);
        const uint8_t* sco = blk + 4;
        const uint8_t* qso = blk + 16;
        size_t abase = s * 256;
        for (uint32_t sb = 0; sb < 8; ++sb) {
            uint32_t sc, mn;
            scale_min(sco, sb, &sc, &mn);
            float dl = d * (float)sc;
            float ml = dmin * (float)mn;
            size_t group = (sb / 2) * 32;
            bool hi = (sb & 1) == 1;
            size_t in0 = abase + sb * 32;
            float wbuf[32];
            for (size_t l = 0; l < 32; ++l) {
                uint32_t qv = qso[group + l];
                uint32_t q4 = hi ? (qv >> 4) : (qv & 0xF);
                wbuf[l] = dl * (float)q4 - ml;
            }
            float partial = 0.0f;
            for (size_t l = 0; l < 32; ++l) partial += a[in0 + l] * wbuf[l];
            acc += partial;
        }
    }
    return acc;
}

// row_dot_q4k_avx2, q4k_simd.rs:38-102: four chunk accumulators, fmsub dequant,
// low-nibble then high-nibble FMA per chunk, tree reduce (0+1)+(2+3).
__attribute__((target("avx2,fma"))) float row_dot_q4k_avx2(const float* a, const uint8_t* bytes,
                                                            size_t row, size_t in_dim) {
    size_t nb = in_dim / 256;
    size_t base = row * nb * 144;
    const __m256i mask = _mm256_set1_epi32(0xF);
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(),
                     _mm256_setzero_ps()};
    for (size_t s = 0; s < nb; ++s) {
        const uint8_t* blk = bytes + base + s * 144;
        float d = f16_at(blk);
        float dmin = f16_at(blk + 2);
        const uint8_t* sco = blk + 4;
        const uint8_t* qso = blk + 16;
        size_t abase = s * 256;
        for (uint32_t g = 0; g < 4; ++g) {
            uint32_t sc0, mn0, sc1, mn1;
            scale_min(sco, 2 * g, &sc0, &mn0);
            scale_min(sco, 2 * g + 1, &sc1, &mn1);
            __m256 dl0 = _mm256_set1_ps(d * (float)sc0);
            __m256 ml0 = _mm256_set1_ps(dmin * (float)mn0);
            __m256 dl1 = _mm256_set1_ps(d * (float)sc1);
            __m256 ml1 = _mm256_set1_ps(dmin * (float)mn1);
            size_t group = g * 32;
            size_t in_lo = abase + 2 * g * 32;
            size_t in_hi = abase + (2 * g + 1) * 32;
            for (size_t c = 0; c < 4; ++c) {
                const uint8_t* qp = qso + group + c * 8;
                __m256i v = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)qp));
                __m256i nlo = _mm256_and_si256(v, mask);
                __m256i nhi = _mm256_and_si256(_mm256_srli_epi32(v, 4), mask);
                __m256 wlo = _mm256_fmsub_ps(dl0, _mm256_cvtepi32_ps(nlo), ml0);
                __m256 whi = _mm256_fmsub_ps(dl1, _mm256_cvtepi32_ps(nhi), ml1);
                acc[c] = _mm256_fmadd_ps(_mm256_loadu_ps(a + in_lo + c * 8), wlo, acc[c]);
                acc[c] = _mm256_fmadd_ps(_mm256_loadu_ps(a + in_hi + c * 8), whi, acc[c]);
            }
        }
    }
    __m256 lo = _mm256_add_ps(acc[0], acc[1]);
    __m256 hi = _mm256_add_ps(acc[2], acc[3]);
    return hsum256(_mm256_add_ps(lo, hi));
}

// row_dot_q4k_avx2_batched, q4k_simd.rs:117-181: decode each sub-block once (four fmsub
// vectors), FMA chunks 0..3 into one 8-lane accumulator per token. The two-row kernel
// (q4k_simd.rs:203-318) is bit-identical to this per row, so it is not restated.
__attribute__((target("avx2,fma"))) void row_dot_q4k_avx2_batched(const float* a,
                                                                   const uint8_t* bytes, size_t row,
                                                                   size_t in_dim, float* out,
                                                                   size_t n, float* acc) {
    size_t nb = in_dim / 256;
    size_t base = row * nb * 144;
    const __m256i mask = _mm256_set1_epi32(0xF);
    std::memset(acc, 0, n * 8 * sizeof(float));
    for (size_t s = 0; s < nb; ++s) {
        const uint8_t* blk = bytes + base + s * 144;
        float d = f16_at(blk);
        float dmin = f16_at(blk + 2);
        const uint8_t* sco = blk + 4;
        const uint8_t* qso = blk + 16;
        size_t abase = s * 256;
        for (uint32_t sb = 0; sb < 8; ++sb) {
            uint32_t sc, mn;
            scale_min(sco, sb, &sc, &mn);
            __m256 dl = _mm256_set1_ps(d * (float)sc);
            __m256 ml = _mm256_set1_ps(dmin * (float)mn);
            size_t group = (sb / 2) * 32;
            bool hi = (sb & 1) == 1;
            size_t in0 = abase + sb * 32;
            __m256 w[4];
            for (size_t c = 0; c < 4; ++c) {
                __m256i v = _mm256_cvtepu8_epi32(
                    _mm_loadl_epi64((const __m128i*)(qso + group + c * 8)));
                __m256i nib = hi ? _mm256_and_si256(_mm256_srli_epi32(v, 4), mask)
                                 : _mm256_and_si256(v, mask);
                w[c] = _mm256_fmsub_ps(dl, _mm256_cvtepi32_ps(nib), ml);
            }
            for (size_t i = 0; i < n; ++i) {
                float* ap = acc + i * 8;
                __m256 ai = _mm256_loadu_ps(ap);
                const float* arow = a + i * in_dim + in0;
                ai = _mm256_fmadd_ps(_mm256_loadu_ps(arow), w[0], ai);
                ai = _mm256_fmadd_ps(_mm256_loadu_ps(arow + 8), w[1], ai);
                ai = _mm256_fmadd_ps(_mm256_loadu_ps(arow + 16), w[2], ai);
                ai = _mm256_fmadd_ps(_mm256_loadu_ps(arow + 24), w[3], ai);
                _mm256_storeu_ps(ap, ai);
            }
        }
    }
    for (size_t i = 0; i < n; ++i) out[i] = hsum256(_mm256_loadu_ps(acc + i * 8));
}

// row_dot_q6k_scalar, q6k.rs:31-64: single accumulator in unpack order,
// acc += ((d*scale)*q)*a.
float row_dot_q6k_scalar(const float* a, const uint8_t* bytes, size_t row, size_t in_dim) {
    size_t nsb = in_dim / 256;
    size_t base = row * nsb * 210;
    float acc = 0.0f;
    for (size_t s = 0; s < nsb; ++s) {
        const uint8_t* blk = bytes + base + s * 210;
        float d = f16_at(blk + 208);
        size_t abase = s * 256;
        for (size_t n = 0; n < 256; n += 128) {
            size_t seg = n / 128;
            const uint8_t* qlb = blk + seg * 64;
            const uint8_t* qhb = blk + 128 + seg * 32;
            const int8_t* scb = (const int8_t*)(blk + 192 + seg * 8);
            for (size_t l = 0; l < 32; ++l) {
                size_t is = l / 16;
                uint32_t lo0 = qlb[l], lo1 = qlb[l + 32], h = qhb[l];
                int32_t q1 = (int32_t)((lo0 & 0xF) | ((h & 3) << 4)) - 32;
                int32_t q2 = (int32_t)((lo1 & 0xF) | (((h >> 2) & 3) << 4)) - 32;
                int32_t q3 = (int32_t)((lo0 >> 4) | (((h >> 4) & 3) << 4)) - 32;
                int32_t q4 = (int32_t)((lo1 >> 4) | (((h >> 6) & 3) << 4)) - 32;
                size_t o = abase + n + l;
                acc += d * (float)scb[is] * (float)q1 * a[o];
                acc += d * (float)scb[is + 2] * (float)q2 * a[o + 32];
                acc += d * (float)scb[is + 4] * (float)q3 * a[o + 64];
                acc += d * (float)scb[is + 6] * (float)q4 * a[o + 96];
            }
        }
    }
    return acc;
}

// unpack_chunk, q6k_simd.rs:39-98: four 8-wide weight vectors (d*scale_k) * (q_k - 32).
__attribute__((target("avx2"))) static inline void q6k_unpack_chunk(const uint8_t* qlb,
                                                                     const uint8_t* qhb,
                                                                     const int8_t* scb, size_t is,
                                                                     size_t l, float d,
                                                                     __m256 w[4]) {
    const __m256i m4 = _mm256_set1_epi32(0xF);
    const __m256i m3 = _mm256_set1_epi32(3);
    const __m256i c32 = _mm256_set1_epi32(32);
    auto load8 = [](const uint8_t* p) {
        return _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)p));
    };
    __m256 dl1 = _mm256_set1_ps(d * (float)scb[is]);
    __m256 dl2 = _mm256_set1_ps(d * (float)scb[is + 2]);
    __m256 dl3 = _mm256_set1_ps(d * (float)scb[is + 4]);
    __m256 dl4 = _mm256_set1_ps(d * (float)scb[is + 6]);
    __m256i lo0 = load8(qlb + l);
    __m256i lo1 = load8(qlb + l + 32);
    __m256i h = load8(qhb + l);
    __m256i q1 = _mm256_sub_epi32(
        _mm256_or_si256(_mm256_and_si256(lo0, m4), _mm256_slli_epi32(_mm256_and_si256(h, m3), 4)),
        c32);
    __m256i q2 = _mm256_sub_epi32(
        _mm256_or_si256(_mm256_and_si256(lo1, m4),
                        _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(h, 2), m3), 4)),
        c32);
    __m256i q3 = _mm256_sub_epi32(
        _mm256_or_si256(_mm256_srli_epi32(lo0, 4),
                        _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(h, 4), m3), 4)),
        c32);
    __m256i q4 = _mm256_sub_epi32(
        _mm256_or_si256(_mm256_srli_epi32(lo1, 4),
                        _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(h, 6), m3), 4)),
        c32);
    w[0] = _mm256_mul_ps(dl1, _mm256_cvtepi32_ps(q1));
    w[1] = _mm256_mul_ps(dl2, _mm256_cvtepi32_ps(q2));
    w[2] = _mm256_mul_ps(dl3, _mm256_cvtepi32_ps(q3));
    w[3] = _mm256_mul_ps(dl4, _mm256_cvtepi32_ps(q4));
}

// row_dot_q6k_avx2, q6k_simd.rs:105-136: one accumulator per quant stream.
__attribute__((target("avx2,fma"))) float row_dot_q6k_avx2(const float* a, const uint8_t* bytes,
                                                            size_t row, size_t in_dim) {
    size_t nsb = in_dim / 256;
    size_t base = row * nsb * 210;
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(),
                     _mm256_setzero_ps()};
    for (size_t s = 0; s < nsb; ++s) {
        const uint8_t* blk = bytes + base + s * 210;
        float d = f16_at(blk + 208);
        size_t abase = s * 256;
        for (size_t n = 0; n < 256; n += 128) {
            size_t seg = n / 128;
            const uint8_t* qlb = blk + seg * 64;
            const uint8_t* qhb = blk + 128 + seg * 32;
            const int8_t* scb = (const int8_t*)(blk + 192 + seg * 8);
            for (size_t l = 0; l < 32; l += 8) {
                __m256 w[4];
                q6k_unpack_chunk(qlb, qhb, scb, l / 16, l, d, w);
                size_t o = abase + n + l;
                acc[0] = _mm256_fmadd_ps(_mm256_loadu_ps(a + o), w[0], acc[0]);
                acc[1] = _mm256_fmadd_ps(_mm256_loadu_ps(a + o + 32), w[1], acc[1]);
                acc[2] = _mm256_fmadd_ps(_mm256_loadu_ps(a + o + 64), w[2], acc[2]);
                acc[3] = _mm256_fmadd_ps(_mm256_loadu_ps(a + o + 96), w[3], acc[3]);
            }
        }
    }
    __m256 lo = _mm256_add_ps(acc[0], acc[1]);
    __m256 hi = _mm256_add_ps(acc[2], acc[3]);
    return hsum256(_mm256_add_ps(lo, hi));
}

// row_dot_q6k_avx2_batched, q6k_simd.rs:145-192 (row2_dot_q6k_avx2_batched is bit-identical
// per row, q6k_simd.rs:194-273).
__attribute__((target("avx2,fma"))) void row_dot_q6k_avx2_batched(const float* a,
                                                                   const uint8_t* bytes, size_t row,
                                                                   size_t in_dim, float* out,
                                                                   size_t n, float* acc) {
    size_t nsb = in_dim / 256;
    size_t base = row * nsb * 210;
    std::memset(acc, 0, n * 8 * sizeof(float));
    for (size_t s = 0; s < nsb; ++s) {
        const uint8_t* blk = bytes + base + s * 210;
        float d = f16_at(blk + 208);
        size_t abase = s * 256;
        for (size_t n2 = 0; n2 < 256; n2 += 128) {
            size_t seg = n2 / 128;
            const uint8_t* qlb = blk + seg * 64;
            const uint8_t* qhb = blk + 128 + seg * 32;
            const int8_t* scb = (const int8_t*)(blk + 192 + seg * 8);
            for (size_t l = 0; l < 32; l += 8) {
                __m256 w[4];
                q6k_unpack_chunk(qlb, qhb, scb, l / 16, l, d, w);
                size_t o = abase + n2 + l;
                for (size_t i = 0; i < n; ++i) {
                    float* ap = acc + i * 8;
                    __m256 ai = _mm256_loadu_ps(ap);
                    const float* ar = a + i * in_dim + o;
                    ai = _mm256_fmadd_ps(_mm256_loadu_ps(ar), w[0], ai);
                    ai = _mm256_fmadd_ps(_mm256_loadu_ps(ar + 32), w[1], ai);
                    ai = _mm256_fmadd_ps(_mm256_loadu_ps(ar + 64), w[2], ai);
                    ai = _mm256_fmadd_ps(_mm256_loadu_ps(ar + 96), w[3], ai);
                    _mm256_storeu_ps(ap, ai);
                }
            }
        }
    }
    for (size_t i = 0; i < n; ++i) out[i] = hsum256(_mm256_loadu_ps(acc + i * 8));
}

static float row_dot(uint32_t format, const float* a, const uint8_t* w, size_t row,
                     size_t in_dim) {
    return format == FMT_Q4_K ? row_dot_q4k_avx2(a, w, row, in_dim)
                              : row_dot_q6k_avx2(a, w, row, in_dim);
}

// q4k::matmul / q6k::matmul (q4k.rs:329-340, q6k.rs:140-151) and their logits twins
// (q4k.rs:344-355, q6k.rs:238-249): rows split by for_units with stride 1.
static void gemv(uint32_t format, float* y, const uint16_t* a_f16, const uint8_t* w,
                 size_t in_dim, size_t out_dim) {
    std::vector<float> a(in_dim);
    f16_slice_to_f32(a_f16, a.data(), in_dim);
    for_units(out_dim, 1, [&](size_t o0, size_t start, size_t end) {
        for (size_t k = 0; k < end - start; ++k) y[start + k] = row_dot(format, a.data(), w, o0 + k, in_dim);
    });
}

}  // namespace gho

using namespace gho;

extern "C" {
float gho_row_dot_q4k_scalar(const float* a, const uint8_t* w, size_t row, size_t in_dim) {
    return row_dot_q4k_scalar(a, w, row, in_dim);
}
float gho_row_dot_q4k_avx2(const float* a, const uint8_t* w, size_t row, size_t in_dim) {
    return row_dot_q4k_avx2(a, w, row, in_dim);
}
float gho_row_dot_q6k_scalar(const float* a, const uint8_t* w, size_t row, size_t in_dim) {
    return row_dot_q6k_scalar(a, w, row, in_dim);
}
float gho_row_dot_q6k_avx2(const float* a, const uint8_t* w, size_t row, size_t in_dim) {
    return row_dot_q6k_avx2(a, w, row, in_dim);
}
void gho_row_dot_q4k_avx2_batched(const float* a, const uint8_t* w, size_t row, size_t in_dim,
                                  float* out, size_t n) {
    std::vector<float> acc(n * 8);
    row_dot_q4k_avx2_batched(a, w, row, in_dim, out, n, acc.data());
}
void gho_row_dot_q6k_avx2_batched(const float* a, const uint8_t* w, size_t row, size_t in_dim,
                                  float* out, size_t n) {
    std::vector<float> acc(n * 8);
    row_dot_q6k_avx2_batched(a, w, row, in_dim, out, n, acc.data());
}

int gho_matmul(uint32_t format, uint16_t* out, const uint16_t* a, const uint8_t* w, size_t in_dim,
               size_t out_dim) {
    if (format != FMT_Q4_K && format != FMT_Q6_K) return -1;
    std::vector<float> y(out_dim);
    gemv(format, y.data(), a, w, in_dim, out_dim);
    f32_slice_to_f16(y.data(), out, out_dim);  // write_f16_from_f32 (RNE)
    return 0;
}

int gho_logits(uint32_t format, float* out, const uint16_t* x, const uint8_t* w, size_t in_dim,
               size_t out_dim) {
    if (format != FMT_Q4_K && format != FMT_Q6_K) return -1;
    gemv(format, out, x, w, in_dim, out_dim);
    return 0;
}

// matmul_batched: n == 1 takes the single-token GEMV (q4k.rs:229-232, q6k.rs:167-170);
// otherwise one accumulator per token (batched kernels), output-row-major scratch then
// the token-major FP16 narrow of write_transposed_f16 (matmul/mod.rs:287-303).
int gho_matmul_batched(uint32_t format, uint16_t* out, const uint16_t* a_f16, const uint8_t* w,
                       size_t in_dim, size_t out_dim, size_t n) {
    if (format != FMT_Q4_K && format != FMT_Q6_K) return -1;
    if (n == 0) return 0;
    if (n == 1) return gho_matmul(format, out, a_f16, w, in_dim, out_dim);
    std::vector<float> a(n * in_dim);
    f16_slice_to_f32(a_f16, a.data(), n * in_dim);
    std::vector<float> yt(out_dim * n);
    for_units(out_dim * n, n, [&](size_t o0, size_t start, size_t end) {
        std::vector<float> acc(n * 8);
        size_t rows = (end - start) / n;
        for (size_t k = 0; k < rows; ++k) {
            float* dst = yt.data() + (o0 + k) * n;
            if (format == FMT_Q4_K)
                row_dot_q4k_avx2_batched(a.data(), w, o0 + k, in_dim, dst, n, acc.data());
            else
                row_dot_q6k_avx2_batched(a.data(), w, o0 + k, in_dim, dst, n, acc.data());
        }
    });
    std::vector<float> col(out_dim);
    for (size_t i = 0; i < n; ++i) {
        for (size_t o = 0; o < out_dim; ++o) col[o] = yt[o * n + i];
        f32_slice_to_f16(col.data(), out + i * out_dim, out_dim);
    }
    return 0;
}
}

// Decode GEMV y = W·x for Q4_K and Q6_K weights in the device layout (gh_kargs.h).
//
// One wavefront per group of R output rows; the in-dimension is split over the 64 lanes in
// units of 64 weights (u = 4*block + g for Q4_K, u = 4*block + 2*seg + half for Q6_K), so
// every quant load of a wave is one contiguous 1 KiB dwordx4 access. The activation slice of
// a unit is loaded once per wave and reused for its R rows.
//
// Inner product: quants become FP16 pairs by OR-ing them into the mantissa of 1024.0
// (0x6400 | q is exactly 1024 + q), then v_dot2_f32_f16 multiplies them with FP16 activation
// pairs in FP32. The 1024·Σx bias is removed by starting the accumulator at -1024·Σx, and the
// block scales are applied once per 32 (Q4_K) / 16 (Q6_K) weights:
//   Σ x·(d·sc·q - dmin·mn) = d·sc·Σ x·q - dmin·mn·Σ x.
// FP32 accumulation throughout; the reordering against the reference's AVX2 loop is within
// the FP32 rounding of the sum (checked to 1e-3 relative by the parity tests).
#include "gh_common.h"

namespace {

// Load the 32 FP16 activations x[0..31] of a unit half as 16 dwords and regroup them into
// the pairs the quant dwords produce: for quant dword k (weights 4k..4k+3),
// p02[k] = (x[4k], x[4k+2]) and p13[k] = (x[4k+1], x[4k+3]).
__device__ __forceinline__ void load_pairs32(const uint16_t* x, uint32_t p02[8], uint32_t p13[8],
                                             float& sum) {
    const uint4* xp = (const uint4*)x;
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 v = xp[i];
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t a = w[2 * k], b = w[2 * k + 1];
        p02[k] = (a & 0xFFFFu) | (b << 16);
        p13[k] = (a >> 16) | (b & 0xFFFF0000u);
        s += gh_h2f(a & 0xFFFFu) + gh_h2f(a >> 16) + gh_h2f(b & 0xFFFFu) + gh_h2f(b >> 16);
    }
    sum = s;
}

// Same for 16 activations (one Q6_K quarter of a unit): 4 quant dwords.
__device__ __forceinline__ void load_pairs16(const uint16_t* x, uint32_t p02[4], uint32_t p13[4],
                                             float& sum) {
    const uint4* xp = (const uint4*)x;
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint4 v = xp[i];
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t a = w[2 * k], b = w[2 * k + 1];
        p02[k] = (a & 0xFFFFu) | (b << 16);
        p13[k] = (a >> 16) | (b & 0xFFFF0000u);
        s += gh_h2f(a & 0xFFFFu) + gh_h2f(a >> 16) + gh_h2f(b & 0xFFFFu) + gh_h2f(b >> 16);
    }
    sum = s;
}

__device__ __forceinline__ void store_out(const GhGemvArgs& a, uint32_t t, uint32_t row, float v) {
    const size_t idx = (size_t)t * a.out_dim + row;
    if (a.out_f32)
        ((float*)a.y)[idx] = v;
    else
        ((uint16_t*)a.y)[idx] = gh_f2h(v);
}

template <int R>
__device__ __forceinline__ void gemv_q4k_body(const GhGemvArgs& a) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nb = a.in_dim >> 8;
    const uint32_t units = nb * 4;
    const uint32_t row0 = (blockIdx.x * (blockDim.x >> 6) + wave) * R;
    if (row0 >= a.out_dim) return;
    const uint8_t* qs = (const uint8_t*)a.w;
    const uint8_t* hdr = qs + (size_t)a.out_dim * nb * GH_Q4K_QS_BYTES;
    const size_t row_bytes = (size_t)nb * GH_Q4K_QS_BYTES;
    const size_t half_bytes = (size_t)nb * 64;

    for (uint32_t t = 0; t < a.n; ++t) {
        const uint16_t* x = (const uint16_t*)a.x + (size_t)t * a.in_dim;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;

        for (uint32_t u0 = 0; u0 < units; u0 += 64) {
            const uint32_t u = u0 + lane;
            if (u < units) {
                const uint32_t b = u >> 2, g = u & 3u;
                uint32_t xl02[8], xl13[8], xh02[8], xh13[8];
                float sum_lo, sum_hi;
                load_pairs32(x + (size_t)b * 256 + g * 64, xl02, xl13, sum_lo);
                load_pairs32(x + (size_t)b * 256 + g * 64 + 32, xh02, xh13, sum_hi);
                const float bias_lo = -1024.0f * sum_lo;
                const float bias_hi = -1024.0f * sum_hi;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t row = row0 + r;
                    if (row < a.out_dim) {
                        const uint8_t* rq = qs + (size_t)row * row_bytes + (size_t)u * 16;
                        const uint4 q0 = *(const uint4*)rq;
                        const uint4 q1 = *(const uint4*)(rq + half_bytes);
                        const uint4 hd = *(const uint4*)(hdr + ((size_t)row * nb + b) * 16);
                        const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
                        float slo = bias_lo, shi = bias_hi;
#pragma unroll
                        for (int k = 0; k < 8; ++k) {
                            const uint32_t v = qw[k];
                            const uint32_t v8 = v >> 8;
                            slo = gh_dot2(xl02[k], (v & 0x000F000Fu) | 0x64006400u, slo);
                            slo = gh_dot2(xl13[k], (v8 & 0x000F000Fu) | 0x64006400u, slo);
                            shi = gh_dot2(xh02[k], (v & 0x00F000F0u) | 0x64006400u, shi);
                            shi = gh_dot2(xh13[k], (v8 & 0x00F000F0u) | 0x64006400u, shi);
                        }
                        const float d = gh_h2f(hd.x & 0xFFFFu);
                        const float dmin = gh_h2f(hd.x >> 16);
                        uint32_t sc0, mn0, sc1, mn1;
                        gh_q4k_scale_min(hd, 2 * g, sc0, mn0);
                        gh_q4k_scale_min(hd, 2 * g + 1, sc1, mn1);
                        // slo = Σx·q_lo; shi = 16·Σx·q_hi
                        acc[r] += (d * (float)sc0) * slo - (dmin * (float)mn0) * sum_lo +
                                  (d * (float)sc1 * 0.0625f) * shi - (dmin * (float)mn1) * sum_hi;
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = gh_wave_sum(acc[r]);
            if (lane == 0 && row0 + r < a.out_dim) store_out(a, t, row0 + r, v);
        }
    }
}

template <int R>
__device__ __forceinline__ void gemv_q6k_body(const GhGemvArgs& a) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nb = a.in_dim >> 8;
    const uint32_t units = nb * 4;
    const uint32_t row0 = (blockIdx.x * (blockDim.x >> 6) + wave) * R;
    if (row0 >= a.out_dim) return;
    const uint8_t* qlh = (const uint8_t*)a.w;
    const uint8_t* scp = qlh + (size_t)a.out_dim * nb * GH_Q6K_QLH_BYTES;
    const uint8_t* dp = qlh + (size_t)a.out_dim * nb * 208;
    const size_t row_bytes = (size_t)nb * GH_Q6K_QLH_BYTES;
    const size_t plane_bytes = (size_t)nb * 64;

    for (uint32_t t = 0; t < a.n; ++t) {
        const uint16_t* x = (const uint16_t*)a.x + (size_t)t * a.in_dim;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;

        for (uint32_t u0 = 0; u0 < units; u0 += 64) {
            const uint32_t u = u0 + lane;
            if (u < units) {
                const uint32_t b = u >> 2, s = (u >> 1) & 1u, h = u & 1u;
                // quarter k covers x[256b + 128s + 32k + 16h + 0..15]
                uint32_t xp02[4][4], xp13[4][4];
                float xs[4], bias[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    load_pairs16(x + (size_t)b * 256 + s * 128 + k * 32 + h * 16, xp02[k], xp13[k],
                                 xs[k]);
                    bias[k] = -1056.0f * xs[k];  // value = 1024 + (q + 32)
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t row = row0 + r;
                    if (row < a.out_dim) {
                        const uint8_t* rq = qlh + (size_t)row * row_bytes + (size_t)u * 16;
                        const uint4 qa = *(const uint4*)rq;
                        const uint4 qb = *(const uint4*)(rq + plane_bytes);
                        const uint4 qh = *(const uint4*)(rq + 2 * plane_bytes);
                        const size_t blk = (size_t)row * nb + b;
                        const uint4 sc = *(const uint4*)(scp + blk * 16);
                        const float d = gh_h2f(*(const uint16_t*)(dp + blk * 2));
                        const uint32_t A[4] = {qa.x, qa.y, qa.z, qa.w};
                        const uint32_t B[4] = {qb.x, qb.y, qb.z, qb.w};
                        const uint32_t H[4] = {qh.x, qh.y, qh.z, qh.w};
                        float sk[4] = {bias[0], bias[1], bias[2], bias[3]};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            uint32_t v[4];
                            v[0] = (A[j] & 0x0F0F0F0Fu) | ((H[j] << 4) & 0x30303030u);
                            v[1] = (B[j] & 0x0F0F0F0Fu) | ((H[j] << 2) & 0x30303030u);
                            v[2] = ((A[j] >> 4) & 0x0F0F0F0Fu) | (H[j] & 0x30303030u);
                            v[3] = ((B[j] >> 4) & 0x0F0F0F0Fu) | ((H[j] >> 2) & 0x30303030u);
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                sk[k] = gh_dot2(xp02[k][j], (v[k] & 0x003F003Fu) | 0x64006400u, sk[k]);
                                sk[k] = gh_dot2(xp13[k][j], ((v[k] >> 8) & 0x003F003Fu) | 0x64006400u,
                                                sk[k]);
                            }
                        }
                        // int8 scales sc[8s + h + 2k], k = 0..3
                        const uint32_t wlo = s ? sc.z : sc.x;
                        const uint32_t whi = s ? sc.w : sc.y;
                        const uint32_t sh = 8 * h;
                        const float s0 = (float)(int8_t)(wlo >> sh);
                        const float s1 = (float)(int8_t)(wlo >> (sh + 16));
                        const float s2 = (float)(int8_t)(whi >> sh);
                        const float s3 = (float)(int8_t)(whi >> (sh + 16));
                        acc[r] += d * (s0 * sk[0] + s1 * sk[1] + s2 * sk[2] + s3 * sk[3]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = gh_wave_sum(acc[r]);
            if (lane == 0 && row0 + r < a.out_dim) store_out(a, t, row0 + r, v);
        }
    }
}

}  // namespace

GH_KERNEL __launch_bounds__(256) void gh_gemv_q4k_r1(GhGemvArgs a) { gemv_q4k_body<1>(a); }
GH_KERNEL __launch_bounds__(256) void gh_gemv_q4k_r2(GhGemvArgs a) { gemv_q4k_body<2>(a); }
GH_KERNEL __launch_bounds__(256) void gh_gemv_q4k_r4(GhGemvArgs a) { gemv_q4k_body<4>(a); }
GH_KERNEL __launch_bounds__(256) void gh_gemv_q6k_r1(GhGemvArgs a) { gemv_q6k_body<1>(a); }
GH_KERNEL __launch_bounds__(256) void gh_gemv_q6k_r2(GhGemvArgs a) { gemv_q6k_body<2>(a); }
GH_KERNEL __launch_bounds__(256) void gh_gemv_q6k_r4(GhGemvArgs a) { gemv_q6k_body<4>(a); }

// Decode GEMV y = W·x for Q4_K and Q6_K weights in the device layout (gh_kargs.h), with fused
// epilogues (FP16/FP32 store, residual add, YaRN RoPE into q or the K cache, V-cache store,
// SwiGLU over gate/up).
//
// Mapping: a launch is a list of wavefront tasks; a task is R consecutive rows of one matrix.
// The in-dimension is split over the 64 lanes in units of 64 weights (u = 4*block + g for
// Q4_K, u = 4*block + 2*seg + half for Q6_K), so every weight load of a wave is one contiguous
// 1 KiB global_load_dwordx4. All R rows' loads of a chunk are issued before any arithmetic, so
// a wave keeps 3R (Q4_K) or 4R (Q6_K) 16-byte loads per lane in flight.
//
// Inner product: quants become FP16 pairs by OR-ing them into the mantissa of 1024.0
// (0x6400 | q is exactly 1024 + q) and v_dot2_f32_f16 multiplies them with FP16 activation
// pairs in FP32. The 1024·Σx bias is removed by starting each accumulator at -1024·Σx, and the
// block scales are applied once per 32 (Q4_K) / 16 (Q6_K) weights:
//   Σ x·(d·sc·q - dmin·mn) = d·sc·Σ x·q - dmin·mn·Σ x.
// FP32 accumulation; the result differs from the reference's AVX2 loop only by the rounding of
// a re-associated FP32 sum (checked to 1e-3 relative by the parity tests). The wave reduction
// is a DPP tree (gh_wave_sum63); row results land in lane 63, which runs the epilogue.
#include "gh_common.h"

namespace {

constexpr uint32_t kQ4K = 12, kQ6K = 14;

// Activations of one Q4_K unit: x[0..63] (sub-block 2g then 2g+1) as FP16 pairs matching the
// quant dwords: for quant dword k (weights 4k..4k+3 of a 32-weight sub-block)
// p02[k] = (x[4k], x[4k+2]), p13[k] = (x[4k+1], x[4k+3]).
struct XQ4 {
    uint32_t lo02[8], lo13[8], hi02[8], hi13[8];
    float bias_lo, bias_hi, sum_lo, sum_hi;
};

__device__ __forceinline__ void pairs32(const uint4 (&v)[4], uint32_t p02[8], uint32_t p13[8],
                                        float& sum) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint4& q = v[k >> 1];
        const uint32_t a = (k & 1) ? q.z : q.x, b = (k & 1) ? q.w : q.y;
        p02[k] = (a & 0xFFFFu) | (b << 16);
        p13[k] = (a >> 16) | (b & 0xFFFF0000u);
        s += (gh_h2f(a & 0xFFFFu) + gh_h2f(a >> 16)) + (gh_h2f(b & 0xFFFFu) + gh_h2f(b >> 16));
    }
    sum = s;
}

__device__ __forceinline__ void load_x_q4(const uint16_t* x, uint32_t b, uint32_t g, XQ4& o) {
    const GH_GLOBAL uint4* p = gh_gp<uint4>((uint64_t)(x + (size_t)b * 256 + g * 64));
    uint4 lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) lo[i] = p[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) hi[i] = p[4 + i];
    pairs32(lo, o.lo02, o.lo13, o.sum_lo);
    pairs32(hi, o.hi02, o.hi13, o.sum_hi);
    o.bias_lo = -1024.0f * o.sum_lo;
    o.bias_hi = -1024.0f * o.sum_hi;
}

struct WQ4 {
    uint4 q0, q1, hd;
};

__device__ __forceinline__ void load_w_q4(const uint8_t* w, uint32_t rows, uint32_t nb,
                                          uint32_t row, uint32_t u, WQ4& o) {
    const uint8_t* rq = w + (size_t)row * GH_Q4K_QS_BYTES * nb + (size_t)u * 16;
    o.q0 = *gh_gp<uint4>((uint64_t)rq);
    o.q1 = *gh_gp<uint4>((uint64_t)(rq + (size_t)nb * 64));
    o.hd = *gh_gp<uint4>((uint64_t)(w + (size_t)rows * GH_Q4K_QS_BYTES * nb +
                                    ((size_t)row * nb + (u >> 2)) * 16));
}

__device__ __forceinline__ float dot_q4(const XQ4& x, const WQ4& w, uint32_t g) {
    const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    float slo = x.bias_lo, shi = x.bias_hi;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t v = qw[k], v8 = v >> 8;
        slo = gh_dot2(x.lo02[k], (v & 0x000F000Fu) | 0x64006400u, slo);
        slo = gh_dot2(x.lo13[k], (v8 & 0x000F000Fu) | 0x64006400u, slo);
        shi = gh_dot2(x.hi02[k], (v & 0x00F000F0u) | 0x64006400u, shi);
        shi = gh_dot2(x.hi13[k], (v8 & 0x00F000F0u) | 0x64006400u, shi);
    }
    const float d = gh_h2f(w.hd.x & 0xFFFFu), dmin = gh_h2f(w.hd.x >> 16);
    uint32_t sc0, mn0, sc1, mn1;
    gh_q4k_scale_min(w.hd, 2 * g, sc0, mn0);
    gh_q4k_scale_min(w.hd, 2 * g + 1, sc1, mn1);
    // slo = Σx·q_lo, shi = 16·Σx·q_hi
    return (d * (float)sc0) * slo - (dmin * (float)mn0) * x.sum_lo +
           (d * (float)sc1 * 0.0625f) * shi - (dmin * (float)mn1) * x.sum_hi;
}

// Activations of one Q6_K unit: quarter k covers x[256b + 128s + 32k + 16h + 0..15].
struct XQ6 {
    uint32_t p02[4][4], p13[4][4];
    float bias[4];
};

__device__ __forceinline__ void load_x_q6(const uint16_t* x, uint32_t b, uint32_t s, uint32_t h,
                                          XQ6& o) {
    uint4 v[4][2];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const GH_GLOBAL uint4* p =
            gh_gp<uint4>((uint64_t)(x + (size_t)b * 256 + s * 128 + k * 32 + h * 16));
        v[k][0] = p[0];
        v[k][1] = p[1];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4& q = v[k][j >> 1];
            const uint32_t a = (j & 1) ? q.z : q.x, c = (j & 1) ? q.w : q.y;
            o.p02[k][j] = (a & 0xFFFFu) | (c << 16);
            o.p13[k][j] = (a >> 16) | (c & 0xFFFF0000u);
            sum += (gh_h2f(a & 0xFFFFu) + gh_h2f(a >> 16)) + (gh_h2f(c & 0xFFFFu) + gh_h2f(c >> 16));
        }
        o.bias[k] = -1056.0f * sum;  // pair value = 1024 + (q + 32)
    }
}

struct WQ6 {
    uint4 qa, qb, qh, sc;
    uint32_t d;
};

__device__ __forceinline__ void load_w_q6(const uint8_t* w, uint32_t rows, uint32_t nb,
                                          uint32_t row, uint32_t u, WQ6& o) {
    const uint8_t* rq = w + (size_t)row * GH_Q6K_QLH_BYTES * nb + (size_t)u * 16;
    const size_t plane = (size_t)nb * 64;
    o.qa = *gh_gp<uint4>((uint64_t)rq);
    o.qb = *gh_gp<uint4>((uint64_t)(rq + plane));
    o.qh = *gh_gp<uint4>((uint64_t)(rq + 2 * plane));
    const size_t blk = (size_t)row * nb + (u >> 2);
    o.sc = *gh_gp<uint4>((uint64_t)(w + (size_t)rows * GH_Q6K_QLH_BYTES * nb + blk * 16));
    o.d = *gh_gp<uint16_t>((uint64_t)(w + (size_t)rows * 208 * nb + blk * 2));
}

__device__ __forceinline__ float dot_q6(const XQ6& x, const WQ6& w, uint32_t s, uint32_t h) {
    const uint32_t A[4] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w};
    const uint32_t B[4] = {w.qb.x, w.qb.y, w.qb.z, w.qb.w};
    const uint32_t H[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
    float sk[4] = {x.bias[0], x.bias[1], x.bias[2], x.bias[3]};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t v[4];
        v[0] = (A[j] & 0x0F0F0F0Fu) | ((H[j] << 4) & 0x30303030u);
        v[1] = (B[j] & 0x0F0F0F0Fu) | ((H[j] << 2) & 0x30303030u);
        v[2] = ((A[j] >> 4) & 0x0F0F0F0Fu) | (H[j] & 0x30303030u);
        v[3] = ((B[j] >> 4) & 0x0F0F0F0Fu) | ((H[j] >> 2) & 0x30303030u);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            sk[k] = gh_dot2(x.p02[k][j], (v[k] & 0x003F003Fu) | 0x64006400u, sk[k]);
            sk[k] = gh_dot2(x.p13[k][j], ((v[k] >> 8) & 0x003F003Fu) | 0x64006400u, sk[k]);
        }
    }
    // int8 scales sc[8s + h + 2k], k = 0..3
    const uint32_t wlo = s ? w.sc.z : w.sc.x, whi = s ? w.sc.w : w.sc.y;
    const uint32_t sh = 8 * h;
    const float s0 = (float)(int8_t)(wlo >> sh), s1 = (float)(int8_t)(wlo >> (sh + 16));
    const float s2 = (float)(int8_t)(whi >> sh), s3 = (float)(int8_t)(whi >> (sh + 16));
    return gh_h2f(w.d) * (s0 * sk[0] + s1 * sk[1] + s2 * sk[2] + s3 * sk[3]);
}

// R rows (and, for SwiGLU, the same R rows of a second matrix) of one format over the whole
// in-dimension; per-lane partial sums in acc[m][r].
template <uint32_t FMT, int R, int M>
__device__ __forceinline__ void rows_dot(const uint8_t* const (&w)[M], uint32_t rows, uint32_t nb,
                                         const uint16_t* x, uint32_t row0, float (&acc)[M][R]) {
    const uint32_t lane = threadIdx.x & 63u, units = nb * 4;
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
    for (uint32_t u0 = 0; u0 < units; u0 += 64) {
        const uint32_t u = u0 + lane;
        if (u >= units) continue;
        const uint32_t b = u >> 2;
        if constexpr (FMT == kQ4K) {
            const uint32_t g = u & 3u;
            WQ4 wr[M][R];
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r)
                    load_w_q4(w[m], rows, nb, min(row0 + r, rows - 1), u, wr[m][r]);
            XQ4 xv;
            load_x_q4(x, b, g, xv);
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r) acc[m][r] += dot_q4(xv, wr[m][r], g);
        } else {
            const uint32_t s = (u >> 1) & 1u, h = u & 1u;
            WQ6 wr[M][R];
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r)
                    load_w_q6(w[m], rows, nb, min(row0 + r, rows - 1), u, wr[m][r]);
            XQ6 xv;
            load_x_q6(x, b, s, h, xv);
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r) acc[m][r] += dot_q6(xv, wr[m][r], s, h);
        }
    }
}

__device__ __forceinline__ uint32_t position(const GhGemvArgs& a) {
    return (a.pos_ptr ? *gh_gp<uint32_t>(a.pos_ptr) : 0u) + a.base;
}

// f16(acc) rotated pairwise: (y0, y1) -> ((y0 c - y1 s) k, (y0 s + y1 c) k), the reference's
// rope_yarn on the FP16 matmul output (cpu/kernels/elementwise/rope.rs:14-39).
__device__ __forceinline__ void rope_pair(const GhGemvArgs& a, uint32_t row, float acc0,
                                          float acc1, bool post, uint32_t pos, uint16_t& o0,
                                          uint16_t& o1) {
#pragma clang fp contract(off)
    const uint16_t h0 = gh_f2h(acc0), h1 = gh_f2h(acc1);
    const uint32_t pair = (row % a.head_dim) >> 1;
    if (pair >= a.pairs) {
        o0 = h0;
        o1 = h1;
        return;
    }
    const float2 cs = gh_gp<float2>(a.table)[(size_t)pos * a.pairs + pair];
    const float k = post ? gh_gp<float>(a.post)[pos] : 1.0f;
    const float x0 = gh_h2f(h0), x1 = gh_h2f(h1);
    o0 = gh_f2h((x0 * cs.x - x1 * cs.y) * k);
    o1 = gh_f2h((x0 * cs.y + x1 * cs.x) * k);
}

template <int R>
__device__ __forceinline__ void epilogue(const GhGemvArgs& a, const GhGemvSeg& sg, uint32_t t,
                                         uint32_t row0, const float (&v)[R], const float* up) {
#pragma clang fp contract(off)
    switch (sg.epi) {
        case GH_EPI_F16:
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < sg.rows) gh_gpw<uint16_t>(sg.out)[(size_t)t * sg.rows + row0 + r] = gh_f2h(v[r]);
            break;
        case GH_EPI_F32:
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < sg.rows) gh_gpw<float>(sg.out)[(size_t)t * sg.rows + row0 + r] = v[r];
            break;
        case GH_EPI_RESID:
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < sg.rows) {
                    GH_GLOBAL float* xr = gh_gpw<float>(sg.out) + row0 + r;
                    *xr = *xr + gh_h2f(gh_f2h(v[r]));
                }
            break;
        case GH_EPI_CACHE: {
            const size_t off = (size_t)position(a) * sg.rows;
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < sg.rows) gh_gpw<uint16_t>(sg.out)[off + row0 + r] = gh_f2h(v[r]);
            break;
        }
        case GH_EPI_ROPE:
        case GH_EPI_ROPE_CACHE: {
            const uint32_t pos = position(a);
            const bool q = sg.epi == GH_EPI_ROPE;
            const size_t off = q ? 0 : (size_t)pos * sg.rows;
#pragma unroll
            for (int r = 0; r + 1 < R; r += 2) {
                if (row0 + r + 1 < sg.rows) {
                    uint16_t o0, o1;
                    rope_pair(a, row0 + r, v[r], v[r + 1], q, pos, o0, o1);
                    GH_GLOBAL uint16_t* dst = gh_gpw<uint16_t>(sg.out) + off + row0 + r;
                    dst[0] = o0;
                    dst[1] = o1;
                }
            }
            break;
        }
        case GH_EPI_SWIGLU:
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < sg.rows) {
                    // silu_mul (activation.rs:16-29) on the FP16-rounded gate/up projections
                    const float g = gh_h2f(gh_f2h(v[r])), u = gh_h2f(gh_f2h(up[r]));
                    const float silu = g / (1.0f + expf(-g));
                    gh_gpw<uint16_t>(sg.out)[row0 + r] = gh_f2h(gh_h2f(gh_f2h(silu)) * u);
                }
            break;
    }
}

// MODE: which row kernels a launch may need (specialized to keep register use low).
enum : int { kModeQ4 = 0, kModeQ6 = 1, kModeMixed = 2, kModeSwiglu = 3 };

template <int R, int MODE>
__device__ __forceinline__ void gemv_body(const GhGemvArgs& a) {
    const uint32_t task = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (task >= a.tasks) return;
    uint32_t si = 0;
    if (a.nseg > 1 && task >= a.seg[1].task0) si = 1;
    if (a.nseg > 2 && task >= a.seg[2].task0) si = 2;
    const GhGemvSeg sg = a.seg[si];
    const uint32_t row0 = (task - sg.task0) * R;
    const uint32_t nb = a.in_dim >> 8;
    const bool lane63 = (threadIdx.x & 63u) == 63u;
    for (uint32_t t = 0; t < a.n; ++t) {
        const uint16_t* x = (const uint16_t*)a.x + (size_t)t * a.in_dim;
        if constexpr (MODE == kModeSwiglu) {
            const uint8_t* const w[2] = {(const uint8_t*)sg.w, (const uint8_t*)a.aux};
            float acc[2][R];
            rows_dot<kQ4K, R, 2>(w, sg.rows, nb, x, row0, acc);
            float g[R], u[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                g[r] = gh_wave_sum63(acc[0][r]);
                u[r] = gh_wave_sum63(acc[1][r]);
            }
            if (lane63) epilogue<R>(a, sg, t, row0, g, u);
        } else {
            const uint8_t* const w[1] = {(const uint8_t*)sg.w};
            float acc[1][R];
            if (MODE == kModeQ4 || (MODE == kModeMixed && sg.fmt == kQ4K))
                rows_dot<kQ4K, R, 1>(w, sg.rows, nb, x, row0, acc);
            else
                rows_dot<kQ6K, R, 1>(w, sg.rows, nb, x, row0, acc);
            float v[R];
#pragma unroll
            for (int r = 0; r < R; ++r) v[r] = gh_wave_sum63(acc[0][r]);
            if (lane63) epilogue<R>(a, sg, t, row0, v, nullptr);
        }
    }
}

}  // namespace

#define GH_GEMV(NAME, R, MODE) \
    GH_KERNEL __launch_bounds__(256) void NAME(GhGemvArgs a) { gemv_body<R, MODE>(a); }
GH_GEMV(gh_gemv_q4k_r1, 1, kModeQ4)
GH_GEMV(gh_gemv_q4k_r2, 2, kModeQ4)
GH_GEMV(gh_gemv_q4k_r4, 4, kModeQ4)
GH_GEMV(gh_gemv_q6k_r1, 1, kModeQ6)
GH_GEMV(gh_gemv_q6k_r2, 2, kModeQ6)
GH_GEMV(gh_gemv_q6k_r4, 4, kModeQ6)
GH_GEMV(gh_gemv_mixed_r2, 2, kModeMixed)
GH_GEMV(gh_gemv_swiglu_r1, 1, kModeSwiglu)
GH_GEMV(gh_gemv_swiglu_r2, 2, kModeSwiglu)

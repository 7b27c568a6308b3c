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
#include <type_traits>

#include "gh_common.h"

namespace {

constexpr uint32_t kQ4K = 12, kQ6K = 14;

// Bit-manipulation constants held in registers: gfx9 VOP3 cannot encode a literal, so with the
// masks in VGPRs and the 1024.0 pair in an SGPR each FP16 pair is one v_and_or_b32.
struct Masks {
    uint32_t lo4, hi4, lo6, bias;
};

__device__ __forceinline__ Masks make_masks() {
    Masks m{0x000F000Fu, 0x00F000F0u, 0x003F003Fu, 0x64006400u};
    asm volatile("" : "+v"(m.lo4), "+v"(m.hi4), "+v"(m.lo6));
    asm volatile("" : "+s"(m.bias));
    return m;
}

// x staged in LDS once per workgroup, as FP16 pairs in the order the quant dwords produce them.
// Unit u's 8 uint4 of pairs sit at xs[k * units + u] (k = 0..7: conflict-free b128 reads);
// its activation sums at sums[u].
//   Q4_K unit (x[256b + 64g .. +64)): k = 0,1: lo02, 2,3: lo13, 4,5: hi02, 6,7: hi13 where
//     for quant dword j of a 32-weight sub-block, p02[j] = (x[4j], x[4j+2]),
//     p13[j] = (x[4j+1], x[4j+3]); sums = (Σ lo half, Σ hi half).
//   Q6_K unit (quarter q: x[256b + 128s + 32q + 16h .. +16)): k = q: p02 of quarter q,
//     k = 4 + q: p13 of quarter q; sums = Σ of each quarter.
__device__ __forceinline__ void pair16(const uint4& a, const uint4& b, uint4& p02, uint4& p13,
                                       float& sum) {
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t e[4], o[4];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = w[2 * j], hi = w[2 * j + 1];
        e[j] = (lo & 0xFFFFu) | (hi << 16);
        o[j] = (lo >> 16) | (hi & 0xFFFF0000u);
        // Σ of the 16 values with v_dot2_f32_f16 against (1, 1): exact products, FP32 sum
        s = gh_dot2(lo, 0x3C003C00u, s);
        s = gh_dot2(hi, 0x3C003C00u, s);
    }
    p02 = make_uint4(e[0], e[1], e[2], e[3]);
    p13 = make_uint4(o[0], o[1], o[2], o[3]);
    sum = s;
}

// x8(e) returns FP16 x[e .. e+8) as a uint4 (e a multiple of 8). The pairs and sums of unit u.
// The 8 uint4 of FP16 x that unit u pairs, in pairing order (Q4_K: x[256b + 64g .. +64);
// Q6_K: quarter q's 16 values at 256b + 128s + 32q + 16h, as two uint4 each).
template <uint32_t FMT, class X8>
__device__ __forceinline__ void load_unit_x(const X8& x8, uint32_t u, uint4 (&v)[8]) {
    if constexpr (FMT == kQ4K) {
        const uint32_t e0 = (u >> 2) * 256 + (u & 3u) * 64;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = x8(e0 + 8 * i);
    } else {
        const uint32_t b = u >> 2, sg = (u >> 1) & 1u, h = u & 1u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t e = b * 256 + sg * 128 + q * 32 + h * 16;
            v[2 * q] = x8(e);
            v[2 * q + 1] = x8(e + 8);
        }
    }
}

template <uint32_t FMT>
__device__ __forceinline__ void pair_raw(const uint4 (&v)[8], uint4 (&xv)[8], float4& sum) {
    float s[4];
    if constexpr (FMT == kQ4K) {
        pair16(v[0], v[1], xv[0], xv[2], s[0]);
        pair16(v[2], v[3], xv[1], xv[3], s[1]);
        pair16(v[4], v[5], xv[4], xv[6], s[2]);
        pair16(v[6], v[7], xv[5], xv[7], s[3]);
        sum = make_float4(s[0] + s[1], s[2] + s[3], 0.0f, 0.0f);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) pair16(v[2 * q], v[2 * q + 1], xv[q], xv[4 + q], s[q]);
        sum = make_float4(s[0], s[1], s[2], s[3]);
    }
}

template <uint32_t FMT, class X8>
__device__ __forceinline__ void pair_unit(const X8& x8, uint32_t u, uint4 (&xv)[8], float4& sum) {
    uint4 v[8];
    load_unit_x<FMT>(x8, u, v);
    pair_raw<FMT>(v, xv, sum);
}
template <uint32_t FMT, class X8>
__device__ __forceinline__ void stage_x(const X8& x8, uint32_t units, uint4* xs, float4* sums) {
    for (uint32_t item = threadIdx.x; item < units * 4; item += 256) {
        const uint32_t u = item >> 2, q = item & 3u;
        uint4 p02, p13;
        float sq;
        if constexpr (FMT == kQ4K) {
            // quarter q: chunks 2q, 2q+1 -> k = {0,2} (q=0), {1,3} (q=1), {4,6} (q=2), {5,7} (q=3)
            const uint32_t e = (u >> 2) * 256 + (u & 3u) * 64 + 16 * q;
            pair16(x8(e), x8(e + 8), p02, p13, sq);
            const uint32_t k0 = (q & 1u) + 4 * (q >> 1);
            xs[k0 * units + u] = p02;
            xs[(k0 + 2) * units + u] = p13;
        } else {
            const uint32_t e = (u >> 2) * 256 + ((u >> 1) & 1u) * 128 + q * 32 + (u & 1u) * 16;
            pair16(x8(e), x8(e + 8), p02, p13, sq);
            xs[q * units + u] = p02;
            xs[(4 + q) * units + u] = p13;
        }
        ((float*)&sums[u])[q] = sq;
    }
}

// Weights are streamed once per token: nontemporal loads (the `nt` bit: streaming, not kept
// in the caches) measured 606 -> 629 tok/s on the 8B decode, 7.31 -> 7.2 us at 12288x4096.
// (The same hint on the prefill GEMM's weights, which two token tiles share, and on the decode
// attention's K/V measured slower: 83 -> 105 us on the 512-token gate, 12.9 -> 14.3 us at ctx 4096.)
__device__ __forceinline__ uint4 gh_ld_nt(uint64_t a) {
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    const u4v v = __builtin_nontemporal_load((const GH_GLOBAL u4v*)a);
    return make_uint4(v.x, v.y, v.z, v.w);
}

struct WQ4 {
    uint4 q0, q1, hd;
};

__device__ __forceinline__ void load_w_q4(const uint8_t* w, uint32_t rows, uint32_t nb,
                                          uint32_t row, uint32_t u, WQ4& o) {
    const uint8_t* rq = w + (size_t)row * GH_Q4K_QS_BYTES * nb + (size_t)u * 16;
    o.q0 = gh_ld_nt((uint64_t)rq);
    o.q1 = gh_ld_nt((uint64_t)(rq + (size_t)nb * 64));
    o.hd = gh_ld_nt((uint64_t)(w + (size_t)rows * GH_Q4K_QS_BYTES * nb + ((size_t)row * nb + (u >> 2)) * 16));
}

// One Q4_K unit: the 32 qs bytes of group g (sub-blocks 2g, 2g+1) against staged x.
__device__ __forceinline__ float dot_q4(const uint4 (&xv)[8], const float4& xsum, const WQ4& w,
                                        uint32_t g, const Masks& m) {
    const uint32_t qw[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    const uint32_t lo02[8] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w, xv[1].x, xv[1].y, xv[1].z, xv[1].w};
    const uint32_t lo13[8] = {xv[2].x, xv[2].y, xv[2].z, xv[2].w, xv[3].x, xv[3].y, xv[3].z, xv[3].w};
    const uint32_t hi02[8] = {xv[4].x, xv[4].y, xv[4].z, xv[4].w, xv[5].x, xv[5].y, xv[5].z, xv[5].w};
    const uint32_t hi13[8] = {xv[6].x, xv[6].y, xv[6].z, xv[6].w, xv[7].x, xv[7].y, xv[7].z, xv[7].w};
    float slo = -1024.0f * xsum.x, shi = -1024.0f * xsum.y;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t v = qw[k], v8 = v >> 8;
        slo = gh_dot2(lo02[k], (v & m.lo4) | m.bias, slo);
        slo = gh_dot2(lo13[k], (v8 & m.lo4) | m.bias, slo);
        shi = gh_dot2(hi02[k], (v & m.hi4) | m.bias, shi);
        shi = gh_dot2(hi13[k], (v8 & m.hi4) | m.bias, shi);
    }
    const float d = gh_h2f(w.hd.x & 0xFFFFu), dmin = gh_h2f(w.hd.x >> 16);
    uint32_t sc0, mn0, sc1, mn1;
    gh_q4k_scale_min(w.hd, 2 * g, sc0, mn0);
    gh_q4k_scale_min(w.hd, 2 * g + 1, sc1, mn1);
    // slo = Σx·q_lo, shi = 16·Σx·q_hi
    return (d * (float)sc0) * slo - (dmin * (float)mn0) * xsum.x +
           (d * (float)sc1 * 0.0625f) * shi - (dmin * (float)mn1) * xsum.y;
}

struct WQ6 {
    uint4 qa, qb, qh, sc;
    uint32_t d;
};

__device__ __forceinline__ void load_w_q6(const uint8_t* w, uint32_t rows, uint32_t nb,
                                          uint32_t row, uint32_t u, WQ6& o) {
    const uint8_t* rq = w + (size_t)row * GH_Q6K_QLH_BYTES * nb + (size_t)u * 16;
    const size_t plane = (size_t)nb * 64;
    o.qa = gh_ld_nt((uint64_t)rq);
    o.qb = gh_ld_nt((uint64_t)(rq + plane));
    o.qh = gh_ld_nt((uint64_t)(rq + 2 * plane));
    const size_t blk = (size_t)row * nb + (u >> 2);
    o.sc = gh_ld_nt((uint64_t)(w + (size_t)rows * GH_Q6K_QLH_BYTES * nb + blk * 16));
    o.d = __builtin_nontemporal_load(gh_gp<uint16_t>((uint64_t)(w + (size_t)rows * 208 * nb + blk * 2)));
}

// One Q6_K unit (segment s, half h of block b): 16 weights of each quarter.
__device__ __forceinline__ float dot_q6(const uint4 (&xv)[8], const float4& xsum, const WQ6& w,
                                        uint32_t s, uint32_t h, const Masks& m) {
    const uint32_t A[4] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w};
    const uint32_t B[4] = {w.qb.x, w.qb.y, w.qb.z, w.qb.w};
    const uint32_t H[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
    // pair value = 1024 + (q + 32): start each quarter at -1056·Σx
    float sk[4] = {-1056.0f * xsum.x, -1056.0f * xsum.y, -1056.0f * xsum.z, -1056.0f * xsum.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t v[4];
        v[0] = (A[j] & 0x0F0F0F0Fu) | ((H[j] << 4) & 0x30303030u);
        v[1] = (B[j] & 0x0F0F0F0Fu) | ((H[j] << 2) & 0x30303030u);
        v[2] = ((A[j] >> 4) & 0x0F0F0F0Fu) | (H[j] & 0x30303030u);
        v[3] = ((B[j] >> 4) & 0x0F0F0F0Fu) | ((H[j] >> 2) & 0x30303030u);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t p02 = j == 0 ? xv[k].x : j == 1 ? xv[k].y : j == 2 ? xv[k].z : xv[k].w;
            const uint32_t p13 = j == 0 ? xv[4 + k].x : j == 1 ? xv[4 + k].y : j == 2 ? xv[4 + k].z : xv[4 + k].w;
            sk[k] = gh_dot2(p02, (v[k] & m.lo6) | m.bias, sk[k]);
            sk[k] = gh_dot2(p13, ((v[k] >> 8) & m.lo6) | m.bias, sk[k]);
        }
    }
    // int8 scales sc[8s + h + 2k], k = 0..3
    const uint32_t wlo = s ? w.sc.z : w.sc.x, whi = s ? w.sc.w : w.sc.y;
    const uint32_t sh = 8 * h;
    const float s0 = (float)(int8_t)(wlo >> sh), s1 = (float)(int8_t)(wlo >> (sh + 16));
    const float s2 = (float)(int8_t)(whi >> sh), s3 = (float)(int8_t)(whi >> (sh + 16));
    return gh_h2f(w.d) * (s0 * sk[0] + s1 * sk[1] + s2 * sk[2] + s3 * sk[3]);
}

template <uint32_t FMT>
using WRow = typename std::conditional<FMT == kQ4K, WQ4, WQ6>::type;

// Weights of one pipeline step: chunk `u0` of rows row0..row0+R-1 of M matrices (lane's unit).
template <uint32_t FMT, int R, int M>
__device__ __forceinline__ void load_step(const uint8_t* const (&w)[M], uint32_t rows,
                                          uint32_t nb, uint32_t row0, uint32_t u,
                                          WRow<FMT> (&wr)[M][R]) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (FMT == kQ4K)
                load_w_q4(w[m], rows, nb, min(row0 + r, rows - 1), u, wr[m][r]);
            else
                load_w_q6(w[m], rows, nb, min(row0 + r, rows - 1), u, wr[m][r]);
        }
}

template <uint32_t FMT, int R, int M>
__device__ __forceinline__ void compute_regs(const uint4 (&xv)[8], const float4& xsum, uint32_t u,
                                             const Masks& mk, const WRow<FMT> (&wr)[M][R],
                                             float (&acc)[M][R]) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (FMT == kQ4K)
                acc[m][r] += dot_q4(xv, xsum, wr[m][r], u & 3u, mk);
            else
                acc[m][r] += dot_q6(xv, xsum, wr[m][r], (u >> 1) & 1u, u & 1u, mk);
            // one row at a time: keeps the temporaries of a single dot product live
            if constexpr (M * R > 2) __builtin_amdgcn_sched_barrier(0);
        }
}

// The Q4_K dot products of R rows against x paired in LDS (stage_x's layout), in two halves
// of a unit's 32 quant bytes so only half the pairs (16 VGPRs) are live at once; the same
// accumulation order as dot_q4.
template <int R>
__device__ __forceinline__ void compute_q4_halves(const uint4* xs, const float4* sums, uint32_t units,
                                                  uint32_t u, const Masks& m, const WQ4 (&wr)[R],
                                                  float (&acc)[R]) {
    const float4 xq = sums[u];
    const float s0 = xq.x + xq.y, s1 = xq.z + xq.w;
    float slo[R], shi[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        slo[r] = -1024.0f * s0;
        shi[r] = -1024.0f * s1;
    }
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        __builtin_amdgcn_sched_barrier(0);  // one half's pairs live at a time
        const uint4 l02 = xs[hf * units + u], l13 = xs[(2 + hf) * units + u];
        const uint4 h02 = xs[(4 + hf) * units + u], h13 = xs[(6 + hf) * units + u];
        const uint32_t L02[4] = {l02.x, l02.y, l02.z, l02.w}, L13[4] = {l13.x, l13.y, l13.z, l13.w};
        const uint32_t H02[4] = {h02.x, h02.y, h02.z, h02.w}, H13[4] = {h13.x, h13.y, h13.z, h13.w};
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint4 q = hf ? wr[r].q1 : wr[r].q0;
            const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t v = qw[k], v8 = v >> 8;
                slo[r] = gh_dot2(L02[k], (v & m.lo4) | m.bias, slo[r]);
                slo[r] = gh_dot2(L13[k], (v8 & m.lo4) | m.bias, slo[r]);
                shi[r] = gh_dot2(H02[k], (v & m.hi4) | m.bias, shi[r]);
                shi[r] = gh_dot2(H13[k], (v8 & m.hi4) | m.bias, shi[r]);
            }
        }
    }
    const uint32_t g = u & 3u;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float d = gh_h2f(wr[r].hd.x & 0xFFFFu), dmin = gh_h2f(wr[r].hd.x >> 16);
        uint32_t sc0, mn0, sc1, mn1;
        gh_q4k_scale_min(wr[r].hd, 2 * g, sc0, mn0);
        gh_q4k_scale_min(wr[r].hd, 2 * g + 1, sc1, mn1);
        acc[r] += (d * (float)sc0) * slo[r] - (dmin * (float)mn0) * s0 +
                  (d * (float)sc1 * 0.0625f) * shi[r] - (dmin * (float)mn1) * s1;
    }
}

template <uint32_t FMT, int R, int M>
__device__ __forceinline__ void compute_step(const uint4* xs, const float4* sums, uint32_t units,
                                             uint32_t u, const Masks& mk,
                                             const WRow<FMT> (&wr)[M][R], float (&acc)[M][R]) {
    uint4 xv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) xv[k] = xs[k * units + u];
    float4 xsum = sums[u];
    if constexpr (FMT == kQ4K) xsum = make_float4(xsum.x + xsum.y, xsum.z + xsum.w, 0.0f, 0.0f);
    compute_regs<FMT, R, M>(xv, xsum, u, mk, wr, acc);
}

__device__ __forceinline__ uint32_t position(const GhGemvArgs& a) {
    return (a.pos_ptr ? *gh_gp<uint32_t>(a.pos_ptr) : 0u) + a.base;
}

__device__ __forceinline__ bool epi_needs_pos(uint32_t epi) {
    return epi == GH_EPI_ROPE || epi == GH_EPI_ROPE_CACHE || epi == GH_EPI_CACHE;
}

// Epilogue inputs that do not depend on the task's dot products — the residual rows, the RoPE
// (cos, sin) of the position and the query post-scale — requested together with the task's
// weights, so their latency overlaps the weight stream instead of following the reduction.
template <int R>
struct EpiIn {
    float res[R];
    float2 cs[R / 2 > 0 ? R / 2 : 1];
    float k;
};

// Branch-free (loads inside branches cost exact wait counts): every value is requested; an
// epilogue that does not use one reads it from x instead, which is always valid memory.
template <int R, bool SW>
__device__ __forceinline__ void epi_load(const GhGemvArgs& a, const GhGemvSeg& sg, uint32_t t,
                                         uint32_t row0, uint32_t pos, EpiIn<R>& e) {
    if constexpr (SW) return;
    const bool resid = sg.epi == GH_EPI_RESID;
    const bool rope = (sg.epi == GH_EPI_ROPE || sg.epi == GH_EPI_ROPE_CACHE) && a.table;
    const bool post = sg.epi == GH_EPI_ROPE && a.post;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint64_t at = sg.out + ((uint64_t)t * sg.rows + min(row0 + r, sg.rows - 1)) * 4;
        e.res[r] = *gh_gp<float>(resid ? at : a.x);
    }
#pragma unroll
    for (int r = 0; r + 1 < R; r += 2) {
        const uint32_t pair = min(((row0 + r) % a.head_dim) >> 1, a.pairs - 1);
        const uint64_t at = a.table + ((uint64_t)pos * a.pairs + pair) * 8;
        e.cs[r / 2] = *gh_gp<float2>(rope ? at : a.x);
    }
    const float k = *gh_gp<float>(post ? a.post + (uint64_t)pos * 4 : a.x);
    e.k = post ? k : 1.0f;
}

// f16(acc) rotated pairwise: (y0, y1) -> ((y0 c - y1 s) k, (y0 s + y1 c) k), the reference's
// rope_yarn on the FP16 matmul output (cpu/kernels/elementwise/rope.rs:14-39).
__device__ __forceinline__ void rope_pair(const GhGemvArgs& a, uint32_t row, float acc0,
                                          float acc1, float2 cs, float k, uint16_t& o0,
                                          uint16_t& o1) {
#pragma clang fp contract(off)
    const uint16_t h0 = gh_f2h(acc0), h1 = gh_f2h(acc1);
    const uint32_t pair = (row % a.head_dim) >> 1;
    if (pair >= a.pairs) {
        o0 = h0;
        o1 = h1;
        return;
    }
    const float x0 = gh_h2f(h0), x1 = gh_h2f(h1);
    o0 = gh_f2h((x0 * cs.x - x1 * cs.y) * k);
    o1 = gh_f2h((x0 * cs.y + x1 * cs.x) * k);
}

template <int R, bool SW>
__device__ __forceinline__ void epilogue(const GhGemvArgs& a, const GhGemvSeg& sg, uint32_t t,
                                         uint32_t row0, const float (&v)[R], const float* up,
                                         uint32_t pos, const EpiIn<R>& e) {
#pragma clang fp contract(off)
    if constexpr (SW) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < sg.rows) {
                    // silu_mul (activation.rs:16-29) on the FP16-rounded gate/up projections
                    const float g = gh_h2f(gh_f2h(v[r])), u = gh_h2f(gh_f2h(up[r]));
                    const float silu = g / (1.0f + expf(-g));
                    gh_gpw<uint16_t>(sg.out)[row0 + r] = gh_f2h(gh_h2f(gh_f2h(silu)) * u);
                }
        return;
    }
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
                if (row0 + r < sg.rows)
                    gh_gpw<float>(sg.out)[(size_t)t * sg.rows + row0 + r] = e.res[r] + gh_h2f(gh_f2h(v[r]));
            break;
        case GH_EPI_CACHE: {
            const size_t off = (size_t)pos * sg.rows;
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < sg.rows) gh_gpw<uint16_t>(sg.out)[off + row0 + r] = gh_f2h(v[r]);
            break;
        }
        case GH_EPI_ROPE:
        case GH_EPI_ROPE_CACHE: {
            const bool q = sg.epi == GH_EPI_ROPE;
            const size_t off = q ? 0 : (size_t)pos * sg.rows;
#pragma unroll
            for (int r = 0; r + 1 < R; r += 2) {
                if (row0 + r + 1 < sg.rows) {
                    uint16_t o0, o1;
                    rope_pair(a, row0 + r, v[r], v[r + 1], e.cs[r / 2], e.k, o0, o1);
                    GH_GLOBAL uint16_t* dst = gh_gpw<uint16_t>(sg.out) + off + row0 + r;
                    dst[0] = o0;
                    dst[1] = o1;
                }
            }
            break;
        }
    }
}

// MODE: which row kernels a launch may need (specialized to keep register use low).
enum : int { kModeQ4 = 0, kModeQ6 = 1, kModeMixed = 2, kModeSwiglu = 3 };

// The launch's first-needed arguments, passed as leading scalar kernel parameters that the
// dispatch preloads into SGPRs (-amdgpu-kernarg-preload-count): x and the first weight
// addresses are known without waiting for a kernarg load (~0.3 us per launch measured).
struct GhHot {
    uint64_t x, w0, nw;  // a.x, a.seg[0].w, a.norm_w
    uint32_t in_dim, rows0, tasks, groups;
};

__device__ __forceinline__ uint32_t i_end(const GhGemvArgs& a, const GhHot& h, uint32_t si) {
    return si + 1 < a.nseg ? a.seg[si + 1].task0 : h.tasks;
}

// A wave's work: tasks first, first + stride, ... < ntask of one segment; a task is nch chunks
// of 64 units. The weights of a chunk (all R rows, both matrices for SwiGLU) are requested
// together before any arithmetic; lanes past the last unit re-read the last unit (addresses
// stay valid, loads stay unconditional so the wait counts stay exact) and add nothing.
// `primed`: the caller already loaded the first chunk of the first task into wa.
// W2 (rows of 65-128 units, in_dim 4160..8192): both chunks' weights are requested before
// either is computed, into two register sets, so a task waits on one memory round trip instead
// of two (the same per-lane order of the sums, so the same bits).
template <uint32_t FMT, int R, int M, bool W2 = false>
__device__ __forceinline__ void run_segment(const GhGemvArgs& a, const GhGemvSeg& sg,
                                            uint32_t first, uint32_t stride, uint32_t ntask,
                                            uint32_t t, uint32_t nb, const uint4* xs,
                                            const float4* sums, const Masks& mk, bool primed,
                                            WRow<FMT> (&wa)[M][R], uint32_t pos_all) {
    const uint32_t lane = threadIdx.x & 63u, units = nb * 4;
    const uint32_t nch = (units + 63) / 64;
    first = __builtin_amdgcn_readfirstlane(first);  // wave-uniform: per-task values go to SGPRs
    const uint8_t* w[M];
    w[0] = (const uint8_t*)sg.w;
    if constexpr (M == 2) w[1] = (const uint8_t*)a.aux;
    const uint32_t pos = epi_needs_pos(sg.epi) ? pos_all : 0u;
    for (uint32_t k = first; k < ntask; k += stride) {
        float acc[M][R];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
        EpiIn<R> ei;
        if constexpr (W2) {
            WRow<FMT> wb[M][R];
            const uint32_t u1 = 64 + lane;
            if (!primed) load_step<FMT, R, M>(w, sg.rows, nb, k * R, lane, wa);
            primed = false;
            load_step<FMT, R, M>(w, sg.rows, nb, k * R, min(u1, units - 1), wb);
            __builtin_amdgcn_sched_barrier(0);  // the weights go out before anything waits
            epi_load<R, M == 2>(a, sg, t, k * R, pos, ei);
            compute_step<FMT, R, M>(xs, sums, units, lane, mk, wa, acc);
            if (u1 < units) compute_step<FMT, R, M>(xs, sums, units, u1, mk, wb, acc);
        } else {
            for (uint32_t c = 0; c < nch; ++c) {
                const uint32_t u = c * 64 + lane, uc = min(u, units - 1);
                if (!primed) load_step<FMT, R, M>(w, sg.rows, nb, k * R, uc, wa);
                primed = false;
                if (c == 0) {
                    __builtin_amdgcn_sched_barrier(0);  // the weights go out before anything waits
                    epi_load<R, M == 2>(a, sg, t, k * R, pos, ei);
                }
                if (u < units) compute_step<FMT, R, M>(xs, sums, units, u, mk, wa, acc);
            }
        }
        float v[M][R];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) v[m][r] = gh_wave_sum63(acc[m][r]);
        if (lane == 63u) epilogue<R, M == 2>(a, sg, t, k * R, v[0], M == 2 ? v[M - 1] : nullptr, pos, ei);
    }
}

// Staged x lives in dynamic LDS: 144 B per 64-weight unit (twice for the mixed kernel).
// Waves are split between the segments in proportion to their tasks (args: seg.task0 is the
// first task index, the wave split is recomputed here), so a wave only ever runs one format.
// PRIME: request the first step's weights before x is staged (their latency overlaps the
// staging); the kernels without RMSNorm do. Off for the RMSNorm kernels, where requesting the
// weights ahead of the norm's loads measured slower: primed, the SwiGLU and QKV kernels ran the
// 8B decode at 567-576 tok/s against 589-592 (605 against 628 with the norm weights also
// requested up front), and an L2 warm-up of the first task (one dword per load) in place of
// priming was slower still; for the output GEMV priming measured neutral.
template <int R, int MODE, bool NORM, bool PRIME = !NORM, bool W2 = false>
__device__ __forceinline__ void gemv_body(const GhGemvArgs& a, const GhHot& h) {
    // The position (RoPE / KV-cache epilogues) is read first: loads complete in issue order,
    // so read at the epilogue it waited for every weight load issued before it (the QKV
    // launch of the 8B decode: 8.44 -> 7.72 us).
    const uint32_t pos_all = position(a);
    extern __shared__ uint4 lds[];
    constexpr int M = MODE == kModeSwiglu ? 2 : 1;
    const uint32_t nb = h.in_dim >> 8, units = nb * 4;
    uint4* xs4 = lds;
    float4* xsum4 = (float4*)(lds + 8 * units);
    uint4* xs6 = lds + 9 * units;
    float4* xsum6 = (float4*)(lds + 17 * units);
    const uint32_t waves = h.groups * 4;  // 256-thread workgroups
    const uint32_t gw = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    // segment of this wave and its position among the segment's waves
    uint32_t si = 0, w0 = 0, nw = waves;
    if (a.nseg > 1) {
        uint32_t acc_w = 0;
        for (uint32_t i = 0; i < a.nseg; ++i) {
            const uint32_t t_end = i + 1 < a.nseg ? a.seg[i + 1].task0 : h.tasks;
            const uint32_t t_n = t_end - a.seg[i].task0;
            uint32_t n_w = i + 1 < a.nseg ? (uint32_t)(((uint64_t)t_n * waves + h.tasks - 1) / h.tasks)
                                          : waves - acc_w;
            n_w = max(1u, min(n_w, waves - acc_w - (a.nseg - 1 - i)));
            if (gw >= acc_w && gw < acc_w + n_w) {
                si = i;
                w0 = acc_w;
                nw = n_w;
            }
            acc_w += n_w;
        }
    }
    const GhGemvSeg sg = a.seg[si];
    const uint32_t ntask = i_end(a, h, si) - sg.task0, first = gw - w0;
    const Masks mk = make_masks();
    // The first step's weights of the kernel's primary format are requested before x is
    // staged, so their latency overlaps the staging.
    constexpr uint32_t F0 = MODE == kModeQ6 ? kQ6K : kQ4K;
    // NORM: the first token's FP32 x row and the norm weights (each thread: chunks tid + 256 k)
    // NORM: each thread owns the 16-value items j = tid, tid + 256 of the FP32 x row (item j:
    // float4 chunks 4j .. 4j + 3), the order gh_rms_inverse_256 reduces them in; in_dim <= 5120
    // is at most 320 items
    constexpr uint32_t kItems = 2;
    const uint32_t n4 = h.in_dim >> 2, n16 = h.in_dim >> 4;
    float4 v[kItems][4];
    uint4 wv[kItems][2];
    auto load_norm_row = [&](uint32_t t) __attribute__((always_inline)) {
        const GH_GLOBAL float4* xr = gh_gp<float4>(h.x + (uint64_t)t * h.in_dim * 4);
#pragma unroll
        for (uint32_t it = 0; it < kItems; ++it)
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) v[it][q] = xr[min(4 * (threadIdx.x + 256 * it) + q, n4 - 1)];
    };
    // the norm weights are requested after Σx²'s partial (they are first used after the
    // reduction), so they are not held in registers next to the primed weights
    auto load_norm_w = [&]() __attribute__((always_inline)) {
        const GH_GLOBAL uint4* wn = gh_gp<uint4>(h.nw);
#pragma unroll
        for (uint32_t it = 0; it < kItems; ++it)
#pragma unroll
            for (uint32_t q = 0; q < 2; ++q) wv[it][q] = wn[min(2 * (threadIdx.x + 256 * it) + q, n4 / 2 - 1)];
    };
    if constexpr (NORM && PRIME) {
        load_norm_row(0);
        __builtin_amdgcn_sched_barrier(0);
    }
    WRow<F0> w0r[M][R];
    const bool primed = PRIME && sg.fmt == F0 && first < ntask;
    if (primed) {
        const uint8_t* w[M];
        w[0] = (const uint8_t*)sg.w;
        if constexpr (M == 2) w[1] = (const uint8_t*)a.aux;
        load_step<F0, R, M>(w, sg.rows, nb, first * R, min(threadIdx.x & 63u, units - 1), w0r);
    }
    // the RMSNorm kernels are single-token (the host rejects n > 1): a constant trip count
    // keeps the first token's x row from being carried across the loop into the dot products
    const uint32_t n_tok = NORM ? 1u : a.n;
    for (uint32_t t = 0; t < n_tok; ++t) {
        if (t) __syncthreads();
        auto stage = [&](const auto& x8) {
            if constexpr (MODE == kModeQ6) {
                stage_x<kQ6K>(x8, units, xs4, xsum4);
            } else {
                stage_x<kQ4K>(x8, units, xs4, xsum4);
                if constexpr (MODE == kModeMixed) stage_x<kQ6K>(x8, units, xs6, xsum6);
            }
        };
        if constexpr (NORM) {
            // rmsnorm_x fused: x is the FP32 residual row. Each thread loads its items (16
            // consecutive values) and their norm weights once, the row's Σx² is reduced in the
            // order of gh_rms_inverse_256 (one barrier), and each
            // item's normalized FP16 values f16((x · inverse) · f16 w) — the bits gh_rmsnorm_x
            // stores — are paired in registers and staged straight into the unit layouts.
            float* red = (float*)(lds + (MODE == kModeMixed ? 18 : 9) * units);
            if (t || !PRIME) load_norm_row(t);
            float ss = 0.0f;
#pragma unroll
            for (uint32_t it = 0; it < kItems; ++it)
#pragma unroll
                for (uint32_t q = 0; q < 4; ++q)
                    if (4 * (threadIdx.x + 256 * it) + q < n4) ss = gh_rms_add(ss, v[it][q]);
            load_norm_w();
            const float inv = gh_rms_finish_256(ss, h.in_dim, a.eps, red);
#pragma unroll
            for (uint32_t it = 0; it < kItems; ++it) {
#pragma clang fp contract(off)
                const uint32_t j = threadIdx.x + 256 * it;
                if (j < n16) {
                    auto n2 = [&](float a0, float a1, uint32_t wp) {
                        return (uint32_t)gh_f2h(a0 * inv * gh_h2f(wp & 0xFFFFu)) |
                               ((uint32_t)gh_f2h(a1 * inv * gh_h2f(wp >> 16)) << 16);
                    };
                    const float4* c = v[it];
                    const uint4 lo = make_uint4(n2(c[0].x, c[0].y, wv[it][0].x), n2(c[0].z, c[0].w, wv[it][0].y),
                                                n2(c[1].x, c[1].y, wv[it][0].z), n2(c[1].z, c[1].w, wv[it][0].w));
                    const uint4 hi = make_uint4(n2(c[2].x, c[2].y, wv[it][1].x), n2(c[2].z, c[2].w, wv[it][1].y),
                                                n2(c[3].x, c[3].y, wv[it][1].z), n2(c[3].z, c[3].w, wv[it][1].w));
                    uint4 p02, p13;
                    float sq;
                    pair16(lo, hi, p02, p13, sq);
                    if constexpr (MODE != kModeQ6) {  // Q4_K unit j / 4, quarter j % 4
                        const uint32_t u = j >> 2, q = j & 3u, k0 = (q & 1u) + 4 * (q >> 1);
                        xs4[k0 * units + u] = p02;
                        xs4[(k0 + 2) * units + u] = p13;
                        ((float*)&xsum4[u])[q] = sq;
                    }
                    if constexpr (MODE == kModeQ6 || MODE == kModeMixed) {
                        // Q6_K unit (block j / 16, segment, half) and quarter of the same values
                        const uint32_t u = (j >> 4) * 4 + ((j >> 3) & 1u) * 2 + (j & 1u), q = (j >> 1) & 3u;
                        uint4* x6 = MODE == kModeQ6 ? xs4 : xs6;
                        float4* s6 = MODE == kModeQ6 ? xsum4 : xsum6;
                        x6[q * units + u] = p02;
                        x6[(4 + q) * units + u] = p13;
                        ((float*)&s6[u])[q] = sq;
                    }
                }
            }
        } else {
            const GH_GLOBAL uint4* xh = gh_gp<uint4>(h.x + (uint64_t)t * h.in_dim * 2);
            stage([&](uint32_t e) { return xh[e >> 3]; });
        }
        __syncthreads();
        if constexpr (MODE == kModeQ6) {
            run_segment<kQ6K, R, M, W2>(a, sg, first, nw, ntask, t, nb, xs4, xsum4, mk, primed && t == 0, w0r, pos_all);
        } else if constexpr (MODE == kModeMixed) {
            if (sg.fmt == kQ4K) {
                run_segment<kQ4K, R, M, W2>(a, sg, first, nw, ntask, t, nb, xs4, xsum4, mk, primed && t == 0, w0r,
                                            pos_all);
            } else {
                WRow<kQ6K> w6[M][R];
                run_segment<kQ6K, R, M, W2>(a, sg, first, nw, ntask, t, nb, xs6, xsum6, mk, false, w6, pos_all);
            }
        } else {
            run_segment<kQ4K, R, M, W2>(a, sg, first, nw, ntask, t, nb, xs4, xsum4, mk, primed && t == 0, w0r, pos_all);
        }
    }
}

// Single-token launch of one Q4_K or Q6_K matrix with in_dim <= 4096 (one unit per lane).
// The workgroup stages x once in LDS as FP16 pairs (each thread pairs 16 values it requested
// before the first task's weights; only an LDS fence and s_barrier separate the staging from
// its reads, so the weight loads stay in flight across it); each task reads its pairs from LDS
// again, half a unit at a time, so no x is held in registers between tasks. That keeps the
// two-row Q4_K kernel at 69 VGPRs: seven waves per SIMD, 7,168 resident waves, so the 6,144
// tasks of a 12288x4096 launch run in one round (pairs held per wave: 104 VGPRs, four waves
// per SIMD, one and a half rounds; 7.7 -> 7.3 us). x fetched per wave instead of staged
// (8 KiB each, 16 waves per CU) measured ~1.5 us of a 10 us 12288x4096 launch.
// Workgroups of GH_DIRECT_WAVES = 8 waves: a 4096x4096 launch is 256 workgroups, one per CU,
// each staging x once (four-wave workgroups, two per CU: Q4_K 4.08 -> 4.01 us, Q6_K 5.00 ->
// 4.90 us back to back over distinct weights; sixteen waves leave half the CUs idle, 5.3 us).
template <int R, uint32_t FMT>
__device__ __forceinline__ void gemv_direct(const GhGemvArgs& a, const GhHot& h) {
    __shared__ uint4 xs[512];     // x as FP16 pairs, stage_x's layout (in_dim <= 4096)
    __shared__ float4 sums[64];
    const uint32_t lane = threadIdx.x & 63u, nb = h.in_dim >> 8, units = nb * 4;
    const uint32_t waves = h.groups * GH_DIRECT_WAVES;
    const uint32_t gw = blockIdx.x * GH_DIRECT_WAVES + (threadIdx.x >> 6);
    GhGemvSeg sg = a.seg[0];
    sg.w = h.w0;
    sg.rows = h.rows0;
    const uint32_t u = min(lane, units - 1);
    const uint8_t* w[1] = {(const uint8_t*)sg.w};
    const GH_GLOBAL uint4* xh = gh_gp<uint4>(h.x);
    // thread t pairs item t = (unit t/4, quarter t%4): 16 FP16 values, two 16-byte loads
    // (threads past the last item load it again and store nothing)
    const uint32_t t = threadIdx.x, it = min(t, units * 4 - 1), iu = it >> 2, iq = it & 3u;
    const uint32_t e = FMT == kQ4K ? 16 * it
                                   : (iu >> 2) * 256 + ((iu >> 1) & 1u) * 128 + iq * 32 + (iu & 1u) * 16;
    const uint4 x0 = xh[e >> 3], x1 = xh[(e >> 3) + 1];
    __builtin_amdgcn_sched_barrier(0);
    // waves past the last task (the grid has at most seven, all in the last workgroup) load
    // the last task's rows, take part in the barrier, and leave
    const uint32_t t0 = min(gw, h.tasks - 1);
    WRow<FMT> wr[1][R];
    load_step<FMT, R, 1>(w, sg.rows, nb, t0 * R, u, wr);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t pos = epi_needs_pos(sg.epi) ? position(a) : 0u;
    EpiIn<R> ei;
    epi_load<R, false>(a, sg, 0, t0 * R, pos, ei);
    if (t < units * 4) {
        uint4 p02, p13;
        float sq;
        pair16(x0, x1, p02, p13, sq);
        if constexpr (FMT == kQ4K) {
            const uint32_t k0 = (iq & 1u) + 4 * (iq >> 1);
            xs[k0 * units + iu] = p02;
            xs[(k0 + 2) * units + iu] = p13;
        } else {
            xs[iq * units + iu] = p02;
            xs[(4 + iq) * units + iu] = p13;
        }
        ((float*)&sums[iu])[iq] = sq;
    }
    gh_lds_barrier();
    if (gw >= h.tasks) return;  // wave-uniform
    const Masks mk = make_masks();
    for (uint32_t k = gw; k < h.tasks; k += waves) {
        if (k != gw) {
            load_step<FMT, R, 1>(w, sg.rows, nb, k * R, u, wr);
            epi_load<R, false>(a, sg, 0, k * R, pos, ei);
        }
        float acc[1][R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[0][r] = 0.0f;
        if (lane < units) {
            // opaque per task: keeps the pair reads inside the loop (not hoisted and held)
            uint32_t ut = u;
            asm volatile("" : "+v"(ut));
            if constexpr (FMT == kQ4K)
                compute_q4_halves<R>(xs, sums, units, ut, mk, wr[0], acc[0]);
            else
                compute_step<FMT, R, 1>(xs, sums, units, u, mk, wr, acc);
        }
        float v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = gh_wave_sum63(acc[0][r]);
        if (lane == 63u) epilogue<R, false>(a, sg, 0, k * R, v, nullptr, pos, ei);
    }
}

// Single-token launch of one matrix with 4096 < in_dim <= 16384: the NW waves of a
// workgroup (64·NW threads) split the in-dimension (wave w: units w·q .. w·q + q, one per lane,
// q = ceil(units / NW)), each pairs its lanes' x slices in registers once, and every task's
// loads go out from all NW waves at once — one memory round trip per task instead of one
// per 64-unit chunk. The NW partial sums of a row are added in wave order through LDS.
// NW = 3 for in_dim 12288 (192 units: every lane busy), 4 otherwise.
template <int R, uint32_t FMT, int NW = 4>
__device__ __forceinline__ void gemv_splitk(const GhGemvArgs& a, const GhHot& h) {
    __shared__ float part[NW][R];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nb = h.in_dim >> 8;
    const uint32_t units = nb * 4, q = (units + NW - 1) / NW;
    const uint32_t uw = wave * q + lane;                    // this lane's unit
    const bool active = lane < q && uw < units;
    const uint32_t u = min(uw, units - 1);
    GhGemvSeg sg = a.seg[0];
    sg.w = h.w0;
    sg.rows = h.rows0;
    const uint8_t* w[1] = {(const uint8_t*)sg.w};
    const GH_GLOBAL uint4* xh = gh_gp<uint4>(h.x);
    uint4 xraw[8];
    load_unit_x<FMT>([&](uint32_t e) { return xh[e >> 3]; }, u, xraw);
    __builtin_amdgcn_sched_barrier(0);
    WRow<FMT> wr[1][R];
    // unconditional (clamped task): loads outside branches keep the wait counts exact
    load_step<FMT, R, 1>(w, sg.rows, nb, min(blockIdx.x, h.tasks - 1) * R, u, wr);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t pos = epi_needs_pos(sg.epi) ? position(a) : 0u;
    EpiIn<R> ei;
    if (blockIdx.x < h.tasks) epi_load<R, false>(a, sg, 0, blockIdx.x * R, pos, ei);
    uint4 xv[8];
    float4 xsum;
    pair_raw<FMT>(xraw, xv, xsum);
    const Masks mk = make_masks();
    for (uint32_t k = blockIdx.x; k < h.tasks; k += h.groups) {
        if (k != blockIdx.x) {
            load_step<FMT, R, 1>(w, sg.rows, nb, k * R, u, wr);
            epi_load<R, false>(a, sg, 0, k * R, pos, ei);
        }
        float acc[1][R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[0][r] = 0.0f;
        if (active) compute_regs<FMT, R, 1>(xv, xsum, u, mk, wr, acc);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = gh_wave_sum63(acc[0][r]);
            if (lane == 63u) part[wave][r] = v;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float v[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                v[r] = part[0][r];
#pragma unroll
                for (int i = 1; i < NW; ++i) v[r] += part[i][r];
            }
            epilogue<R, false>(a, sg, 0, k * R, v, nullptr, pos, ei);
        }
        __syncthreads();
    }
}

}  // namespace

// Kernel parameters: the hot scalars (GhHot), preloaded into SGPRs, then the full arguments.
#define GH_HOT_PARAMS                                                                            \
    uint64_t x, uint64_t w0, uint64_t nw, uint32_t in_dim, uint32_t rows0, uint32_t tasks,        \
        uint32_t groups, GhGemvArgs a
#define GH_HOT GhHot{x, w0, nw, in_dim, rows0, tasks, groups}

// NORM kernels (suffix _n) stage the RMSNorm of an FP32 x (norm_w set); the others read FP16 x.
#define GH_GEMV(NAME, R, MODE)                                                                   \
    GH_KERNEL __launch_bounds__(256) void NAME(GH_HOT_PARAMS) { gemv_body<R, MODE, false>(a, GH_HOT); } \
    GH_KERNEL __launch_bounds__(256) void NAME##_n(GH_HOT_PARAMS) { gemv_body<R, MODE, true>(a, GH_HOT); }
GH_GEMV(gh_gemv_q4k_r1, 1, kModeQ4)
GH_GEMV(gh_gemv_q4k_r2, 2, kModeQ4)
GH_GEMV(gh_gemv_q6k_r1, 1, kModeQ6)
GH_GEMV(gh_gemv_q6k_r2, 2, kModeQ6)
GH_KERNEL __launch_bounds__(256) void gh_gemv_mixed_r2(GH_HOT_PARAMS) { gemv_body<2, kModeMixed, false>(a, GH_HOT); }
// The RMSNorm mixed (Q/K/V) kernel runs at least three waves per SIMD (it needs 106 VGPRs, so
// four): with 3 x 256 CUs x 4 waves resident, an 8B-shaped QKV launch (4096 + 1024 + 1024 rows,
// R = 2) is one task per wave instead of two rounds.
GH_KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void gh_gemv_mixed_r2_n(GH_HOT_PARAMS) {
    gemv_body<2, kModeMixed, true>(a, GH_HOT);
}
GH_GEMV(gh_gemv_swiglu_r1, 1, kModeSwiglu)
GH_GEMV(gh_gemv_swiglu_r2, 2, kModeSwiglu)
// RMSNorm kernels for rows of 65-128 units (in_dim 4160..8192, e.g. the 14B shape's 5120): both
// 64-unit chunks of a task requested at once (suffix _nw)
GH_KERNEL __launch_bounds__(256) void gh_gemv_q4k_r2_nw(GH_HOT_PARAMS) {
    gemv_body<2, kModeQ4, true, false, true>(a, GH_HOT);
}
GH_KERNEL __launch_bounds__(256) void gh_gemv_q6k_r2_nw(GH_HOT_PARAMS) {
    gemv_body<2, kModeQ6, true, false, true>(a, GH_HOT);
}
GH_KERNEL __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void gh_gemv_mixed_r2_nw(GH_HOT_PARAMS) {
    gemv_body<2, kModeMixed, true, false, true>(a, GH_HOT);
}
GH_KERNEL __launch_bounds__(256) void gh_gemv_swiglu_r2_nw(GH_HOT_PARAMS) {
    gemv_body<2, kModeSwiglu, true, false, true>(a, GH_HOT);
}
// direct-x variants (suffix _d): single token, one matrix, in_dim <= 4096, no RMSNorm
GH_KERNEL __launch_bounds__(512) void gh_gemv_q4k_r1_d(GH_HOT_PARAMS) { gemv_direct<1, kQ4K>(a, GH_HOT); }
GH_KERNEL __launch_bounds__(512) void gh_gemv_q4k_r2_d(GH_HOT_PARAMS) { gemv_direct<2, kQ4K>(a, GH_HOT); }
GH_KERNEL __launch_bounds__(512) void gh_gemv_q6k_r1_d(GH_HOT_PARAMS) { gemv_direct<1, kQ6K>(a, GH_HOT); }
GH_KERNEL __launch_bounds__(512) void gh_gemv_q6k_r2_d(GH_HOT_PARAMS) { gemv_direct<2, kQ6K>(a, GH_HOT); }
// split-K variants (suffix _k): single token, one matrix, 4096 < in_dim <= 16384, no RMSNorm
GH_KERNEL __launch_bounds__(256) void gh_gemv_q4k_r1_k(GH_HOT_PARAMS) { gemv_splitk<1, kQ4K>(a, GH_HOT); }
GH_KERNEL __launch_bounds__(256) void gh_gemv_q4k_r2_k(GH_HOT_PARAMS) { gemv_splitk<2, kQ4K>(a, GH_HOT); }
GH_KERNEL __launch_bounds__(256) void gh_gemv_q6k_r1_k(GH_HOT_PARAMS) { gemv_splitk<1, kQ6K>(a, GH_HOT); }
GH_KERNEL __launch_bounds__(256) void gh_gemv_q6k_r2_k(GH_HOT_PARAMS) { gemv_splitk<2, kQ6K>(a, GH_HOT); }
GH_KERNEL __launch_bounds__(192) void gh_gemv_q4k_r4_k3(GH_HOT_PARAMS) { gemv_splitk<4, kQ4K, 3>(a, GH_HOT); }
GH_KERNEL __launch_bounds__(192) void gh_gemv_q6k_r4_k3(GH_HOT_PARAMS) { gemv_splitk<4, kQ6K, 3>(a, GH_HOT); }

// Prefill GEMM on the matrix cores: out[t][r] = Σ_k x[t][k] · w[r][k] for n tokens of FP16
// activations against Q4_K / Q6_K weights in the device layout (gh_kargs.h).
//
// Tiling: a 256-thread workgroup owns 128 tokens x 128 weight rows; its four waves own 64 x 64
// each as 4 x 4 tiles of v_mfma_f32_16x16x32_f16 (A = activations, M = tokens; B = weights,
// N = rows; FP32 accumulators). K advances one 64-weight unit per stage. Each stage, the
// workgroup copies the x tile (128 x 64 FP16) and dequantizes the w tile (128 rows x 64) into
// LDS: w = FP16(RNE(the reference's FP32 dequantized weight)), computed per weight exactly as
// dequant_row does (Q4_K: (d·sc)·q - dmin·mn; Q6_K: (d·sc)·(q - 32); cpu/dequant.rs:93-123,
// 274-308). LDS is double-buffered; the next unit's global loads are in flight while the
// matrix cores run on the current one, and one barrier separates stages.
//
// A Q6_K unit's 64 weights are not contiguous in k (16 from each quarter of a 128-weight half
// block); x is staged in the same permuted order, which leaves every dot product unchanged.
//
// Numerics: the only departure from the reference CPU kernel (q4k.rs:218-325 / q6k.rs:157-235,
// FP32 dequantized weights, FP32 accumulation) is the FP16 rounding of each dequantized
// weight (relative 2^-12 at most) — the rounding the reference's own cooperative-matrix
// prefill shaders carry (vulkan/shaders/matmul/matmul_q4_k_coopmat_f16out.comp). Products of
// FP16 values are exact in FP32; accumulation is FP32.
//
// Split-K (grid.z > 1): each split covers a contiguous range of units and writes FP32
// partials [split][n][rows]; gh_gemm_reduce sums them in split order and rounds to FP16.
#include "gh_common.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kQ4K = 12, kQ6K = 14;
constexpr int BK = 64;        // k per stage: one 64-weight unit
constexpr int LDK = BK + 8;   // LDS row pitch in FP16 (144 B: conflict-free 16-byte reads)
constexpr int BT = 128;       // tokens per workgroup
constexpr int BR = 128;       // weight rows per workgroup

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return (uint32_t)gh_f2h(a) | ((uint32_t)gh_f2h(b) << 16);
}

// k of FP16 chunk c (8 consecutive weights) of unit u, in LDS order.
template <uint32_t FMT>
__device__ __forceinline__ uint32_t chunk_k(uint32_t u, uint32_t c) {
    if constexpr (FMT == kQ4K) {
        return u * 64 + c * 8;
    } else {
        // unit (block b, half s, h): position 16q + i holds k = 256b + 128s + 32q + 16h + i
        return (u >> 2) * 256 + ((u >> 1) & 1u) * 128 + (u & 1u) * 16 + (c >> 1) * 32 + (c & 1u) * 8;
    }
}

struct XStage {
    uint4 v0, v1, v2, v3;
};

struct WStage {
    uint4 q, hd, qh;  // Q4_K: q plane chunk + block header; Q6_K: ql chunk, scales, qh chunk
    uint32_t d;       // Q6_K: d (FP16 bits)
};

struct Tile {
    uint32_t t0, r0, n, rows, in_dim, nb;
};

template <uint32_t FMT>
__device__ __forceinline__ void load_stage(const GhGemmArgs& a, const Tile& tl, uint32_t u,
                                           XStage& xs, WStage& ws) {
    const uint32_t tid = threadIdx.x;
    // chunk c = tid + 256 i: token c / 8, FP16 chunk c % 8 (the same for every i)
    const uint32_t kc = chunk_k<FMT>(u, tid & 7u);
    auto xload = [&](uint32_t i) {
        const uint32_t tok = min(tl.t0 + ((tid + 256u * i) >> 3), tl.n - 1);
        return *gh_gp<uint4>(a.x + ((uint64_t)tok * tl.in_dim + kc) * 2);
    };
    xs.v0 = xload(0);
    xs.v1 = xload(1);
    xs.v2 = xload(2);
    xs.v3 = xload(3);
    const uint32_t row = min(tl.r0 + (tid >> 1), tl.rows - 1), part = tid & 1u;
    const uint64_t nb = tl.nb, blk = (uint64_t)row * nb + (u >> 2);
    if constexpr (FMT == kQ4K) {
        ws.q = *gh_gp<uint4>(a.w + (uint64_t)row * GH_Q4K_QS_BYTES * nb + part * nb * 64 + u * 16);
        ws.hd = *gh_gp<uint4>(a.w + (uint64_t)tl.rows * GH_Q4K_QS_BYTES * nb + blk * 16);
    } else {
        const uint64_t rq = a.w + (uint64_t)row * GH_Q6K_QLH_BYTES * nb + u * 16;
        ws.q = *gh_gp<uint4>(rq + part * nb * 64);
        ws.qh = *gh_gp<uint4>(rq + 2 * nb * 64);
        ws.hd = *gh_gp<uint4>(a.w + (uint64_t)tl.rows * GH_Q6K_QLH_BYTES * nb + blk * 16);
        ws.d = *gh_gp<uint16_t>(a.w + (uint64_t)tl.rows * 208 * nb + blk * 2);
    }
}

// Copy x and dequantize w into one LDS buffer.
template <uint32_t FMT>
__device__ __forceinline__ void store_stage(uint32_t u, const XStage& xs, const WStage& ws,
                                            _Float16* xb, _Float16* wb) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x;
    _Float16* xd = xb + (tid >> 3) * LDK + (tid & 7u) * 8;  // + 32 tokens per i
    *(uint4*)(xd) = xs.v0;
    *(uint4*)(xd + 32 * LDK) = xs.v1;
    *(uint4*)(xd + 64 * LDK) = xs.v2;
    *(uint4*)(xd + 96 * LDK) = xs.v3;
    const uint32_t row = tid >> 1, part = tid & 1u;
    _Float16* dst = wb + row * LDK;
    const uint32_t qw[4] = {ws.q.x, ws.q.y, ws.q.z, ws.q.w};
    uint32_t lo[8], hi[8];
    if constexpr (FMT == kQ4K) {
        const uint32_t g = u & 3u;
        uint32_t sc0, mn0, sc1, mn1;
        gh_q4k_scale_min(ws.hd, 2 * g, sc0, mn0);
        gh_q4k_scale_min(ws.hd, 2 * g + 1, sc1, mn1);
        const float d = gh_h2f(ws.hd.x & 0xFFFFu), dmin = gh_h2f(ws.hd.x >> 16);
        const float d1 = d * (float)sc0, m1 = dmin * (float)mn0;
        const float d2 = d * (float)sc1, m2 = dmin * (float)mn1;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const uint32_t b0 = (qw[j] >> (8 * e)) & 0xFFu, b1 = (qw[j] >> (8 * e + 8)) & 0xFFu;
                lo[2 * j + e / 2] = pack_h2(d1 * (float)(b0 & 0xFu) - m1, d1 * (float)(b1 & 0xFu) - m1);
                hi[2 * j + e / 2] = pack_h2(d2 * (float)(b0 >> 4) - m2, d2 * (float)(b1 >> 4) - m2);
            }
        // low nibbles: sub-block 2g, positions 16·part + i; high: sub-block 2g+1, 32 + 16·part + i
        *(uint4*)(dst + 16 * part) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *(uint4*)(dst + 16 * part + 8) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
        *(uint4*)(dst + 32 + 16 * part) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *(uint4*)(dst + 40 + 16 * part) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
    } else {
        // part 0: ql plane a -> quarters 0 (low nibble, qh bits 0-1) and 2 (high, bits 4-5);
        // part 1: plane b -> quarters 1 (bits 2-3) and 3 (bits 6-7). Scale of quarter q:
        // int8 scales[8s + h + 2q].
        const uint32_t s = (u >> 1) & 1u, h = u & 1u;
        const uint32_t scw[4] = {ws.hd.x, ws.hd.y, ws.hd.z, ws.hd.w};
        const uint32_t ia = 8 * s + h + 2 * part, ib = ia + 4;
        const float d = gh_h2f(ws.d);
        const float da = d * (float)(int8_t)(scw[ia >> 2] >> (8 * (ia & 3u)));
        const float db = d * (float)(int8_t)(scw[ib >> 2] >> (8 * (ib & 3u)));
        const uint32_t qh[4] = {ws.qh.x, ws.qh.y, ws.qh.z, ws.qh.w};
        const uint32_t sl = 2 * part, sh = 4 + 2 * part;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const uint32_t b0 = (qw[j] >> (8 * e)) & 0xFFu, b1 = (qw[j] >> (8 * e + 8)) & 0xFFu;
                const uint32_t h0 = (qh[j] >> (8 * e)) & 0xFFu, h1 = (qh[j] >> (8 * e + 8)) & 0xFFu;
                const int32_t qa0 = (int32_t)((b0 & 0xFu) | (((h0 >> sl) & 3u) << 4)) - 32;
                const int32_t qa1 = (int32_t)((b1 & 0xFu) | (((h1 >> sl) & 3u) << 4)) - 32;
                const int32_t qb0 = (int32_t)((b0 >> 4) | (((h0 >> sh) & 3u) << 4)) - 32;
                const int32_t qb1 = (int32_t)((b1 >> 4) | (((h1 >> sh) & 3u) << 4)) - 32;
                lo[2 * j + e / 2] = pack_h2(da * (float)qa0, da * (float)qa1);
                hi[2 * j + e / 2] = pack_h2(db * (float)qb0, db * (float)qb1);
            }
        *(uint4*)(dst + 16 * part) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *(uint4*)(dst + 16 * part + 8) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
        *(uint4*)(dst + 32 + 16 * part) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *(uint4*)(dst + 40 + 16 * part) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
    }
}

template <uint32_t FMT>
__device__ __forceinline__ void gemm_body(const GhGemmArgs& a) {
    __shared__ __attribute__((aligned(16))) _Float16 xbuf[2][BT * LDK];
    __shared__ __attribute__((aligned(16))) _Float16 wbuf[2][BR * LDK];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    Tile tl{blockIdx.y * BT, blockIdx.x * BR, a.n, a.rows, a.in_dim, a.in_dim >> 8};
    const uint32_t units = a.in_dim / 64;
    const uint32_t per = (units + gridDim.z - 1) / gridDim.z;
    const uint32_t u0 = blockIdx.z * per, u1 = min(units, u0 + per);
    const uint32_t wt = (wave & 1u) * 64, wr = (wave >> 1) * 64;  // this wave's sub-tile
    const uint32_t fm = lane & 15u, fk = (lane >> 4) * 8;        // fragment row, k offset

    f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    if (u0 < u1) {
        XStage xs;
        WStage ws;
        load_stage<FMT>(a, tl, u0, xs, ws);
        store_stage<FMT>(u0, xs, ws, xbuf[0], wbuf[0]);
        __syncthreads();
        for (uint32_t u = u0; u < u1; ++u) {
            const uint32_t cur = (u - u0) & 1u;
            const bool more = u + 1 < u1;
            if (more) load_stage<FMT>(a, tl, u + 1, xs, ws);
            const _Float16* xb = xbuf[cur];
            const _Float16* wb = wbuf[cur];
#pragma unroll
            for (int kk = 0; kk < BK; kk += 32) {
                h8 af[4], bf[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) af[i] = *(const h8*)(xb + (wt + 16 * i + fm) * LDK + kk + fk);
#pragma unroll
                for (int j = 0; j < 4; ++j) bf[j] = *(const h8*)(wb + (wr + 16 * j + fm) * LDK + kk + fk);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
            if (more) store_stage<FMT>(u + 1, xs, ws, xbuf[cur ^ 1u], wbuf[cur ^ 1u]);
            __syncthreads();
        }
    }

    // D[m][n] of tile (i, j): lane holds m = 4·(lane/16) + e, n = lane % 16.
    const uint32_t row = tl.r0 + wr + fm;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t t = tl.t0 + wt + 16 * i + 4 * (lane >> 4) + e;
            if (t >= tl.n) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t r = row + 16 * j;
                if (r >= tl.rows) continue;
                if (gridDim.z == 1)
                    gh_gpw<uint16_t>(a.out)[(uint64_t)t * tl.rows + r] = gh_f2h(acc[i][j][e]);
                else
                    gh_gpw<float>(a.part)[((uint64_t)blockIdx.z * tl.n + t) * tl.rows + r] = acc[i][j][e];
            }
        }
}

}  // namespace

GH_KERNEL __launch_bounds__(256) void gh_gemm_q4k(GhGemmArgs a) { gemm_body<kQ4K>(a); }
GH_KERNEL __launch_bounds__(256) void gh_gemm_q6k(GhGemmArgs a) { gemm_body<kQ6K>(a); }

// Sum split-K partials in split order, round to FP16: out[i] = f16(Σ_s part[s][i]).
GH_KERNEL __launch_bounds__(256) void gh_gemm_reduce(GhGemmArgs a) {
    const uint64_t total = (uint64_t)a.n * a.rows;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        float s = 0.0f;
        for (uint32_t k = 0; k < a.splits; ++k) s += gh_gp<float>(a.part)[k * total + i];
        gh_gpw<uint16_t>(a.out)[i] = gh_f2h(s);
    }
}

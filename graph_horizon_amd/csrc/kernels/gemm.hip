// Prefill GEMM on the matrix cores: out[t][r] = Σ_k x[t][k] · w[r][k] for n tokens of FP16
// activations against Q4_K / Q6_K weights in the device layout (gh_kargs.h).
//
// Every GEMM is a 512-thread workgroup over 256 (or 128) tokens x BR weight rows, K advancing
// one 64-weight unit per stage through a 3-stage LDS ring, one barrier per unit, with
// v_mfma_f32_32x32x16_f16 tiles (A = activations, M = tokens; B = weights, N = rows; FP32
// accumulators). Two forms:
//   gemm3_body (dequantizing; the C3 workload): warp-specialized. Waves 4-7 (producers) fetch
//     the raw weight bytes of their rows a 256-weight block (4 units) at a time, the next block
//     in flight while the current one is dequantized, and write each unit into its LDS stage as
//     FP16, one row per lane; waves 0-3 (consumers) fetch their activation lines one unit
//     ahead (three in the 128-token tiles) straight into LDS with global_load_lds_dwordx4 and
//     run the MFMA tiles. K splits start and end on block boundaries (gh_gemm_split_units).
//     Q4_K: w = FP16(RNE(the reference's FP32 dequantized weight)), computed as dequant_row
//     does ((d·sc)·q - dmin·mn, cpu/dequant.rs:93-123). Q6_K: (q - 32)·(d·sc) as one fused
//     multiply-add u·da + (-32·da) rounded once to FP16 (v_fma_mix); the reference rounds the
//     same exact product to FP32 first (dequant.rs:274-308), and the two roundings differ by
//     one FP16 ulp when that FP32 value lands exactly on an FP16 tie.
//   gemm4_body (over FP16 weight copies made by dequant_f16, the same values): every wave runs
//     the matrix cores; activation lines and weight rows both arrive by LDS DMA, and the k
//     order of every sum is gemm3_body's, so the bits are the same.
// A multi-matrix launch (gemm3_mixed, the prefill's Q/K/V) runs each row tile in its matrix's
// format over the shared LDS block. SwiGLU's gate and up run as one launch of pair tiles
// (gh_gemm3/4w_swiglu_*): each tile holds matching gate and up rows (pair_row), K unsplit, and
// the consumers apply silu_mul to their sums in registers (pair_write96 / pair_write128).
//
// A Q6_K unit's 64 weights are not contiguous in k (16 from each quarter of a 128-weight half
// block); x is staged in the same permuted order, which leaves every dot product unchanged.
//
// Numerics: the only departure from the reference CPU kernel (q4k.rs:218-325 / q6k.rs:157-235,
// FP32 dequantized weights, FP32 accumulation) is the FP16 rounding of each dequantized
// weight (relative 2^-11 at most) — the rounding the reference's own cooperative-matrix
// prefill shaders carry (vulkan/shaders/matmul/matmul_q4_k_coopmat_f16out.comp). Products of
// FP16 values are exact in FP32; accumulation is FP32.
//
// Split-K (grid.z > 1): each split covers a contiguous range of units and writes FP32
// partials [split][n][rows]; gh_gemm_reduce sums them in split order and rounds to FP16
// (gh_gemm_reduce_seg, gh_gemm_reduce_swiglu and gh_gemm_tail fold the prefill driver's RoPE,
// K/V-cache writes, silu_mul, residual add and RMSNorm into that sum).
#include "gh_common.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));  // a first-class vector (no struct copies)

constexpr uint32_t kQ4K = 12, kQ6K = 14;
constexpr int BK = 64;        // k per stage: one 64-weight unit
constexpr int LDK = BK + 8;   // LDS row pitch in FP16 (144 B: conflict-free 16-byte reads)

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

struct WStage {
    uint4 q, hd, qh;  // Q4_K: q plane chunk + block header; Q6_K: ql chunk, scales, qh chunk
    uint32_t d;       // Q6_K: d (FP16 bits)
};

// Thread tid < 2·BR loads part tid / BR of weight row r0 + tid % BR for unit u (consecutive
// lanes on consecutive rows: their 16-byte LDS stores, one row pitch apart, hit distinct banks).
template <uint32_t FMT, int BR>
__device__ __forceinline__ void load_w(const GhGemmArgs& a, uint32_t r0, uint32_t u, WStage& ws,
                                       uint32_t tid = threadIdx.x) {
    const uint32_t nb = a.in_dim >> 8;
    const uint32_t row = min(r0 + tid % BR, a.rows - 1), part = tid / BR;
    const uint64_t blk = (uint64_t)row * nb + (u >> 2);
    if constexpr (FMT == kQ4K) {
        ws.q = *gh_gp<uint4>(a.w + (uint64_t)row * GH_Q4K_QS_BYTES * nb + (uint64_t)part * nb * 64 + u * 16);
        ws.hd = *gh_gp<uint4>(a.w + (uint64_t)a.rows * GH_Q4K_QS_BYTES * nb + blk * 16);
    } else {
        const uint64_t rq = a.w + (uint64_t)row * GH_Q6K_QLH_BYTES * nb + u * 16;
        ws.q = *gh_gp<uint4>(rq + (uint64_t)part * nb * 64);
        ws.qh = *gh_gp<uint4>(rq + 2ull * nb * 64);
        ws.hd = *gh_gp<uint4>(a.w + (uint64_t)a.rows * GH_Q6K_QLH_BYTES * nb + blk * 16);
        ws.d = *gh_gp<uint16_t>(a.w + (uint64_t)a.rows * 208 * nb + blk * 2);
    }
}

// The raw bytes of one thread's part of a weight row over a whole 256-weight block (its 4
// units), for the producers of gemm3_body. A unit's chunk of one row is 16 bytes, and the
// 4 units of a block are 64 contiguous bytes of each plane, so the block's loads of each plane
// are issued back to back: all but the first find the row's line already requested in the
// CU's L1. Fetched one unit at a time, each 16-byte load of a different row is its own L1
// miss, and the line is requested again for the next unit (it does not survive the activation
// stream in the L1 between units), which held the kernels at the L1's rate of misses.
template <uint32_t FMT>
struct WBlock {
    uint4 q[4];                       // Q4_K: qs chunks (half `part`); Q6_K: ql plane `part`
    uint4 qh[FMT == kQ6K ? 4 : 1];    // Q6_K: qh chunks
    uint4 hd;                         // Q4_K: block header; Q6_K: int8 scales
    uint32_t d;                       // Q6_K: d (FP16 bits)
};

// PAIR (SwiGLU's gate and up in one tile, the gh_gemm3/4w_swiglu_* kernels; the gate matrix at
// a.w, the up matrix of the same shape at a.aux), r0 = BR / 2 · tile. BR = 96: LDS row lr holds gate row
// r0 + lr (lr < 32), up row r0 + lr - 32 (< 64), gate row r0 + lr - 32 (< 80) or up row
// r0 + lr - 48. BR = 128: rows alternate by 32, gate rows r0 .. + 32 | up rows r0 .. + 32 |
// gate rows r0 + 32 .. + 32 | up rows r0 + 32 .. + 32.
template <int BR>
__device__ __forceinline__ uint32_t pair_row(uint32_t lr, uint64_t& wbase, const GhGemmArgs& a) {
    if constexpr (BR == 96) {
        wbase = ((lr >= 32 && lr < 64) || lr >= 80) ? a.aux : a.w;
        return lr < 64 ? lr % 32u : 32u + (lr - 64) % 16u;
    } else {
        wbase = (lr / 32) % 2 ? a.aux : a.w;
        return (lr / 64) * 32 + lr % 32;
    }
}

template <uint32_t FMT, int BR, bool PAIR = false>
__device__ __forceinline__ void load_wblock(const GhGemmArgs& a, uint32_t r0, uint32_t b, WBlock<FMT>& wb,
                                            uint32_t tid) {
    const uint32_t nb = a.in_dim >> 8;
    const uint32_t lr = tid % BR, part = tid / BR;
    uint64_t wbase = a.w;
    uint32_t row = r0 + lr;
    if constexpr (PAIR) row = r0 + pair_row<BR>(lr, wbase, a);
    row = min(row, a.rows - 1);
    const uint64_t blk = (uint64_t)row * nb + b;
    if constexpr (FMT == kQ4K) {
        const uint64_t q = wbase + (uint64_t)row * GH_Q4K_QS_BYTES * nb + (uint64_t)part * nb * 64 + b * 64;
#pragma unroll
        for (int j = 0; j < 4; ++j) wb.q[j] = *gh_gp<uint4>(q + 16 * j);
        wb.hd = *gh_gp<uint4>(wbase + (uint64_t)a.rows * GH_Q4K_QS_BYTES * nb + blk * 16);
        wb.d = 0;
    } else {
        static_assert(!PAIR, "the gate/up pair tiles are Q4_K");
        const uint64_t rq = a.w + (uint64_t)row * GH_Q6K_QLH_BYTES * nb + b * 64;
#pragma unroll
        for (int j = 0; j < 4; ++j) wb.q[j] = *gh_gp<uint4>(rq + (uint64_t)part * nb * 64 + 16 * j);
#pragma unroll
        for (int j = 0; j < 4; ++j) wb.qh[j] = *gh_gp<uint4>(rq + 2ull * nb * 64 + 16 * j);
        wb.hd = *gh_gp<uint4>(a.w + (uint64_t)a.rows * GH_Q6K_QLH_BYTES * nb + blk * 16);
        wb.d = *gh_gp<uint16_t>(a.w + (uint64_t)a.rows * 208 * nb + blk * 2);
    }
}

// Dequantize the thread's 32 weights into its LDS row.
template <uint32_t FMT, int BR>
__device__ __forceinline__ void store_w(uint32_t u, const WStage& ws, _Float16* wb,
                                        uint32_t tid = threadIdx.x) {
#pragma clang fp contract(off)
    const uint32_t row = tid % BR, part = tid / BR;
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
        // nibbles four at a time: byte e of lo4 / hi4 is the low / high nibble of byte e.
        // d·sc and dmin·mn are exact in FP32 (an FP16 times a 6-bit integer), and so is
        // (d·sc)·q for a 4-bit q (at most 21 significant bits): the reference's product,
        // then difference, rounds once, as one FMA does, so the FMA gives the same FP32 value.
        auto w2 = [](uint32_t q4, int e, float sc, float mn) __attribute__((always_inline)) {
            typedef _Float16 hv2 __attribute__((ext_vector_type(2)));
            const float f0 = (float)((q4 >> (8 * e)) & 0xFFu), f1 = (float)((q4 >> (8 * e + 8)) & 0xFFu);
            float v0 = __builtin_fmaf(sc, f0, -mn), v1 = __builtin_fmaf(sc, f1, -mn);
            // the FP32 values are rounded to FP16 as a second step (v_cvt_pk_f16_f32), not fused
            // into one rounding of the exact value (v_fma_mix), which differs on FP16 ties
            asm volatile("" : "+v"(v0), "+v"(v1));
            const hv2 r = {(_Float16)v0, (_Float16)v1};
            return __builtin_bit_cast(uint32_t, r);
        };
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t lo4 = qw[j] & 0x0F0F0F0Fu, hi4 = (qw[j] >> 4) & 0x0F0F0F0Fu;
            // opaque: with the masks' known zero bits the compiler would extract each byte
            // separately instead of converting it in place (v_cvt_f32_ubyte1..3)
            asm volatile("" : "+v"(lo4), "+v"(hi4));
            lo[2 * j] = w2(lo4, 0, d1, m1);
            lo[2 * j + 1] = w2(lo4, 2, d1, m1);
            hi[2 * j] = w2(hi4, 0, d2, m2);
            hi[2 * j + 1] = w2(hi4, 2, d2, m2);
        }
    } else {
        // part 0: ql plane a -> quarters 0 (low nibble, qh bits 0-1) and 2 (high, bits 4-5);
        // part 1: plane b -> quarters 1 (bits 2-3) and 3 (bits 6-7). Scale of quarter q:
        // int8 scales[8s + h + 2q]. Four quants per dword: the nibble and the two high bits
        // are combined byte-parallel into unsigned 6-bit values u, and each weight is
        // (u - 32)·da = u·da + (-32·da) (the bias exact: a power-of-two multiple), one fused
        // multiply-add rounded once to FP16.
        const uint32_t s = (u >> 1) & 1u, h = u & 1u;
        const uint32_t scw[4] = {ws.hd.x, ws.hd.y, ws.hd.z, ws.hd.w};
        const uint32_t ia = 8 * s + h + 2 * part, ib = ia + 4;
        const float d = gh_h2f(ws.d);
        const float da = d * (float)(int8_t)(scw[ia >> 2] >> (8 * (ia & 3u)));
        const float db = d * (float)(int8_t)(scw[ib >> 2] >> (8 * (ib & 3u)));
        const float na = -32.0f * da, nb = -32.0f * db;
        const uint32_t qh[4] = {ws.qh.x, ws.qh.y, ws.qh.z, ws.qh.w};
        // the two high bits of each quant moved to bits 4-5 of its byte in one shift:
        // ((qh >> 2 part) & 3) << 4 = (qh << (4 - 2 part)) & 0x30, ((qh >> (4 + 2 part)) & 3) << 4
        // = (qh >> 2 part) & 0x30 (part is 0 or 1)
        const uint32_t sl = 4 - 2 * part, sh = 2 * part;
        auto w2 = [](uint32_t q4, int e, float sc, float bias) __attribute__((always_inline)) {
            typedef _Float16 hv2 __attribute__((ext_vector_type(2)));
            const float f0 = (float)((q4 >> (8 * e)) & 0xFFu), f1 = (float)((q4 >> (8 * e + 8)) & 0xFFu);
            const hv2 r = {(_Float16)__builtin_fmaf(f0, sc, bias), (_Float16)__builtin_fmaf(f1, sc, bias)};
            return __builtin_bit_cast(uint32_t, r);
        };
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t qa4 = (qw[j] & 0x0F0F0F0Fu) | ((qh[j] << sl) & 0x30303030u);
            const uint32_t qb4 = ((qw[j] >> 4) & 0x0F0F0F0Fu) | ((qh[j] >> sh) & 0x30303030u);
            lo[2 * j] = w2(qa4, 0, da, na);
            lo[2 * j + 1] = w2(qa4, 2, da, na);
            hi[2 * j] = w2(qb4, 0, db, nb);
            hi[2 * j + 1] = w2(qb4, 2, db, nb);
        }
    }
    // low nibbles (quarter 2·part for Q6_K): positions 16·part + i; high: 32 + 16·part + i
    *(uint4*)(dst + 16 * part) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    *(uint4*)(dst + 16 * part + 8) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
    *(uint4*)(dst + 32 + 16 * part) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *(uint4*)(dst + 40 + 16 * part) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
}

// One FP16 output of the GEMM (its FP32 sum `acc`), with the launch's epilogue.
__device__ __forceinline__ void gemm_store(const GhGemmArgs& a, uint64_t i, float acc) {
    uint16_t h = gh_f2h(acc);
    if (a.epi == GH_GEMM_EPI_SILU) h = gh_silu_mul_h(gh_gp<uint16_t>(a.aux)[i], h);
    gh_gpw<uint16_t>(a.out)[i] = h;
}

// The accumulator tiles of one wave to memory. D of tile (i, j), register r: token
// t0 + 32 i + 8 (r / 4) + 4 fg + r % 4, row r0 + 32 j + fm. FP32 partials of split z when the
// launch splits K; otherwise FP16 with the epilogue. The SiLU epilogue (SILU: compiled in; the
// warp-specialized kernels only, whose registers have room) requests a tile column's 16 x TJ
// gate values at once (clamped addresses, no branch around the loads) before using any,
// rather than one round trip per output.
// Partials: element (t, row) of split z at part[z n ps + t ps + pc + row] (ps: the partials'
// row length, pc: this matrix's first column in it).
template <int TI, int TJ, bool SILU>
__device__ __forceinline__ void gemm_write(const GhGemmArgs& a, const f16v (&acc)[TI][TJ], uint32_t t0,
                                           uint32_t r0, uint32_t fm, uint32_t fg, uint32_t z,
                                           uint64_t ps, uint64_t pc) {
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        uint16_t g[16][TJ];
        if (SILU && a.splits == 1 && a.epi == GH_GEMM_EPI_SILU) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    const uint32_t t = min(t0 + 32 * i + 8 * (r >> 2) + 4 * fg + (r & 3), a.n - 1);
                    const uint32_t row = min(r0 + 32 * j + fm, a.rows - 1);
                    g[r][j] = gh_gp<uint16_t>(a.aux)[(uint64_t)t * a.rows + row];
                }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t t = t0 + 32 * i + 8 * (r >> 2) + 4 * fg + (r & 3);
            if (t >= a.n) continue;
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const uint32_t row = r0 + 32 * j + fm;
                if (row >= a.rows) continue;
                const uint64_t o = (uint64_t)t * a.rows + row;
                if (a.splits > 1)
                    gh_gpw<float>(a.part)[((uint64_t)z * a.n + t) * ps + pc + row] = acc[i][j][r];
                else if (SILU && a.epi == GH_GEMM_EPI_SILU)
                    gh_gpw<uint16_t>(a.out)[o] = gh_silu_mul_h(g[r][j], gh_f2h(acc[i][j][r]));
                else
                    gh_gpw<uint16_t>(a.out)[o] = gh_f2h(acc[i][j][r]);
            }
        }
    }
}

// The 96-row pair tiles' output (one split, the host's plan): one wave's 32 tokens from tc;
// tile 0 holds gate rows r0 + fm, tile 1 the up rows of the same lanes, tile 2 gate rows
// r0 + 32 + fm in lanes fm < 16 and the matching up rows 16 lanes up. out = silu_mul(f16(gate),
// f16(up)), as gh_gemm_reduce_swiglu computes it.
__device__ __forceinline__ void pair_write96(const GhGemmArgs& a, const f16v (&acc)[1][3], uint32_t tc, uint32_t r0,
                                             uint32_t fm, uint32_t fg) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float up2 = __shfl_xor(acc[0][2][r], 16);
        const uint32_t t = tc + 8 * (r >> 2) + 4 * fg + (r & 3);
        if (t >= a.n) continue;
        GH_GLOBAL uint16_t* o = gh_gpw<uint16_t>(a.out) + (uint64_t)t * a.rows;
        if (r0 + fm < a.rows) o[r0 + fm] = gh_silu_mul_h(gh_f2h(acc[0][0][r]), gh_f2h(acc[0][1][r]));
        if (fm < 16 && r0 + 32 + fm < a.rows) o[r0 + 32 + fm] = gh_silu_mul_h(gh_f2h(acc[0][2][r]), gh_f2h(up2));
    }
}

// The 128-row pair tiles' output (one split): a wave holding 64 tile rows has gate rows
// row0 + fm in its tile 0 and the up rows of the same lanes in tile 1, for TI token tiles of 32
// from tc. out = silu_mul(f16(gate), f16(up)), as gh_gemm_reduce_swiglu computes it.
template <int TI>
__device__ __forceinline__ void pair_write128(const GhGemmArgs& a, const f16v (&acc)[TI][2], uint32_t tc,
                                              uint32_t row0, uint32_t fm, uint32_t fg) {
    const uint32_t row = row0 + fm;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t t = tc + 32 * i + 8 * (r >> 2) + 4 * fg + (r & 3);
            if (t < a.n && row < a.rows)
                gh_gpw<uint16_t>(a.out)[(uint64_t)t * a.rows + row] =
                    gh_silu_mul_h(gh_f2h(acc[i][0][r]), gh_f2h(acc[i][1][r]));
        }
}

// Warp-specialized variant for long batches: a 512-thread workgroup owns 4·WT tokens x BR rows
// (WT = 64: 256 tokens; WT = 32: 128 tokens, for chunks of fewer than 256 rows, where split K
// has to spread the units over many workgroups). Waves 0-3 (consumers) run the matrix cores
// (WT tokens each, B from LDS). Waves 4-7 (producers) stream the weight bytes a block ahead of
// use (two block register sets, selected statically by unrolling the block loop twice) and
// dequantize each unit into a kS-stage LDS ring one unit ahead of the consumers. One barrier
// per unit: in the interval of unit u the consumers read stage (u - u0) % kS while the
// producers fill unit u + 1 into the stage read during unit u - 2.
// LDS of gemm3_body: kS = 3 weight stages, then each consumer wave's GH_GEMM3_XB(WT) activation
// buffers (one unit each: the unit being read and the units in flight behind it). Three units
// in flight for the 128-token tiles (8B prefill of 128 tokens 6.50 -> 6.45 ms, bit-identical);
// the 256-token tiles keep one (two measured no faster: 512 x 12288 -> 4096 105 -> 108 us).
#define GH_GEMM3_XB(WT) ((WT) == 32 ? 4 : 2)
#define GH_GEMM3_LDS_T(BR, WT) (3 * (BR) * LDK + 4 * GH_GEMM3_XB(WT) * (WT) * 64)

// Tile (bx, by) and split bz of one matrix (a.w, a.rows, a.out); lds3 holds the kernel's LDS
// block (GH_GEMM3_LDS_T / GH_GEMM3_LDS_C8 halves); partials go to columns pc .. of rows ps long.
// NC: consumer waves (4, or 8 with WT = 32: 256 tokens in eight 32-token waves, two per SIMD,
// the four producer waves after them in a 768-thread workgroup; XB: activation buffers per
// consumer wave (GH_GEMM3_XB(WT) by default).
// Wave roles of the consumers. NF waves fetch the tile's activations, WT token rows each (the
// tile is NF·WT tokens); NC waves multiply them, in NC / CR token groups x CR row groups: wave w
// takes TW = NF·WT·CR / NC tokens from (w / CR)·TW against rows (BR / CR)·(w % CR) .. + BR / CR.
//   NC = NF = 4, CR = 1: each consumer multiplies the tokens it fetched against all rows;
//   NC = NF = 8, CR = 1 or 2: 256 tokens in eight 32-token fetches, two consumers per SIMD
//     (CR = 2: 64 tokens x half the rows each);
//   NC = 8, NF = 4, CR = 2: 128 tokens fetched by waves 0-3, consumers of 32 tokens x half the
//     rows, two per SIMD.
// With CR = 2 each weight fragment is read from LDS by half as many waves.
template <uint32_t FMT, int BR, int WT = 64, int NC = 4, int XB = GH_GEMM3_XB(WT), int CR = 1, int NF = NC,
          bool PAIR = false>
__device__ __forceinline__ void gemm3_body(const GhGemmArgs& a, _Float16* lds3, uint32_t bx, uint32_t by,
                                           uint32_t bz, uint64_t ps, uint64_t pc) {
    static_assert(WT == 64 || WT == 32, "fetches of 64 or 32 tokens");
    static_assert((NC == 4 || NC == 8) && (NF == 4 || NF == 8) && NF <= NC, "four or eight consumers");
    static_assert(CR == 1 || (CR == 2 && BR % 64 == 0), "row halves of 64-row multiples");
    constexpr int TW = NF * WT * CR / NC;  // tokens per consumer wave
    static_assert(TW % 32 == 0 && TW * NC == NF * WT * CR, "whole 32-token tiles per consumer");
    // per consumer wave: TI x TJ tiles of 32 x 32; NX: activation line loads per unit
    constexpr int TI = TW / 32, TJ = BR / (32 * CR), NX = WT / 8;
    constexpr int kS = 3;
    auto wstage = [&](uint32_t st) __attribute__((always_inline)) { return lds3 + st * (BR * LDK); };
    static_assert(!PAIR || (BR == 96 && NC == NF && WT == 32 && CR == 1) || (BR == 128 && NC == 8 && CR == 2),
                  "pair tiles: 96 rows (consumers of 32 tokens x 96 rows) or 128 rows (eight consumers of 64 rows)");
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t r0 = bx * (PAIR ? BR / 2 : BR);
    const uint32_t units = a.in_dim / 64;
    const uint32_t per = gh_gemm_split_units(units, a.splits);
    const uint32_t u0 = bz * per, u1 = min(units, u0 + per);
    if (u0 >= u1) return;  // workgroup-uniform; the host sizes splits so that none is empty
    auto uc = [&](uint32_t u) __attribute__((always_inline)) { return min(u, u1 - 1); };

    if (wave >= (uint32_t)NC) {
        // ---- producers ----
        // Raw weight bytes a block (4 units) at a time, two blocks in registers: block i + 2 is
        // requested once block i has been dequantized, so each block has the 4 units of block
        // i + 1 to arrive (splits start and end on block boundaries, gh_gemm_split_units).
        // Unit u0 + k goes into stage k % kS one unit ahead of the consumers: every store is
        // followed by a barrier (the first is the consumers' start), and one more closes the
        // consumers' last interval (1 + n_units barriers, as the consumers meet).
        const uint32_t pt = threadIdx.x - 64 * NC;
        const bool wload = pt < 2 * BR;
        const uint32_t b0 = u0 / 4, nblk = (u1 - u0) / 4;
        auto bc = [&](uint32_t i) __attribute__((always_inline)) { return b0 + min(i, nblk - 1); };
        WBlock<FMT> wb[2];
        load_wblock<FMT, BR, PAIR>(a, r0, bc(0), wb[0], pt);
        load_wblock<FMT, BR, PAIR>(a, r0, bc(1), wb[1], pt);
        auto block = [&](uint32_t i, WBlock<FMT>& w) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t k = 4 * i + j;
                if (wload)
                    store_w<FMT, BR>(u0 + k, WStage{w.q[j], w.hd, w.qh[FMT == kQ6K ? j : 0], w.d}, wstage(k % kS),
                                     pt);
                __syncthreads();
            }
            // the reload stays after the block's last use of w (hoisted above it, the
            // compiler gives w two registers sets and copies between them at the loop's back
            // edge, which waits for the loads just issued)
            __builtin_amdgcn_sched_barrier(0);
            load_wblock<FMT, BR, PAIR>(a, r0, bc(i + 2), w, pt);
            __builtin_amdgcn_sched_barrier(0);
        };
        uint32_t i = 0;
        for (; i + 2 <= nblk; i += 2) {  // no exits inside the unrolled body
            block(i, wb[0]);
            block(i + 1, wb[1]);
        }
        if (i < nblk) block(i, wb[0]);
        __syncthreads();
        return;
    }

    // ---- consumers ----
    // Activations are fetched as whole lines straight into the wave's own LDS rows (only this
    // wave touches them), kXA units ahead of the unit being read, from which the A fragments are
    // read — each 128-byte line is requested once instead of once per 16-k step, and no
    // registers hold it on the way. The loads are issued from inline assembly so that the
    // compiler does not count them: with the builtin, the workgroup fence of every per-unit
    // barrier waited for all of them (vmcnt(0)), so each unit waited out a full L2 round trip
    // for the next one. Here each unit waits only until the next unit's lines have landed
    // (loads complete in issue order; the consumers issue no other memory operations in the
    // loop), so kXA units stay in flight.
    constexpr int kXB = XB, kXA = kXB - 1;
    const bool fetcher = wave < (uint32_t)NF;
    const uint32_t t0 = by * (NF * WT) + wave * WT;  // the tokens this wave fetches
    // the tokens and rows it multiplies: tile i's 32 token rows are rows xr_i .. + 32 of fetch
    // wave xf_i's buffers
    const uint32_t tb = (wave / CR) * TW, tc = by * (NF * WT) + tb, rc = (wave % CR) * (BR / CR);
    const uint32_t fm = lane & 31u, fg = lane >> 5;
    const GH_GLOBAL uint16_t* x = gh_gp<uint16_t>(a.x);
    uint64_t xg[NX];
#pragma unroll
    for (int i = 0; i < NX; ++i)
        xg[i] = (uint64_t)(uintptr_t)(x + (uint64_t)min(t0 + 8 * i + (lane >> 3), a.n - 1) * a.in_dim);
    // global_load_lds_dwordx4: lane l of a load lands at byte 16 l of its 1 KiB destination. Load
    // i covers rows 8 i .. 8 i + 7 of the wave's WT; lane l fetches chunk (l % 8) ^ sw(r) of row
    // r = 8 i + l / 8, so chunk c of row r sits at slot c ^ sw(r). Every row starts at bank 0
    // (128-byte pitch); with sw(r) = (r / 2) % 8 a fragment read (rows fm = 0..31 of one chunk)
    // is free of bank conflicts, as measured with SQ_LDS_BANK_CONFLICT on gfx950 (sw(r) =
    // (r / 4) % 8 and r % 8 are two-way conflicted: 7.3 against 3.8 LDS-active cycles per read).
    _Float16* xw = lds3 + kS * BR * LDK + wave * (kXB * WT * 64);
    const _Float16* xs = lds3 + kS * BR * LDK;
    uint32_t xoff[TI], xrow[TI];  // tile i: offset of its fetch wave's buffers, first row
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        xoff[i] = ((tb + 32 * i) / WT) * (kXB * WT * 64);
        xrow[i] = (tb + 32 * i) % WT;
    }
    auto load_rows = [&](uint32_t u, uint32_t b) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const uint32_t r = 8 * i + (lane >> 3), c = (lane & 7u) ^ ((r >> 1) & 7u);
            const uint32_t dst = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(
                xw + b * (WT * 64) + i * 512);
            asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(xg[i] + 2ull * chunk_k<FMT>(u, c)),
                         "{m0}"(__builtin_amdgcn_readfirstlane(dst))
                         : "memory");
        }
    };
    f16v acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f16v{};
#pragma unroll
    for (int i = 0; i < kXA; ++i)
        if (NF == NC || fetcher) load_rows(uc(u0 + i), i);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NX * (kXA - 1)) : "memory");  // unit u0 has landed
    __syncthreads();
    // unit u is read from buffer b = (u - u0) % kXB; unit u + kXA goes into buffer (b + kXA) %
    // kXB, the one read during unit u - 1 (those reads ended before its barrier)
    auto step = [&](uint32_t u, uint32_t b) __attribute__((always_inline)) {
        if (NF == NC || fetcher) load_rows(uc(u + kXA), (b + kXA) % kXB);
        __builtin_amdgcn_sched_barrier(0);  // the loads go out before anything waits
        const _Float16* wb = wstage((u - u0) % kS) + rc * LDK;
        const _Float16* xb = xs + b * (WT * 64);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            h8 af[TI], bf[TJ];
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const uint32_t r = xrow[i] + fm, c = (2 * ks + fg) ^ ((r >> 1) & 7u);
                af[i] = *(const h8*)(xb + xoff[i] + r * 64 + c * 8);
            }
#pragma unroll
            for (int j = 0; j < TJ; ++j) bf[j] = *(const h8*)(wb + (32 * j + fm) * LDK + 16 * ks + 8 * fg);
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NX * (kXA - 1)) : "memory");  // unit u + 1 has landed
        __syncthreads();
    };
    // the unrolled body has no exits and compile-time buffer indices; tail after
    uint32_t u = u0;
    for (; u + kXB <= u1; u += kXB) {
#pragma unroll
        for (int b = 0; b < kXB; ++b) step(u + b, b);
    }
#pragma unroll
    for (int b = 0; b < kXB - 1; ++b)
        if (u + b < u1) step(u + b, b);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped loads past u1 have landed
    if constexpr (PAIR && BR == 128) {
        pair_write128(a, acc, tc, r0 + (rc / 64) * 32, fm, fg);
    } else if constexpr (PAIR) {
        pair_write96(a, acc, tc, r0, fm, fg);
    } else {
        gemm_write<TI, TJ, true>(a, acc, tc, r0 + rc, fm, fg, bz, ps, pc);
    }
}

}  // namespace

// Warp-specialized 256-token tiles: eight 32-token consumer waves (two per SIMD, so one wave's
// fragment reads and waits overlap the other's matrix work) and four producer waves, 768
// threads, one unit of activation lookahead; 128-row tiles with the consumers tiled 4 x 2
// (64 tokens x 64 rows each), 96-row tiles 8 x 1. Against four 64-token consumers (512 threads),
// same box, bit-identical: 512 x 4096 -> 12288 (96 rows) 76.7 -> 71.8 us, 512 x 12288 -> 4096
// (128 rows, 4 splits) 80.2 -> 73.6, 2048 x 4096 -> 4096 105.4 -> 92.7 (4 x 2 tiles; 101.3 as
// 8 x 1), 2048 x 4096 -> 12288 291.6 -> 207.8 (128 rows 4 x 2, where the 96-row tiles take
// 233.9).
#define GH_GEMM3_LDS_C8(BR) (3 * (BR) * LDK + 8 * 2 * 32 * 64)
#define GH_GEMM3(NAME, FMT, BR)                                                                    \
    GH_KERNEL __launch_bounds__(768) void NAME(GhGemmArgs a) {                                     \
        __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM3_LDS_C8(BR)];                \
        gemm3_body<FMT, BR, 32, 8, 2, (BR) == 128 ? 2 : 1>(a, lds, blockIdx.x, blockIdx.y, blockIdx.z, a.rows, 0); \
    }
GH_GEMM3(gh_gemm3_q4k_r128, kQ4K, 128)
GH_GEMM3(gh_gemm3_q6k_r128, kQ6K, 128)
GH_GEMM3(gh_gemm3_q4k_r96, kQ4K, 96)
GH_GEMM3(gh_gemm3_q6k_r96, kQ6K, 96)
// SwiGLU's gate (a.w) and up (a.aux) Q4_K projections in one launch of 256-token tiles, each
// 96-row tile 48 gate rows and the same 48 up rows (pair_row), K unsplit, silu_mul in the
// epilogue (pair_write96): the gate's FP16 output is neither written nor read back
GH_KERNEL __launch_bounds__(768) void gh_gemm3_swiglu_r96(GhGemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM3_LDS_C8(96)];
    gemm3_body<kQ4K, 96, 32, 8, 2, 1, 8, true>(a, lds, blockIdx.x, blockIdx.y, blockIdx.z, a.rows, 0);
}
// the same over 128-row tiles of 64 gate + 64 up rows (pair_row<128>; eight consumers of 64
// tokens x 64 rows), where the separate launches take 128-row tiles
GH_KERNEL __launch_bounds__(768) void gh_gemm3_swiglu_r128(GhGemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM3_LDS_C8(128)];
    gemm3_body<kQ4K, 128, 32, 8, 2, 2, 8, true>(a, lds, blockIdx.x, blockIdx.y, blockIdx.z, a.rows, 0);
}
// 128-token tiles (consumer waves of 32 tokens)
#define GH_GEMM3T(NAME, FMT, BR)                                                                   \
    GH_KERNEL __launch_bounds__(512) void NAME(GhGemmArgs a) {                                     \
        __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM3_LDS_T(BR, 32)];             \
        gemm3_body<FMT, BR, 32>(a, lds, blockIdx.x, blockIdx.y, blockIdx.z, a.rows, 0);            \
    }
GH_GEMM3T(gh_gemm3_q4k_r96_t128, kQ4K, 96)
GH_GEMM3T(gh_gemm3_q6k_r96_t128, kQ6K, 96)
// SwiGLU's gate (a.w) and up (a.aux) Q4_K projections of one input in one launch, for batches
// of at most 128 tokens: each 96-row tile holds 48 gate rows and the same 48 up rows (PAIR in
// load_wblock), K unsplit, and writes silu_mul(f16(x wg^T), f16(x wu^T)) straight to a.out
// [n][rows] — no FP32 partials and no split reduce. Each output's sum runs over every unit in
// k order, the sum of the unsplit gh_gemm3_q4k_*_t128 kernels.
GH_KERNEL __launch_bounds__(512) void gh_gemm3_swiglu_r96_t128(GhGemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM3_LDS_T(96, 32)];
    gemm3_body<kQ4K, 96, 32, 4, GH_GEMM3_XB(32), 1, 4, true>(a, lds, blockIdx.x, blockIdx.y, blockIdx.z, a.rows, 0);
}
// the same over 128-row tiles of 64 gate + 64 up rows, eight consumers (outputs whose 48-row
// pairs would overfill one wave of workgroups: 14B 16384 rows, 256 tiles of 64)
GH_KERNEL __launch_bounds__(768) void gh_gemm3_swiglu_r128_t128(GhGemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM3_LDS_T(128, 32)];
    gemm3_body<kQ4K, 128, 32, 8, GH_GEMM3_XB(32), 2, 4, true>(a, lds, blockIdx.x, blockIdx.y, blockIdx.z, a.rows, 0);
}
// 128-token tiles of 128 rows: the activations fetched by four waves, eight consumers of 32
// tokens x 64 rows (two per SIMD), four producers, 768 threads. Against four consumers of 32
// tokens x 128 rows, same box, bit-identical: 128 x 12288 -> 4096 (8 splits) 35.8 -> 33.9 us,
// 128 x 4096 -> 4096 (4 splits) 17.2 (96-row tiles) -> 16.2, 128 x 5120 -> 16384 39.0 -> 37.1.
#define GH_GEMM3T8(NAME, FMT, BR)                                                                  \
    GH_KERNEL __launch_bounds__(768) void NAME(GhGemmArgs a) {                                     \
        __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM3_LDS_T(BR, 32)];             \
        gemm3_body<FMT, BR, 32, 8, GH_GEMM3_XB(32), 2, 4>(a, lds, blockIdx.x, blockIdx.y, blockIdx.z, a.rows, 0); \
    }
GH_GEMM3T8(gh_gemm3_q4k_r128_t128, kQ4K, 128)
GH_GEMM3T8(gh_gemm3_q6k_r128_t128, kQ6K, 128)

// Over FP16 weight copies, every wave of the workgroup runs the matrix cores: 512 threads own
// 256 tokens x BR rows, two waves per SIMD, so that one wave's LDS reads and waits overlap the
// other's matrix work. BR = 128: wave w takes the 64 tokens of group w / 2 against rows
// 64 (w % 2) .. + 64 (2 x 2 tiles of v_mfma_f32_32x32x16_f16); BR = 96: the 32 tokens of
// group w against all 96 rows (1 x 3 tiles), which makes 256 workgroups of a 12288-row output
// at 512 tokens instead of 192. Each unit's activation lines and weight rows go into a
// 3-stage LDS ring by LDS DMA that every wave shares in (activation rows 32 w .. + 32 and
// weight row blocks w, w + 8 of 8 rows, 1 KiB loads from inline assembly; both operands in
// 128-byte rows with chunk c of row r at slot c ^ (r / 2) % 8). Each wave holds one unit's
// fragments in registers and reads the next unit's into a second set while the matrix cores
// work on the first, so no k-step waits on an LDS read. After the barrier of iteration u
// (unit u + 1 landed, every wave's reads of unit u done) unit u + 3 goes into unit u's stage.
// The k order of every output's sum is the one gemm3_body uses: the same bits.
#define GH_GEMM4_LDS(BR) (3 * (256 + (BR)) * 64)
template <uint32_t FMT, int BR, bool PAIR = false>
__device__ __forceinline__ void gemm4_body(const GhGemmArgs& a, _Float16* lds, uint32_t bx, uint32_t by,
                                           uint32_t bz, uint64_t ps, uint64_t pc) {
    static_assert(BR == 128 || BR == 96, "all-waves-MFMA tiles: 128 or 96 rows");

    constexpr uint32_t WTOK = BR == 128 ? 64 : 32, WROW = BR == 128 ? 64 : 96;
    constexpr uint32_t NR = BR / WROW, TI = WTOK / 32, TJ = WROW / 32, NB = BR / 8;
    constexpr uint32_t kStage = (256 + BR) * 64;  // halves: A (256 token rows), then B (BR rows)
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, g = wave / NR, hr = wave % NR;
    const uint32_t r0 = bx * (PAIR ? BR / 2 : BR);
    const uint32_t units = a.in_dim / 64;
    const uint32_t per = gh_gemm_split_units(units, a.splits);
    const uint32_t u0 = bz * per, u1 = min(units, u0 + per);
    if (u0 >= u1) return;  // workgroup-uniform; the host sizes splits so that none is empty
    auto uc = [&](uint32_t u) __attribute__((always_inline)) { return min(u, u1 - 1); };
    const uint32_t fm = lane & 31u, fg = lane >> 5;
    // this wave's loads: activation rows 32 w + 8 i + lane / 8 (i < 4), weight rows
    // 8 d + lane / 8 of blocks d = w, w + 8 (< NB); lane l fetches chunk (l % 8) ^ sw(row)
    const GH_GLOBAL uint16_t* x = gh_gp<uint16_t>(a.x);
    constexpr uint32_t kB = (NB + 7) / 8;  // weight blocks of wave 0 (waves >= NB - 8 have one fewer)
    const bool two = NB >= 16 || wave + 8 < NB;  // compile-time true for 128 rows
    uint64_t xa[4], wa[kB];
    uint32_t xc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = 32 * wave + 8 * i + (lane >> 3);
        xc[i] = (lane & 7u) ^ ((r >> 1) & 7u);
        xa[i] = (uint64_t)(uintptr_t)(x + (uint64_t)min(by * 256 + r, a.n - 1) * a.in_dim);
    }
#pragma unroll
    for (uint32_t i = 0; i < kB; ++i) {
        const uint32_t r = 8 * (wave + 8 * i) + (lane >> 3), c = (lane & 7u) ^ ((r >> 1) & 7u);
        uint64_t wbase = a.w;
        const uint32_t wr = PAIR ? pair_row<BR>(min(r, (uint32_t)BR - 1), wbase, a) : r;
        wa[i] = wbase + ((uint64_t)min(r0 + wr, a.rows - 1) * units) * 128 + c * 16;
    }
    auto stage = [&](uint32_t st) __attribute__((always_inline)) { return lds + st * kStage; };
    auto issue = [&](uint32_t u, uint32_t st) __attribute__((always_inline)) {
        _Float16* sa = stage(st);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t dst =
                (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(sa + (32 * wave + 8 * i) * 64);
            asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(xa[i] + 2ull * chunk_k<FMT>(u, xc[i])),
                         "{m0}"(__builtin_amdgcn_readfirstlane(dst))
                         : "memory");
        }
#pragma unroll
        for (uint32_t i = 0; i < kB; ++i) {
            if (i == 1 && !two) break;  // wave-uniform
            const uint32_t dst = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(
                sa + (256 + 8 * (wave + 8 * i)) * 64);
            asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(wa[i] + (uint64_t)u * 128),
                         "{m0}"(__builtin_amdgcn_readfirstlane(dst))
                         : "memory");
        }
    };
    f16v acc[TI][TJ];
#pragma unroll
    for (uint32_t i = 0; i < TI; ++i)
#pragma unroll
        for (uint32_t j = 0; j < TJ; ++j) acc[i][j] = f16v{};
    // one unit's fragments: 4 k-steps x (TI activation + TJ weight) 8-half lane slices
    struct Frags {
        h8 a[4][TI], b[4][TJ];
    };
    auto read = [&](uint32_t st, Frags& f) __attribute__((always_inline)) {
        const _Float16* xb = stage(st) + (WTOK * g) * 64;
        const _Float16* wb = stage(st) + 256 * 64;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
            for (uint32_t i = 0; i < TI; ++i) {
                const uint32_t r = 32 * i + fm, c = (2 * ks + fg) ^ ((r >> 1) & 7u);
                f.a[ks][i] = *(const h8*)(xb + r * 64 + c * 8);
            }
#pragma unroll
            for (uint32_t j = 0; j < TJ; ++j) {
                const uint32_t r = WROW * hr + 32 * j + fm, c = (2 * ks + fg) ^ ((r >> 1) & 7u);
                f.b[ks][j] = *(const h8*)(wb + r * 64 + c * 8);
            }
        }
    };
    auto mma = [&](const Frags& f) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (uint32_t i = 0; i < TI; ++i)
#pragma unroll
                for (uint32_t j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[ks][i], f.b[ks][j], acc[i][j], 0, 0, 0);
    };
    // all but this wave's last n issues have landed
    auto wait_but = [&](int n) __attribute__((always_inline)) {
        if (kB == 1 || two) {
            if (n == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * (4 + kB)) : "memory");
            else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 + kB) : "memory");
        } else {
            if (n == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * (4 + kB - 1)) : "memory");
            else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 + kB - 1) : "memory");
        }
    };
    // iteration k (unit u): unit u + 1 has landed -> barrier (every wave's reads of unit u are
    // done, so its stage k % 3 takes unit u + 3) -> the next unit's fragments are read while
    // this unit's matrix work runs from registers
    auto step = [&](uint32_t u, Frags& cur, Frags& nxt) __attribute__((always_inline)) {
        const uint32_t k = u - u0;
        wait_but(1);
        __syncthreads();
        issue(uc(u + 3), k % 3);
        read((k + 1) % 3, nxt);
        mma(cur);
        // one fragment read between consecutive matrix instructions
#pragma unroll
        for (uint32_t q = 0; q < 4 * (TI + TJ); ++q) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        }
    };
    issue(u0, 0);
    issue(uc(u0 + 1), 1);
    issue(uc(u0 + 2), 2);
    wait_but(2);
    __syncthreads();
    Frags f0, f1;
    read(0, f0);
    uint32_t u = u0;
    for (; u + 1 < u1; u += 2) {
        step(u, f0, f1);
        step(u + 1, f1, f0);
    }
    if (u < u1) step(u, f0, f1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last (unused) loads have landed
    if constexpr (PAIR && BR == 128)
        pair_write128(a, acc, by * 256 + WTOK * g, r0 + 32 * hr, fm, fg);
    else if constexpr (PAIR)
        pair_write96(a, acc, by * 256 + WTOK * g, r0, fm, fg);
    else
        gemm_write<TI, TJ, true>(a, acc, by * 256 + WTOK * g, r0 + WROW * hr, fm, fg, bz, ps, pc);
}
#define GH_GEMM4W(NAME, FMT, BR)                                                                   \
    GH_KERNEL __launch_bounds__(512) void NAME(GhGemmArgs a) {                                     \
        __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM4_LDS(BR)];                   \
        gemm4_body<FMT, BR>(a, lds, blockIdx.x, blockIdx.y, blockIdx.z, a.rows, 0);                \
    }
GH_GEMM4W(gh_gemm4w_q4k_r128, kQ4K, 128)
GH_GEMM4W(gh_gemm4w_q6k_r128, kQ6K, 128)
GH_GEMM4W(gh_gemm4w_q4k_r96, kQ4K, 96)
GH_GEMM4W(gh_gemm4w_q6k_r96, kQ6K, 96)
// gh_gemm3_swiglu_r96 over the FP16 copies of gate (a.w) and up (a.aux): the same pair tiles,
// the same k order
GH_KERNEL __launch_bounds__(512) void gh_gemm4w_swiglu_r96(GhGemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM4_LDS(96)];
    gemm4_body<kQ4K, 96, true>(a, lds, blockIdx.x, blockIdx.y, blockIdx.z, a.rows, 0);
}
GH_KERNEL __launch_bounds__(512) void gh_gemm4w_swiglu_r128(GhGemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM4_LDS(128)];
    gemm4_body<kQ4K, 128, true>(a, lds, blockIdx.x, blockIdx.y, blockIdx.z, a.rows, 0);
}

// A Q4_K / Q6_K matrix [rows][in_dim] dequantized to FP16 in the GEMM's unit order, the layout
// gemm4_body reads: thread t handles half p = t % 2 of unit u of row r, t / 2 = r · units + u,
// with load_w and store_w (one row per "tile"), so each value is the one the dequantizing
// producers stage. a.w: device layout, a.out: FP16 [rows][units][64].
template <uint32_t FMT>
__device__ __forceinline__ void dequant_f16(const GhGemmArgs& a) {
    const uint32_t units = a.in_dim / 64;
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x, ru = t >> 1;
    if (ru >= (uint64_t)a.rows * units) return;
    const uint32_t p = (uint32_t)(t & 1u), r = (uint32_t)(ru / units), u = (uint32_t)(ru % units);
    WStage ws;
    load_w<FMT, 1>(a, r, u, ws, p);
    store_w<FMT, 1>(u, ws, (_Float16*)(uintptr_t)a.out + ru * 64, p);
}
GH_KERNEL __launch_bounds__(256) void gh_dequant_f16_q4k(GhGemmArgs a) { dequant_f16<kQ4K>(a); }
GH_KERNEL __launch_bounds__(256) void gh_dequant_f16_q6k(GhGemmArgs a) { dequant_f16<kQ6K>(a); }

// Several matrices of one input in one launch (the prefill's Q, K and V projections): row tile
// blockIdx.x belongs to the matrix whose tiles start at or below it, and runs that matrix's
// format (Q4_K or Q6_K) over the shared LDS block; a.rows is the total row count, the
// partials' row length.
template <int WT>
__device__ __forceinline__ void gemm3_mixed(const GhGemmArgs& a, _Float16* lds) {
    uint32_t s = 0;
    for (uint32_t i = 1; i < a.nseg; ++i)
        if (blockIdx.x >= a.seg[i].tile0) s = i;
    GhGemmArgs m = a;
    m.w = a.seg[s].w;
    m.rows = a.seg[s].rows;
    m.out = a.seg[s].out;
    const uint32_t bx = blockIdx.x - a.seg[s].tile0;
    // the 768-thread forms: 256-token tiles (WT = 64) in eight 32-token fetches, 128-token tiles
    // (WT = 32) in four; eight consumers of half the rows each
    constexpr int XB = WT == 64 ? 2 : GH_GEMM3_XB(32), NF = WT == 64 ? 8 : 4;
    if (a.seg[s].fmt == kQ4K)
        gemm3_body<kQ4K, 128, 32, 8, XB, 2, NF>(m, lds, bx, blockIdx.y, blockIdx.z, a.rows, a.seg[s].col0);
    else
        gemm3_body<kQ6K, 128, 32, 8, XB, 2, NF>(m, lds, bx, blockIdx.y, blockIdx.z, a.rows, a.seg[s].col0);
}
GH_KERNEL __launch_bounds__(768) void gh_gemm3_mixed_r128(GhGemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM3_LDS_C8(128)];
    gemm3_mixed<64>(a, lds);
}
// 128-token tiles, for batches of fewer than 256 tokens
GH_KERNEL __launch_bounds__(768) void gh_gemm3_mixed_r128_t128(GhGemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM3_LDS_T(128, 32)];
    gemm3_mixed<32>(a, lds);
}

// The multi-matrix launch over FP16 weights with every wave on the matrix cores (gemm4_body).
GH_KERNEL __launch_bounds__(512) void gh_gemm4w_mixed_r128(GhGemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[GH_GEMM4_LDS(128)];
    uint32_t s = 0;
    for (uint32_t i = 1; i < a.nseg; ++i)
        if (blockIdx.x >= a.seg[i].tile0) s = i;
    GhGemmArgs m = a;
    m.w = a.seg[s].w;
    m.rows = a.seg[s].rows;
    m.out = a.seg[s].out;
    const uint32_t bx = blockIdx.x - a.seg[s].tile0;
    if (a.seg[s].fmt == kQ4K)
        gemm4_body<kQ4K, 128>(m, lds, bx, blockIdx.y, blockIdx.z, a.rows, a.seg[s].col0);
    else
        gemm4_body<kQ6K, 128>(m, lds, bx, blockIdx.y, blockIdx.z, a.rows, a.seg[s].col0);
}

// Sum split-K partials in split order, round to FP16: out[i] = f16(Σ_s part[s][i]).
GH_KERNEL __launch_bounds__(256) void gh_gemm_reduce(GhGemmArgs a) {
    const uint64_t total = (uint64_t)a.n * a.rows;
    // launched with min(ceil(total / 256), 4096) workgroups of 256
    const uint64_t groups = min((total + 255) / 256, (uint64_t)4096);
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += groups * 256) {
        float s = 0.0f;
        for (uint32_t k = 0; k < a.splits; ++k) s += gh_gp<float>(a.part)[k * total + i];
        gemm_store(a, i, s);
    }
}

// SwiGLU's gate and up GEMMs reduced together: partials [2][splits][n][rows] (the gate's, then
// the up projection's), each sum taken in split order and rounded to FP16 as gh_gemm_reduce
// rounds it, then out = silu_mul(gate, up) (gh_silu_mul_h, elementwise/activation.rs:16-29):
// the bits of gh_gemm_reduce on the gate followed by the up reduce with the SiLU epilogue.
// Four adjacent outputs per thread (rows is a multiple of 4).
GH_KERNEL __launch_bounds__(256) void gh_gemm_reduce_swiglu(GhGemmArgs a) {
    const uint64_t nq = (uint64_t)a.n * a.rows / 4;
    // launched with min(ceil(nq / 256), 4096) workgroups of 256
    const uint64_t groups = min((nq + 255) / 256, (uint64_t)4096);
    const GH_GLOBAL float4* p = gh_gp<float4>(a.part);
    for (uint64_t q = (uint64_t)blockIdx.x * 256 + threadIdx.x; q < nq; q += groups * 256) {
        float4 g = make_float4(0.0f, 0.0f, 0.0f, 0.0f), u = g;
        for (uint32_t z = 0; z < a.splits; ++z) {
            const float4 pg = p[z * nq + q], pu = p[(a.splits + z) * nq + q];
            g.x += pg.x;
            g.y += pg.y;
            g.z += pg.z;
            g.w += pg.w;
            u.x += pu.x;
            u.y += pu.y;
            u.z += pu.z;
            u.w += pu.w;
        }
        const uint32_t o0 = gh_silu_mul_h(gh_f2h(g.x), gh_f2h(u.x)) | ((uint32_t)gh_silu_mul_h(gh_f2h(g.y), gh_f2h(u.y)) << 16);
        const uint32_t o1 = gh_silu_mul_h(gh_f2h(g.z), gh_f2h(u.z)) | ((uint32_t)gh_silu_mul_h(gh_f2h(g.w), gh_f2h(u.w)) << 16);
        gh_gpw<uint2>(a.out)[q] = make_uint2(o0, o1);
    }
}

// Split-K sum of a multi-matrix launch (partials [splits][n][Σ rows]): one thread per adjacent
// column pair, summed in split order and rounded to FP16 as gh_gemm_reduce does, then, for a
// matrix with a RoPE role, rotated and post-scaled exactly as gh_rope does (rope_yarn,
// rope.rs:14-39; pairs at or past rope_dim / 2 stored unrotated, the post-scale on the query
// role only); written to the matrix's own output [n][rows]. Token t sits at position base + t.
GH_KERNEL __launch_bounds__(256) void gh_gemm_reduce_seg(GhGemmArgs a) {
#pragma clang fp contract(off)
    const uint64_t total = (uint64_t)a.n * a.rows, npairs = total / 2;
    const uint64_t groups = min((npairs + 255) / 256, (uint64_t)4096);
    for (uint64_t k = (uint64_t)blockIdx.x * 256 + threadIdx.x; k < npairs; k += groups * 256) {
        const uint64_t i = 2 * k;
        float s0 = 0.0f, s1 = 0.0f;
        for (uint32_t z = 0; z < a.splits; ++z) {
            const float2 p = gh_gp<float2>(a.part)[(z * total + i) / 2];
            s0 += p.x;
            s1 += p.y;
        }
        const uint32_t t = (uint32_t)(i / a.rows), col = (uint32_t)(i % a.rows);
        uint32_t sg = 0;
        for (uint32_t j = 1; j < a.nseg; ++j)
            if (col >= a.seg[j].col0) sg = j;
        const GhGemmSeg g = a.seg[sg];
        const uint32_t c = col - g.col0;
        uint32_t h0 = gh_f2h(s0), h1 = gh_f2h(s1);
        const uint32_t pair = (c % a.head_dim) / 2;
        if (g.role && pair < a.pairs) {
            const uint32_t pos = a.base + t;
            const float2 cs = gh_gp<float2>(a.table)[(uint64_t)pos * a.pairs + pair];
            const float scale = g.role == GH_GEMM_ROLE_ROPE_QUERY ? gh_gp<float>(a.post)[pos] : 1.0f;
            const float x0 = gh_h2f(h0), x1 = gh_h2f(h1);
            h0 = gh_f2h((x0 * cs.x - x1 * cs.y) * scale);
            h1 = gh_f2h((x0 * cs.y + x1 * cs.x) * scale);
        }
        gh_gpw<uint32_t>(g.out)[((uint64_t)t * g.rows + c) / 2] = h0 | (h1 << 16);
    }
}

// The GEMM's output row t folded into the residual stream, one 1024-thread workgroup per row:
// h = f16(Σ_s part[s][t][c]) in split order (gh_gemm_reduce; with one split the GEMM's FP16
// output), x[t][c] += f32(h) (residual_add, residual.rs:12-22), and with a norm weight the
// row's RMSNorm f16(x · inverse · f16 w) into `normed` — gh_rmsnorm_x's arithmetic, its Σx²
// in gh_rms_inverse_256's order (threads t < 256: the 16-value items t, t + 256 of the row,
// then the four waves' sums in order) — so the three ops' bits in one pass. rows (the row
// width) is a multiple of 16 and at most 8192. The elementwise passes run on all 1024 threads
// (16 waves of loads in flight per row: with 256 threads, 128-token chunks held 6.9 us for
// about 10 MB of partials).
GH_KERNEL __launch_bounds__(1024) void gh_gemm_tail(GhGemmArgs a) {
#pragma clang fp contract(off)
    const uint32_t t = blockIdx.x, d = a.rows, n4 = d >> 2, tid = threadIdx.x;
    const uint64_t total = (uint64_t)a.n * d, row0 = (uint64_t)t * d;
    GH_GLOBAL float4* x = gh_gpw<float4>(a.aux) + row0 / 4;
    __shared__ float red[4];
    __shared__ float4 ys[2048];  // the updated residual row (rows <= 8192)
    // Pass 1, coalesced: thread t takes float4 j0 + t (a wave's loads cover whole lines), 1024
    // per round. Every load of a round and a group of four splits is requested before any is
    // summed (clamped indices, no branch around the loads); the splits are summed in order, the
    // sum rounded to FP16, added into the residual, and the new row kept in LDS.
    for (uint32_t j0 = 0; j0 < n4; j0 += 1024) {  // launch-uniform: one round up to 4096 rows
        const uint32_t c = min(j0 + tid, n4 - 1);
        float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float4 xv = x[c];
        if (a.splits > 1) {
            for (uint32_t k0 = 0; k0 < a.splits; k0 += 4) {
                float4 p[4];
#pragma unroll
                for (uint32_t kk = 0; kk < 4; ++kk)
                    p[kk] = gh_gp<float4>(a.part)[(min(k0 + kk, a.splits - 1) * total + row0) / 4 + c];
#pragma unroll
                for (uint32_t kk = 0; kk < 4; ++kk)
                    if (k0 + kk < a.splits) {
                        s.x += p[kk].x;
                        s.y += p[kk].y;
                        s.z += p[kk].z;
                        s.w += p[kk].w;
                    }
            }
        } else {
            const uint2 o = gh_gp<uint2>(a.out)[row0 / 4 + c];
            s = make_float4(gh_h2f(o.x & 0xFFFFu), gh_h2f(o.x >> 16), gh_h2f(o.y & 0xFFFFu), gh_h2f(o.y >> 16));
        }
        if (j0 + tid < n4) {
            // one split: s already holds the FP16 output; several: round their sum to FP16
            const float4 h = a.splits > 1 ? make_float4(gh_h2f(gh_f2h(s.x)), gh_h2f(gh_f2h(s.y)),
                                                        gh_h2f(gh_f2h(s.z)), gh_h2f(gh_f2h(s.w)))
                                          : s;
            float4 y = xv;
            y.x = y.x + h.x;
            y.y = y.y + h.y;
            y.z = y.z + h.z;
            y.w = y.w + h.w;
            x[c] = y;
            ys[c] = y;
        }
    }
    if (!a.norm) return;  // launch-uniform
    __syncthreads();
    // Pass 2: threads t < 256 take the 16-value items t, t + 256 of the row back from LDS, in
    // gh_rms_inverse_256's order, for the sum of squares (gh_rms_finish_256's reduction, its
    // four waves' sums in order); every thread then normalizes float4s tid + 1024 k.
    float ss = 0.0f;
    if (tid < 256) {
#pragma unroll
        for (uint32_t it = 0; it < 2; ++it)
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) {
                const uint32_t c = 4 * (tid + 256 * it) + q;
                if (c < n4) ss = gh_rms_add(ss, ys[c]);
            }
    }
    ss = gh_wave_sum63(ss);
    if (tid < 256 && (tid & 63) == 63) red[tid >> 6] = ss;
    __syncthreads();
    const float inverse = 1.0f / __builtin_sqrtf((((red[0] + red[1]) + red[2]) + red[3]) / (float)d + a.eps);
    const GH_GLOBAL uint2* w = gh_gp<uint2>(a.norm);
    GH_GLOBAL uint2* out = gh_gpw<uint2>(a.normed) + row0 / 4;
    for (uint32_t c = tid; c < n4; c += 1024) {
        const float4 xv = ys[c];
        const uint2 wv = w[c];
        const uint32_t o0 = gh_f2h(xv.x * inverse * gh_h2f(wv.x & 0xFFFFu));
        const uint32_t o1 = gh_f2h(xv.y * inverse * gh_h2f(wv.x >> 16));
        const uint32_t o2 = gh_f2h(xv.z * inverse * gh_h2f(wv.y & 0xFFFFu));
        const uint32_t o3 = gh_f2h(xv.w * inverse * gh_h2f(wv.y >> 16));
        out[c] = make_uint2(o0 | (o1 << 16), o2 | (o3 << 16));
    }
}

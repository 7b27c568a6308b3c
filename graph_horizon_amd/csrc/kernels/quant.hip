// Q4_K / Q6_K weight repack (GGUF blocks -> device layout) and bit-exact dequantization.
// The device layout is a lossless byte permutation described in gh_kargs.h: quant bytes in
// planes of 16-byte chunks ordered so that lane i of a wavefront reads chunk i (one 1 KiB
// coalesced dwordx4 load per wave), headers in their own plane.
#include "gh_common.h"

// One thread per 16-byte chunk of a 144-byte Q4_K block (9 chunks: header, then 8 of qs).
GH_KERNEL __launch_bounds__(256) void gh_repack_q4k(GhRepackArgs a) {
    const size_t total = (size_t)a.rows * a.nb * 9;
    const size_t c = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= total) return;
    const size_t blk = c / 9;  // row * nb + b
    const uint32_t k = (uint32_t)(c % 9);
    const size_t row = blk / a.nb;
    const uint32_t b = (uint32_t)(blk % a.nb);
    const uint4 v = *(const uint4*)((const uint8_t*)a.src + blk * 144 + (size_t)k * 16);
    uint8_t* dst = (uint8_t*)a.dst;
    size_t off;
    if (k == 0) {
        off = (size_t)a.rows * a.nb * GH_Q4K_QS_BYTES + blk * 16;
    } else {
        const uint32_t q = k - 1;  // qs bytes [16q, 16q + 16)
        const uint32_t g = q >> 1, h = q & 1;
        off = row * GH_Q4K_QS_BYTES * a.nb + (size_t)h * 64 * a.nb + (size_t)(4 * b + g) * 16;
    }
    *(uint4*)(dst + off) = v;
}

// One thread per byte of a 210-byte Q6_K block (blocks are not 16-byte aligned in GGUF).
GH_KERNEL __launch_bounds__(256) void gh_repack_q6k(GhRepackArgs a) {
    const size_t total = (size_t)a.rows * a.nb * 210;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const size_t blk = i / 210;
    const uint32_t j = (uint32_t)(i % 210);
    const size_t row = blk / a.nb;
    const uint32_t b = (uint32_t)(blk % a.nb);
    const size_t nb = a.nb;
    size_t off;
    if (j < 128) {  // ql
        const uint32_t s = j / 64, w = j % 64;
        const uint32_t p = w / 32, l = w % 32;
        const uint32_t u = 4 * b + 2 * s + l / 16;
        off = row * GH_Q6K_QLH_BYTES * nb + (size_t)p * 64 * nb + (size_t)u * 16 + (l % 16);
    } else if (j < 192) {  // qh
        const uint32_t jj = j - 128;
        const uint32_t s = jj / 32, l = jj % 32;
        const uint32_t u = 4 * b + 2 * s + l / 16;
        off = row * GH_Q6K_QLH_BYTES * nb + 2 * 64 * nb + (size_t)u * 16 + (l % 16);
    } else if (j < 208) {  // scales
        off = (size_t)a.rows * GH_Q6K_QLH_BYTES * nb + blk * 16 + (j - 192);
    } else {  // d
        off = (size_t)a.rows * 208 * nb + blk * 2 + (j - 208);
    }
    ((uint8_t*)a.dst)[off] = ((const uint8_t*)a.src)[i];
}

// dequant_row_q4_k (backend/cpu/dequant.rs:93-123): w = (d*sc)*q - dmin*mn with two
// roundings (mul, mul, sub; contraction off), one thread per output value.
GH_KERNEL __launch_bounds__(256) void gh_dequant_q4k(GhDequantArgs a) {
#pragma clang fp contract(off)
    const uint32_t in_dim = a.nb * 256;
    const size_t total = (size_t)a.rows * in_dim;
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= total) return;
    const uint32_t r = (uint32_t)(t / in_dim);
    const uint32_t i = (uint32_t)(t % in_dim);
    const uint32_t row = a.row_list ? ((const uint32_t*)a.row_list)[r]
                                    : (a.row_ptr ? *(const uint32_t*)a.row_ptr : a.row0) + r;
    const uint32_t b = i >> 8, within = i & 255;
    const uint32_t j = within >> 5, l = within & 31;  // sub-block, index inside it
    const uint32_t g = j >> 1, h = l >> 4;
    const uint8_t* base = (const uint8_t*)a.w;
    const size_t nb = a.nb;
    const uint8_t qbyte = base[(size_t)row * GH_Q4K_QS_BYTES * nb + (size_t)h * 64 * nb +
                               (size_t)(4 * b + g) * 16 + (l & 15)];
    const uint4 hd = *(const uint4*)(base + (size_t)a.wrows * GH_Q4K_QS_BYTES * nb +
                                     ((size_t)row * nb + b) * 16);
    const float d = gh_h2f(hd.x & 0xFFFFu);
    const float dmin = gh_h2f(hd.x >> 16);
    uint32_t sc, mn;
    gh_q4k_scale_min(hd, j, sc, mn);
    const float dl = d * (float)sc;
    const float ml = dmin * (float)mn;
    const uint32_t q = (j & 1) ? (qbyte >> 4) : (qbyte & 0xFu);
    ((float*)a.out)[(size_t)r * in_dim + i] = dl * (float)q - ml;
}

// dequant_row_q6_k (backend/cpu/dequant.rs:274-308): w = (d*scale)*(q6 - 32).
GH_KERNEL __launch_bounds__(256) void gh_dequant_q6k(GhDequantArgs a) {
#pragma clang fp contract(off)
    const uint32_t in_dim = a.nb * 256;
    const size_t total = (size_t)a.rows * in_dim;
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= total) return;
    const uint32_t r = (uint32_t)(t / in_dim);
    const uint32_t i = (uint32_t)(t % in_dim);
    const uint32_t row = a.row_list ? ((const uint32_t*)a.row_list)[r]
                                    : (a.row_ptr ? *(const uint32_t*)a.row_ptr : a.row0) + r;
    const uint32_t b = i >> 8, within = i & 255;
    const uint32_t s = within >> 7, quarter = (within >> 5) & 3, l = within & 31;
    const uint32_t h = l >> 4;
    const uint32_t u = 4 * b + 2 * s + h;
    const uint8_t* base = (const uint8_t*)a.w;
    const size_t nb = a.nb;
    const uint8_t* plane = base + (size_t)row * GH_Q6K_QLH_BYTES * nb;
    const uint32_t ql = plane[(size_t)(quarter & 1) * 64 * nb + (size_t)u * 16 + (l & 15)];
    const uint32_t qh = plane[2 * 64 * nb + (size_t)u * 16 + (l & 15)];
    const uint32_t lo4 = (quarter & 2) ? (ql >> 4) : (ql & 0xFu);
    const uint32_t hi2 = (qh >> (2 * quarter)) & 3u;
    const int32_t q = (int32_t)(lo4 | (hi2 << 4)) - 32;
    const int8_t scale = (int8_t)base[(size_t)a.wrows * GH_Q6K_QLH_BYTES * nb +
                                      ((size_t)row * nb + b) * 16 + 8 * s + h + 2 * quarter];
    const uint16_t dbits =
        *(const uint16_t*)(base + (size_t)a.wrows * 208 * nb + ((size_t)row * nb + b) * 2);
    const float d = gh_h2f(dbits);
    ((float*)a.out)[(size_t)r * in_dim + i] = d * (float)scale * (float)q;
}

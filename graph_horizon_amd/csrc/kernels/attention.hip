// Causal GQA attention over the FP16 KV cache: split-K flash decode.
//
// Grid (kv_heads, splits, rows). A workgroup takes one kv head, the G = q_heads/kv_heads
// query heads that share it (each K/V row is read once for all G), and a contiguous range
// of split_len positions of one query row. It leaves per-head partials (max m, Σexp l,
// Σexp·V acc); gh_attn_merge combines the splits:
//   out = Σ_s e^{m_s-M} acc_s / Σ_s e^{m_s-M} l_s,  M = max_s m_s,
// which is the reference's softmax-weighted V sum (attention/mod.rs:220-258) re-associated.
// head_dim 128 (16 lanes x 8 FP16 per K row; 64 lanes x 2 FP16 per V row).
#include "gh_common.h"

namespace {
constexpr int kWaves = 4;
constexpr int kMaxSplitLen = 256;

__device__ __forceinline__ float sum16(float v) {
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) v += __shfl_xor(v, off, 16);
    return v;
}

template <int G>
__device__ __forceinline__ void attn_split_body(const GhAttnArgs& a) {
    __shared__ float sc[G][kMaxSplitLen];
    __shared__ float red[kWaves][G][128];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t kvh = blockIdx.x, split = blockIdx.y, row = blockIdx.z;
    const uint32_t pos = (a.pos_ptr ? *(const uint32_t*)a.pos_ptr : 0u) + a.base + row;
    const uint32_t len = pos + 1;
    const uint32_t t0 = split * a.split_len;
    const uint32_t h0 = kvh * G;
    const size_t part = ((size_t)row * a.q_heads + h0) * a.splits + split;  // + h*splits
    if (t0 >= len) return;  // beyond the causal range: the merge ignores this split
    const uint32_t n = min(len - t0, a.split_len);
    const size_t kv_row = (size_t)a.kv_heads * 128;  // elements per position
    const uint16_t* kbase = (const uint16_t*)a.kc + ((size_t)a.layer * a.context) * kv_row + kvh * 128;
    const uint16_t* vbase = (const uint16_t*)a.vc + ((size_t)a.layer * a.context) * kv_row + kvh * 128;

    // Pass 1: scores. 4 positions per wave instruction, 16 lanes x 8 FP16 each.
    const uint32_t sub = lane >> 4, d0 = (lane & 15u) * 8;
    float q[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const uint4 v = *(const uint4*)((const uint16_t*)a.q + ((size_t)row * a.q_heads + h0 + h) * 128 + d0);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            q[h][2 * j] = gh_h2f(w[j] & 0xFFFFu);
            q[h][2 * j + 1] = gh_h2f(w[j] >> 16);
        }
    }
    for (uint32_t p = wave * 4 + sub; p < ((n + 15) & ~15u); p += kWaves * 4) {
        const bool valid = p < n;
        uint4 kv = make_uint4(0, 0, 0, 0);
        if (valid) kv = *(const uint4*)(kbase + (size_t)(t0 + p) * kv_row + d0);
        const uint32_t w[4] = {kv.x, kv.y, kv.z, kv.w};
        float k[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            k[2 * j] = gh_h2f(w[j] & 0xFFFFu);
            k[2 * j + 1] = gh_h2f(w[j] >> 16);
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) s += q[h][j] * k[j];
            s = sum16(s);
            if (valid && (lane & 15u) == 0) sc[h][p] = s * a.scale;
        }
    }
    __syncthreads();

    // Pass 2: per-head max and exp, one wave per head.
    for (uint32_t h = wave; h < (uint32_t)G; h += kWaves) {
        float m = -__builtin_inff();
        for (uint32_t p = lane; p < n; p += 64) m = fmaxf(m, sc[h][p]);
        m = gh_wave_max(m);
        float l = 0.0f;
        for (uint32_t p = lane; p < n; p += 64) {
            const float e = expf(sc[h][p] - m);
            sc[h][p] = e;
            l += e;
        }
        l = gh_wave_sum(l);
        if (lane == 0) {
            ((float*)a.part_m)[part + (size_t)h * a.splits] = m;
            ((float*)a.part_l)[part + (size_t)h * a.splits] = l;
        }
    }
    __syncthreads();

    // Pass 3: Σ e·V, each wave a quarter of the positions, lane = 2 value dims.
    float acc[G][2];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h][0] = acc[h][1] = 0.0f;
    for (uint32_t p = wave; p < n; p += kWaves) {
        const uint32_t v = *(const uint32_t*)(vbase + (size_t)(t0 + p) * kv_row + 2 * lane);
        const float v0 = gh_h2f(v & 0xFFFFu), v1 = gh_h2f(v >> 16);
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float e = sc[h][p];
            acc[h][0] += e * v0;
            acc[h][1] += e * v1;
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        red[wave][h][2 * lane] = acc[h][0];
        red[wave][h][2 * lane + 1] = acc[h][1];
    }
    __syncthreads();
    for (uint32_t i = tid; i < (uint32_t)G * 128; i += blockDim.x) {
        const uint32_t h = i >> 7, d = i & 127u;
        const float s = (red[0][h][d] + red[1][h][d]) + (red[2][h][d] + red[3][h][d]);
        ((float*)a.part_acc)[(part + (size_t)h * a.splits) * 128 + d] = s;
    }
}

}  // namespace

GH_KERNEL __launch_bounds__(256) void gh_attn_split_g1(GhAttnArgs a) { attn_split_body<1>(a); }
GH_KERNEL __launch_bounds__(256) void gh_attn_split_g2(GhAttnArgs a) { attn_split_body<2>(a); }
GH_KERNEL __launch_bounds__(256) void gh_attn_split_g4(GhAttnArgs a) { attn_split_body<4>(a); }
GH_KERNEL __launch_bounds__(256) void gh_attn_split_g8(GhAttnArgs a) { attn_split_body<8>(a); }

// Merge: grid (q_heads, rows), 128 threads = value dims.
GH_KERNEL __launch_bounds__(128) void gh_attn_merge(GhAttnArgs a) {
    const uint32_t h = blockIdx.x, row = blockIdx.y, d = threadIdx.x;
    const uint32_t pos = (a.pos_ptr ? *(const uint32_t*)a.pos_ptr : 0u) + a.base + row;
    const uint32_t valid = (pos + a.split_len) / a.split_len;  // splits covering 0..pos
    const size_t part = ((size_t)row * a.q_heads + h) * a.splits;
    const float* pm = (const float*)a.part_m + part;
    const float* pl = (const float*)a.part_l + part;
    const float* pa = (const float*)a.part_acc + part * 128;
    float M = -__builtin_inff();
    for (uint32_t s = 0; s < valid; ++s) M = fmaxf(M, pm[s]);
    float L = 0.0f, acc = 0.0f;
    for (uint32_t s = 0; s < valid; ++s) {
        const float w = expf(pm[s] - M);
        L += w * pl[s];
        acc += w * pa[(size_t)s * 128 + d];
    }
    ((uint16_t*)a.out)[((size_t)row * a.q_heads + h) * 128 + d] = gh_f2h(acc / L);
}

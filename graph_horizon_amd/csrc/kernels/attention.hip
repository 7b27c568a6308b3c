// Causal GQA attention over the FP16 KV cache: split-K flash decode in one kernel.
//
// Grid (splits, kv_heads, rows); 256 threads. A workgroup takes one kv head, the G =
// q_heads/kv_heads query heads sharing it (each K/V row is read once for all G), and every
// nsplit-th chunk of 64 positions of one query row (pos_r = base + r, or *pos_ptr + base + r):
//   scores  4 lanes per position, 32 FP16 of the K row each, v_dot2_f32_f16 against the FP16
//           query (products of FP16 values are exact in FP32), quad DPP sum, x 1/sqrt(128);
//   online softmax per head across the workgroup's chunks: running max m, Σe l, Σe·V acc
//           (each lane owns 2 value dims; waves split the positions of a chunk).
// The workgroup's (m, l, acc) goes to the workspace; the last workgroup of a (row, kv head)
// to finish (agent-scope atomic counter, which it resets for the next launch) merges them:
//   out = Σ_s e^{m_s-M} acc_s / Σ_s e^{m_s-M} l_s,  M = max_s m_s
// — the reference's three-pass softmax-weighted V sum (attention/mod.rs:220-258), re-associated.
// head_dim = value_dim = 128; splits <= 32.
#include "gh_common.h"

namespace {
constexpr uint32_t kChunk = 64;  // positions per chunk
constexpr int kWaves = 4;
constexpr uint32_t kMaxSplits = 32;

template <int G>
__device__ __forceinline__ void attn_body(const GhAttnArgs& a) {
    __shared__ float sc[G][kChunk];
    __shared__ float stat[G][2];  // per head: running max, rescale factor of this chunk
    __shared__ float red[kWaves][G][128];
    __shared__ float wsplit[G][kMaxSplits];
    __shared__ uint32_t last;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t split = blockIdx.x, kvh = blockIdx.y, row = blockIdx.z;
    const uint32_t pos = (a.pos_ptr ? *gh_gp<uint32_t>(a.pos_ptr) : 0u) + a.base + row;
    const uint32_t len = pos + 1;
    const uint32_t nchunk = (len + kChunk - 1) / kChunk;
    const uint32_t nsplit = min(nchunk, a.splits);
    if (split >= nsplit) return;  // fixed grids (replayed graphs) may exceed the causal range
    const uint32_t h0 = kvh * G;
    const size_t kv_row = (size_t)a.kv_heads * 128;
    const size_t cache0 = (size_t)a.layer * a.context * kv_row + (size_t)kvh * 128;
    const uint16_t* kc = (const uint16_t*)a.kc + cache0;
    const uint16_t* vc = (const uint16_t*)a.vc + cache0;
    const uint32_t qd = lane & 3u;
    const uint32_t pl = wave * 16 + (lane >> 2);  // this lane's position within a chunk (scores)

    // FP16 query slices [32·qd, +32) of the G heads, as 16 pairs each
    uint4 qv[G][4];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const GH_GLOBAL uint4* qp =
            gh_gp<uint4>(a.q + (((uint64_t)row * a.q_heads + h0 + h) * 128 + qd * 32) * 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[h][i] = qp[i];
    }
    float m_run[G], l_run[G], acc[G][2];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m_run[h] = -__builtin_inff();
        l_run[h] = 0.0f;
        acc[h][0] = acc[h][1] = 0.0f;
    }

    for (uint32_t c = split; c < nchunk; c += nsplit) {
        const uint32_t t0 = c * kChunk;
        const uint32_t n = min(len - t0, kChunk);
        // issue this chunk's K (4 x 16 B per lane) and V (16 dwords per lane) loads together
        uint4 kr[4];
        {
            const GH_GLOBAL uint4* src =
                gh_gp<uint4>((uint64_t)(kc + (size_t)(t0 + min(pl, n - 1)) * kv_row + qd * 32));
#pragma unroll
            for (int i = 0; i < 4; ++i) kr[i] = src[i];
        }
        uint32_t vv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t pp = min(wave + 4 * (uint32_t)i, n - 1);
            vv[i] = gh_gp<uint32_t>((uint64_t)(vc + (size_t)(t0 + pp) * kv_row))[lane];
        }
        // scores
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s = gh_dot2(qv[h][i].x, kr[i].x, s);
                s = gh_dot2(qv[h][i].y, kr[i].y, s);
                s = gh_dot2(qv[h][i].z, kr[i].z, s);
                s = gh_dot2(qv[h][i].w, kr[i].w, s);
            }
            s += GH_DPP(s, 0xB1, 0xF);  // quad_perm [1,0,3,2]
            s += GH_DPP(s, 0x4E, 0xF);  // quad_perm [2,3,0,1]
            if (qd == 0 && pl < n) sc[h][pl] = s * a.scale;
        }
        __syncthreads();
        // chunk max and exponentials, one wave per head
        for (uint32_t h = wave; h < (uint32_t)G; h += kWaves) {
            const float v = lane < n ? sc[h][lane] : -__builtin_inff();
            const float m_new = fmaxf(m_run[h], gh_wave_max(v));
            if (lane < n) sc[h][lane] = expf(v - m_new);
            if (lane == 0) {
                stat[h][0] = m_new;
                stat[h][1] = expf(m_run[h] - m_new);  // 0 on the first chunk
            }
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float f = stat[h][1];
            m_run[h] = stat[h][0];
            float e_sum = 0.0f;
            acc[h][0] *= f;
            acc[h][1] *= f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t pp = wave + 4 * (uint32_t)i;
                if (pp < n) {
                    const float e = sc[h][pp];
                    acc[h][0] += e * gh_h2f(vv[i] & 0xFFFFu);
                    acc[h][1] += e * gh_h2f(vv[i] >> 16);
                }
            }
            for (uint32_t pp = lane; pp < n; pp += 64) e_sum += sc[h][pp];
            l_run[h] = l_run[h] * f + gh_wave_sum(e_sum);
        }
        __syncthreads();  // sc is rewritten by the next chunk
    }

    // this workgroup's partial: (m, l) per head, acc summed over the waves
#pragma unroll
    for (int h = 0; h < G; ++h) {
        red[wave][h][2 * lane] = acc[h][0];
        red[wave][h][2 * lane + 1] = acc[h][1];
    }
    __syncthreads();
    for (uint32_t i = tid; i < (uint32_t)G * 128; i += blockDim.x) {
        const uint32_t h = i >> 7, d = i & 127u;
        const float v = (red[0][h][d] + red[1][h][d]) + (red[2][h][d] + red[3][h][d]);
        const size_t pi = ((size_t)row * a.q_heads + h0 + h) * a.splits + split;
        gh_gpw<float>(a.part_acc)[pi * 128 + d] = v;
        if (d == 0) {
            gh_gpw<float>(a.part_m)[pi] = m_run[h];
            gh_gpw<float>(a.part_l)[pi] = l_run[h];
        }
    }

    // the last workgroup of this (row, kv head) merges the splits
    __syncthreads();
    if (tid == 0) {
        uint32_t* ctr = (uint32_t*)a.counters + (size_t)row * a.kv_heads + kvh;
        const uint32_t done =
            __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last = (done + 1 == nsplit) ? 1u : 0u;
        if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // weights e^{m_s - M} per (head, split), and L = Σ_s w_s l_s
    for (uint32_t h = wave; h < (uint32_t)G; h += kWaves) {
        const size_t base = ((size_t)row * a.q_heads + h0 + h) * a.splits;
        const float ms = lane < nsplit ? gh_gp<float>(a.part_m)[base + lane] : -__builtin_inff();
        const float M = gh_wave_max(ms);
        const float w = lane < nsplit ? expf(ms - M) : 0.0f;
        const float L = gh_wave_sum(lane < nsplit ? w * gh_gp<float>(a.part_l)[base + lane] : 0.0f);
        if (lane < nsplit) wsplit[h][lane] = w / L;
    }
    __syncthreads();
    for (uint32_t i = tid; i < (uint32_t)G * 128; i += blockDim.x) {
        const uint32_t h = i >> 7, d = i & 127u;
        const size_t base = ((size_t)row * a.q_heads + h0 + h) * a.splits;
        const GH_GLOBAL float* pa = gh_gp<float>(a.part_acc) + base * 128 + d;
        float pv[kMaxSplits];
#pragma unroll
        for (uint32_t s2 = 0; s2 < kMaxSplits; ++s2) pv[s2] = s2 < nsplit ? pa[(size_t)s2 * 128] : 0.0f;
        float o = 0.0f;
#pragma unroll
        for (uint32_t s2 = 0; s2 < kMaxSplits; ++s2)
            if (s2 < nsplit) o += wsplit[h][s2] * pv[s2];
        gh_gpw<uint16_t>(a.out)[((size_t)row * a.q_heads + h0 + h) * 128 + d] = gh_f2h(o);
    }
}

}  // namespace

GH_KERNEL __launch_bounds__(256) void gh_attn_g1(GhAttnArgs a) { attn_body<1>(a); }
GH_KERNEL __launch_bounds__(256) void gh_attn_g2(GhAttnArgs a) { attn_body<2>(a); }
GH_KERNEL __launch_bounds__(256) void gh_attn_g4(GhAttnArgs a) { attn_body<4>(a); }
GH_KERNEL __launch_bounds__(256) void gh_attn_g8(GhAttnArgs a) { attn_body<8>(a); }

// Causal GQA attention over the FP16 KV cache: split-K flash decode in one kernel.
//
// Grid (splits, kv_heads, rows); 256 threads. A workgroup takes one kv head, the G =
// q_heads/kv_heads query heads sharing it (each K/V row is read once for all G), and every
// nsplit-th chunk of 64 positions of one query row (pos_r = base + r, or *pos_ptr + base + r).
// Wave w owns positions 16 w .. 16 w + 15 of each chunk and keeps its own online-softmax
// state, so chunks need no workgroup barrier. Two forms of the per-wave work:
//   G = 4, 8 (attn_mfma_body): scores and the weighted V sum on the matrix cores (below);
//   G = 1, 2 (attn_body): 4 lanes per position, 32 FP16 of the K row each, v_dot2_f32_f16
//           against the FP16 query (products of FP16 values are exact in FP32), quad DPP
//           sum; running max m, Σe l and Σe·V per head (each lane owns 2 value dims; the
//           weights of the wave's 16 positions are broadcast with v_readlane).
// K and V are read through range-bounded buffer loads (kv_rsrc); the next chunk's loads are
// issued before the current chunk is computed. At the end the four waves merge in LDS
// (attn_finish); with one split the workgroup writes the output, otherwise it writes
// (m, l, acc) to the workspace and the last workgroup of its (row, kv head) (agent-scope atomic
// counter, reset by that workgroup for the next launch) merges the splits:
//   out = Σ_s e^{m_s-M} acc_s / Σ_s e^{m_s-M} l_s,  M = max_s m_s
// — the reference's three-pass softmax-weighted V sum (attention/mod.rs:220-258), re-associated.
// head_dim = value_dim = 128; splits <= kMaxSplits.
//
// XCD-local form (the `_x` kernels): grid (xcds, splits, ceil(rows·kv_heads / xcds)), where
// workgroup (x, split, z) serves the (row, kv head) pair p = z·xcds + x. The dispatcher hands
// workgroup i of a launch to XCD i mod xcds (the host verifies this at start-up with
// gh_xcd_probe and keeps the agent-scope form otherwise), so every split of a pair runs on one
// XCD and the partials travel through that XCD's L2 — plain stores, which the CU's L1 writes
// through into the L2, and loads that miss the L1 — instead of through device memory.
#include "gh_common.h"

namespace {
constexpr uint32_t kChunk = 64;  // positions per chunk
// Buffer resource word 3 for gfx9-family raw buffers (32-bit data format, no swizzle).
constexpr int kBufWord3 = 0x00020000;
constexpr int kWaves = 4;
constexpr uint32_t kMaxSplits = 32;

template <int G>
struct ChunkRegs {
    uint4 k[4];       // K row of position 16·wave + lane/4, dims 32·(lane%4) .. +32
    uint32_t v[16];   // V dims 2·lane, 2·lane+1 of positions 16·wave + i
};

// K and V of one kv head are read through raw buffer resources whose range ends at position
// lim: the row's length (lim = len), or for the first chunk, whose loads go out before the
// position is read, the cache's context. Positions past the range read as zero without a
// memory access, so the request for a chunk past the last (the loop's unconditional
// prefetch) costs no round trip.
struct KVRsrc {
    __amdgpu_buffer_rsrc_t k, v;
};
__device__ __forceinline__ KVRsrc kv_rsrc(const uint16_t* kc, const uint16_t* vc, size_t kv_row, uint32_t lim) {
    // the host keeps (context + 2048) x kv_row x 2 bytes below 2^31, so every offset below
    // (chunks up to max(32, nchunk) + 1) fits
    const int bytes = (int)((size_t)lim * kv_row * 2);
    return {__builtin_amdgcn_make_buffer_rsrc((void*)kc, 0, bytes, kBufWord3),
            __builtin_amdgcn_make_buffer_rsrc((void*)vc, 0, bytes, kBufWord3)};
}

template <int G>
__device__ __forceinline__ void load_chunk(const KVRsrc& rs, uint32_t row_bytes, uint32_t c, ChunkRegs<G>& r) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t p0 = c * kChunk + wave * 16;
    const uint32_t ok = (p0 + (lane >> 2)) * row_bytes + (lane & 3u) * 64;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r.k[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.k, ok + 16 * i, 0, 0));
#pragma unroll
    for (int i = 0; i < 16; ++i)
        r.v[i] = __builtin_amdgcn_raw_buffer_load_b32(rs.v, (p0 + (uint32_t)i) * row_bytes + lane * 4, 0, 0);
}

// Zero the V values of positions >= len in the first chunk, which is read before the
// position is known (slots past the row may hold anything, and their weight 0 times a NaN
// would not be 0); their scores are replaced by -inf in chunk_step.
template <int G>
__device__ __forceinline__ void mask_chunk(uint32_t c, uint32_t len, ChunkRegs<G>& r) {
    const uint32_t p0 = c * kChunk + (threadIdx.x >> 6) * 16;
#pragma unroll
    for (int i = 0; i < 16; ++i) r.v[i] = p0 + (uint32_t)i < len ? r.v[i] : 0u;
}

template <int G>
__device__ __forceinline__ void chunk_step(const ChunkRegs<G>& r, const uint4 (&qv)[G][4], float scale,
                                           uint32_t c, uint32_t len, float (&m)[G], float (&l)[G],
                                           float (&acc)[G][2]) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t pos = c * kChunk + wave * 16 + (lane >> 2);
    const bool valid = pos < len;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s = gh_dot2(qv[h][i].x, r.k[i].x, s);
            s = gh_dot2(qv[h][i].y, r.k[i].y, s);
            s = gh_dot2(qv[h][i].z, r.k[i].z, s);
            s = gh_dot2(qv[h][i].w, r.k[i].w, s);
        }
        s += GH_DPP(s, 0xB1, 0xF);  // quad_perm [1,0,3,2]
        s += GH_DPP(s, 0x4E, 0xF);  // quad_perm [2,3,0,1]
        s = valid ? s * scale : -__builtin_inff();
        // max over the wave's 16 positions: rotate by 4 and 8 within each 16-lane row, then
        // the four rows' maxima through SGPRs
        float mx = fmaxf(s, GH_DPP(s, 0x124, 0xF));  // row_ror:4
        mx = fmaxf(mx, GH_DPP(mx, 0x128, 0xF));      // row_ror:8
        mx = fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 0)),
                         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 16))),
                   fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 32)),
                         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 48))));
        const float m_new = fmaxf(m[h], mx);  // finite: the wave's first position is valid
        const float f = m_new == -__builtin_inff() ? 1.0f : expf(m[h] - m_new);
        const float p = valid ? expf(s - m_new) : 0.0f;
        m[h] = m_new;
        l[h] = l[h] * f + ((lane & 3u) == 0 ? p : 0.0f);  // per-lane partial of Σe
        float a0 = acc[h][0] * f, a1 = acc[h][1] * f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float pi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), 4 * i));
            a0 += pi * gh_h2f(r.v[i] & 0xFFFFu);
            a1 += pi * gh_h2f(r.v[i] >> 16);
        }
        acc[h][0] = a0;
        acc[h][1] = a1;
    }
}

// The decode kernels' first-needed arguments, passed as leading scalar kernel parameters that
// the dispatch preloads into SGPRs: the query, cache and position loads need no kernarg load.
struct AttnHot {
    uint64_t q, kc, vc, pos_ptr;
    uint32_t layer, context, q_heads, kv_heads;
    uint32_t rows, xcds;  // query rows of the launch; XCD count of the XL grid
};

// The workgroup's split, kv head and query row: from the grid's three axes, or (XL) from the
// (row, kv head) pair p = z·xcds + x, whose splits run along y. row >= rows marks a
// workgroup of the last z past the pairs (it exits before any load).
struct AttnIds {
    uint32_t split, kvh, row;
};
template <bool XL>
__device__ __forceinline__ AttnIds attn_ids(const GhAttnArgs& a, const AttnHot& hot) {
    if constexpr (!XL) {
        return {blockIdx.x, blockIdx.y, blockIdx.z};
    } else {
        const uint32_t p = blockIdx.z * hot.xcds + blockIdx.x;
        return {blockIdx.y, p % hot.kv_heads, p / hot.kv_heads};
    }
}

// The split partials' exchange. Agent scope (any placement of the splits): stores written
// through to the device coherence point and loads that do not hit another XCD's stale L2
// line. XCD-local (XL, every split of the pair on this XCD): plain stores, which land in the
// shared L2 (the CU's L1 writes through), and loads that miss the reading CU's L1 (the
// workgroup-scope atomic load is encoded with sc0, an L1 miss; the data comes from the L2).
template <bool XL>
__device__ __forceinline__ void st_part(GH_GLOBAL float* p, float v) {
    if constexpr (XL) *p = v;
    else __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool XL>
__device__ __forceinline__ float ld_part(const GH_GLOBAL float* p) {
    if constexpr (XL) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-wave softmax state of a decode workgroup, merged by attn_finish.
template <int G>
struct AttnShared {
    float wm[kWaves][G], wl[kWaves][G];  // running max and Σe of each wave, per head
    // Σe·V of each wave, per head and value dim; rows padded to 132 floats so that the lanes of
    // the G heads, which store the same value dims at once, do not share banks
    float wacc[kWaves][G][132];
    float we[kWaves][G];       // e^{m_w - M} per wave and head (the wave merge's weights)
    float hm[G], hl[G];        // M and L per head
    float wsplit[G][kMaxSplits];
    uint32_t last;
};

template <int G, bool XL, uint32_t MS = kMaxSplits>
__device__ __forceinline__ void attn_finish(const GhAttnArgs& a, const AttnHot& hot, AttnShared<G>& sh,
                                            AttnIds id, uint32_t nsplit);

template <int G, bool XL>
__device__ __forceinline__ void attn_body(const GhAttnArgs& a, const AttnHot& hot) {
    __shared__ AttnShared<G> sh;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const AttnIds id = attn_ids<XL>(a, hot);
    if (XL && id.row >= hot.rows) return;
    const uint32_t split = id.split, kvh = id.kvh, row = id.row;
    const uint32_t h0 = kvh * G;
    // FP16 query slices [32·qd, +32) of the G heads, as 16 pairs each (issued before the
    // position is known)
    uint4 qv[G][4];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const GH_GLOBAL uint4* qp =
            gh_gp<uint4>(hot.q + (((uint64_t)row * hot.q_heads + h0 + h) * 128 + (lane & 3u) * 32) * 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[h][i] = qp[i];
    }
    const size_t kv_row = (size_t)hot.kv_heads * 128;
    const size_t cache0 = (size_t)hot.layer * hot.context * kv_row + (size_t)kvh * 128;
    const uint16_t* kc = (const uint16_t*)hot.kc + cache0;
    const uint16_t* vc = (const uint16_t*)hot.vc + cache0;
    const uint32_t row_bytes = (uint32_t)kv_row * 2;
    // this split's first chunk (chunk `split`) is requested before the position arrives
    ChunkRegs<G> ra, rb;
    load_chunk<G>(kv_rsrc(kc, vc, kv_row, hot.context), row_bytes, split, ra);
    const uint32_t pos = (hot.pos_ptr ? *gh_gp<uint32_t>(hot.pos_ptr) : 0u) + a.base + row;
    const uint32_t len = pos + 1;
    const uint32_t nchunk = (len + kChunk - 1) / kChunk;
    const uint32_t nsplit = min(nchunk, a.splits);
    if (split >= nsplit) return;  // fixed grids (replayed graphs) may exceed the causal range

    float m[G], l[G], acc[G][2];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = -__builtin_inff();
        l[h] = 0.0f;
        acc[h][0] = acc[h][1] = 0.0f;
    }
    // chunks split, split + nsplit, ...; a wave whose 16 positions of a chunk all lie past
    // the row's length still runs it (every weight is 0) so the loop stays wave-uniform. The
    // next chunk is requested unconditionally (a load under a branch makes the compiler wait
    // for every load at the join); past the last chunk the request is out of range.
    const KVRsrc rs = kv_rsrc(kc, vc, kv_row, len);
    for (uint32_t c = split; c < nchunk; c += 2 * nsplit) {
        const uint32_t c1 = c + nsplit, c2 = c + 2 * nsplit;
        load_chunk<G>(rs, row_bytes, min(c1, nchunk), rb);
        if (c == split) mask_chunk<G>(c, len, ra);  // after the next chunk's loads are out
        if (c * kChunk + wave * 16 < len) chunk_step<G>(ra, qv, a.scale, c, len, m, l, acc);
        if (c1 >= nchunk) break;
        load_chunk<G>(rs, row_bytes, min(c2, nchunk), ra);
        if (c1 * kChunk + wave * 16 < len) chunk_step<G>(rb, qv, a.scale, c1, len, m, l, acc);
    }

#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float lt = gh_wave_sum(l[h]);
        if (lane == 0) {
            sh.wm[wave][h] = m[h];
            sh.wl[wave][h] = lt;
        }
        sh.wacc[wave][h][2 * lane] = acc[h][0];
        sh.wacc[wave][h][2 * lane + 1] = acc[h][1];
    }
    attn_finish<G, XL>(a, hot, sh, id, nsplit);
}

// Merge of the four waves' states (in sh) into the workgroup's partial or, with one split,
// the output; with several splits the last workgroup of the (row, kv head) merges them:
//   M = max m_w, L = Σ l_w e^{m_w - M}, ACC = Σ acc_w e^{m_w - M}, then across splits
//   out = Σ_s e^{m_s-M} acc_s / Σ_s e^{m_s-M} l_s.
// MS: split slots the merge reads (the launch's split count is at most MS); slots past nsplit
// re-read the last split and get weight 0, which leaves every sum's bits unchanged.
template <int G, bool XL, uint32_t MS>
__device__ __forceinline__ void attn_finish(const GhAttnArgs& a, const AttnHot& hot, AttnShared<G>& sh,
                                            AttnIds id, uint32_t nsplit) {
    auto& wm = sh.wm;
    auto& wl = sh.wl;
    auto& wacc = sh.wacc;
    auto& wsplit = sh.wsplit;
    auto& last = sh.last;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t split = id.split, kvh = id.kvh, row = id.row;
    const uint32_t h0 = kvh * G;
    __syncthreads();
    // the waves' weights, M and L once per head (not once per value dim)
    if (tid < (uint32_t)G) {
        const uint32_t h = tid;
        float M = -__builtin_inff();
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, wm[w][h]);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float e = wm[w][h] == -__builtin_inff() ? 0.0f : expf(wm[w][h] - M);
            sh.we[w][h] = e;
            L += e * wl[w][h];
        }
        sh.hm[h] = M;
        sh.hl[h] = L;
    }
    __syncthreads();
    const size_t pbase = ((size_t)row * hot.q_heads + h0) * a.splits;
    for (uint32_t i = tid; i < (uint32_t)G * 128; i += 256) {
        const uint32_t h = i >> 7, d = i & 127u;
        const float M = sh.hm[h], L = sh.hl[h];
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) v += sh.we[w][h] * wacc[w][h][d];
        if (nsplit == 1) {
            gh_gpw<uint16_t>(a.out)[((size_t)row * hot.q_heads + h0 + h) * 128 + d] = gh_f2h(v / L);
        } else {
            const size_t pi = pbase + (size_t)h * a.splits + split;
            st_part<XL>(gh_gpw<float>(a.part_acc) + pi * 128 + d, v);
            if (d == 0) {
                st_part<XL>(gh_gpw<float>(a.part_m) + pi, M);
                st_part<XL>(gh_gpw<float>(a.part_l) + pi, L);
            }
        }
    }
    if (nsplit == 1) return;

    // The last workgroup of this (row, kv head) merges the splits. Every partial crosses
    // workgroups only through agent-scope atomic accesses — stores written through to the
    // device coherence point, loads that do not hit a stale L2 line of another XCD — so the
    // exchange needs no L2 writeback or invalidation (an agent-scope release/acquire pair
    // would do both to the whole L2: ~3 us per launch measured). Each thread waits for its
    // own stores to complete before the barrier (the wait is an asm statement that clobbers
    // memory, so the compiler keeps the stores ahead of it), so the counter increment follows
    // all of the workgroup's partials; the last workgroup issues its loads only after it has
    // seen the count (the barrier that publishes `last` orders them after the atomic's return).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        uint32_t* ctr = (uint32_t*)a.counters + (size_t)row * hot.kv_heads + kvh;
        const uint32_t done = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = (done + 1 == nsplit) ? 1u : 0u;
        if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    // every partial this workgroup needs is requested before any is used (indexes past
    // nsplit re-read split nsplit - 1 and get weight 0; unconditional loads measured faster
    // than skipping them)
    constexpr uint32_t kOut = (uint32_t)G * 128 / 256;  // outputs per thread (G >= 2)
    float pv[kOut > 0 ? kOut : 1][MS];
#pragma unroll
    for (uint32_t o = 0; o < kOut; ++o) {
        const uint32_t i = tid + 256 * o, h = i >> 7, d = i & 127u;
        const GH_GLOBAL float* pa = gh_gp<float>(a.part_acc) + (pbase + (size_t)h * a.splits) * 128 + d;
#pragma unroll
        for (uint32_t j = 0; j < MS; ++j) pv[o][j] = ld_part<XL>(pa + (size_t)min(j, nsplit - 1) * 128);
    }
    // weights e^{m_s - M} / L per (head, split): lanes are splits, wave h handles head h
    for (uint32_t h = wave; h < (uint32_t)G; h += kWaves) {
        const size_t base = pbase + (size_t)h * a.splits;
        const uint32_t s2 = min(lane, nsplit - 1);
        const float ms = ld_part<XL>(gh_gp<float>(a.part_m) + base + s2);
        const float ls = ld_part<XL>(gh_gp<float>(a.part_l) + base + s2);
        const float M = gh_wave_max(lane < nsplit ? ms : -__builtin_inff());
        const float w = lane < nsplit ? expf(ms - M) : 0.0f;
        const float L = gh_wave_sum(w * ls);
        if (lane < kMaxSplits) wsplit[h][lane] = w / L;
    }
    __syncthreads();
    if constexpr (kOut > 0) {
#pragma unroll
        for (uint32_t o = 0; o < kOut; ++o) {
            const uint32_t i = tid + 256 * o, h = i >> 7, d = i & 127u;
            float acc_o = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < MS; ++j) acc_o += wsplit[h][j] * pv[o][j];
            gh_gpw<uint16_t>(a.out)[((size_t)row * hot.q_heads + h0 + h) * 128 + d] = gh_f2h(acc_o);
        }
    } else {
        // G = 1: 128 outputs, threads 0..127
        if (tid < 128) {
            const GH_GLOBAL float* pa = gh_gp<float>(a.part_acc) + pbase * 128 + tid;
            float acc_o = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < MS; ++j)
                acc_o += wsplit[0][j] * ld_part<XL>(pa + (size_t)min(j, nsplit - 1) * 128);
            gh_gpw<uint16_t>(a.out)[((size_t)row * hot.q_heads + h0) * 128 + tid] = gh_f2h(acc_o);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// The same decode on the matrix cores, for G = 4 or 8 query heads per kv head (head_dim =
// value_dim = 128). Same grid, chunking, splits and merge as attn_body; per wave and 16
// positions of a chunk:
//   S^T = K · Q^T   4 x v_mfma_f32_16x16x32_f16: A = the 16 K rows straight from memory (lane
//                   l: position l % 16, dims 32 s + 8 (l / 16) .. + 8), B = the FP16 query
//                   (column n = l % 16 is head n; columns >= G are zero). Lane l receives the
//                   scores of head n = l % 16 at positions 4 (l / 16) + i, i < 4;
//   softmax         per lane, for its head: the running max is shared by the head's four
//                   lanes (permlane swaps), each lane keeps its partial Σe;
//   O^T += V^T·P^T  per 8-dim tile t, 2 x v_mfma_f32_16x16x16_f16: B = the lane's own four
//                   weights (P split into FP16 hi + lo, so P·V keeps FP32-level accuracy),
//                   A = V^T with output row m standing for value dim 8 m + t: lane l loads the
//                   16-byte V row slice of dims 8 (l % 16) .. + 8 at its four positions and
//                   picks element t of each. Lane l then holds head n's value dims
//                   8 (4 (l / 16) + i) + t, i.e. 32 (l / 16) .. + 32.
// Products of FP16 values are exact in FP32; accumulation is FP32 (in a different order from
// attn_body's, within the tests' bar against the oracle).
typedef _Float16 dh8 __attribute__((ext_vector_type(8)));
typedef _Float16 dh4 __attribute__((ext_vector_type(4)));
typedef float df4 __attribute__((ext_vector_type(4)));

// max / sum over the four lanes n, n + 16, n + 32, n + 48 of a head (the 16-lane rows)
__device__ __forceinline__ float rows_max(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

struct MChunk {
    uint4 k[4];  // K: position l % 16, dims 32 s + 8 (l / 16) .. + 8 (s = k-step)
    uint4 v[4];  // V: position 4 (l / 16) + i, dims 8 (l % 16) .. + 8
};

__device__ __forceinline__ void load_mchunk(const KVRsrc& rs, uint32_t row_bytes, uint32_t c, MChunk& r) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, n = lane & 15u, g = lane >> 4;
    const uint32_t p0 = c * kChunk + wave * 16;
    const uint32_t ok = (p0 + n) * row_bytes + 16 * g;
#pragma unroll
    for (int s = 0; s < 4; ++s)
        r.k[s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.k, ok + 64 * s, 0, 0));
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r.v[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rs.v, (p0 + 4 * g + (uint32_t)i) * row_bytes + 16 * n, 0, 0));
}

// element t of the 16-byte slices of four positions, as one A fragment (k = the positions)
__device__ __forceinline__ dh4 v_column(const uint4 (&v)[4], int t) {
    auto word = [&](int i) __attribute__((always_inline)) {
        const uint4 x = v[i];
        const uint32_t w = (t >> 1) == 0 ? x.x : (t >> 1) == 1 ? x.y : (t >> 1) == 2 ? x.z : x.w;
        return w;
    };
    uint32_t d0, d1;
    if (t & 1) {
        d0 = (word(0) >> 16) | (word(1) & 0xFFFF0000u);
        d1 = (word(2) >> 16) | (word(3) & 0xFFFF0000u);
    } else {
        d0 = (word(0) & 0xFFFFu) | (word(1) << 16);
        d1 = (word(2) & 0xFFFFu) | (word(3) << 16);
    }
    return __builtin_bit_cast(dh4, make_uint2(d0, d1));
}

__device__ __forceinline__ void mchunk_step(const MChunk& r, const dh8 (&qf)[4], float scale, uint32_t c,
                                            uint32_t len, float& m, float& l, df4 (&acc)[8]) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, g = lane >> 4;
    const uint32_t p0 = c * kChunk + wave * 16 + 4 * g;  // this lane's first position
    df4 st = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
        st = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(dh8, r.k[s]), qf[s], st, 0, 0, 0);
    float sc[4];
    float mx = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sc[i] = p0 + (uint32_t)i < len ? st[i] * scale : -__builtin_inff();
        mx = fmaxf(mx, sc[i]);
    }
    const float m_new = fmaxf(m, rows_max(mx));  // finite: the wave's first position is valid
    const float f = m_new == -__builtin_inff() ? 1.0f : expf(m - m_new);
    float p[4], ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        p[i] = p0 + (uint32_t)i < len ? expf(sc[i] - m_new) : 0.0f;
        ps += p[i];
    }
    m = m_new;
    l = l * f + ps;
    dh4 ph, pl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ph[i] = (_Float16)p[i];
        pl[i] = (_Float16)(p[i] - (float)ph[i]);
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        acc[t] *= f;
        const dh4 vt = v_column(r.v, t);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(vt, ph, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(vt, pl, acc[t], 0, 0, 0);
    }
}

template <int G, bool XL, uint32_t MS = kMaxSplits>
__device__ __forceinline__ void attn_mfma_body(const GhAttnArgs& a, const AttnHot& hot) {
    static_assert(G == 4 || G == 8, "matrix-core decode serves 4 or 8 query heads per kv head");
    __shared__ AttnShared<G> sh;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, n = lane & 15u, g = lane >> 4;
    const AttnIds id = attn_ids<XL>(a, hot);
    if (XL && id.row >= hot.rows) return;
    const uint32_t split = id.split, kvh = id.kvh, row = id.row;
    const uint32_t h0 = kvh * G;
    // B fragments of the query: head n (zero past G), dims 32 s + 8 g .. + 8
    dh8 qf[4];
    const GH_GLOBAL uint4* qp =
        gh_gp<uint4>(hot.q + (((uint64_t)row * hot.q_heads + h0 + min(n, (uint32_t)G - 1)) * 128 + 8 * g) * 2);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint4 x = qp[4 * s];
        qf[s] = __builtin_bit_cast(dh8, n < (uint32_t)G ? x : make_uint4(0u, 0u, 0u, 0u));
    }
    const size_t kv_row = (size_t)hot.kv_heads * 128;
    const size_t cache0 = (size_t)hot.layer * hot.context * kv_row + (size_t)kvh * 128;
    const uint16_t* kc = (const uint16_t*)hot.kc + cache0;
    const uint16_t* vc = (const uint16_t*)hot.vc + cache0;
    const uint32_t row_bytes = (uint32_t)kv_row * 2;
    MChunk ra, rb;
    load_mchunk(kv_rsrc(kc, vc, kv_row, hot.context), row_bytes, split, ra);
    const uint32_t pos = (hot.pos_ptr ? *gh_gp<uint32_t>(hot.pos_ptr) : 0u) + a.base + row;
    const uint32_t len = pos + 1;
    const uint32_t nchunk = (len + kChunk - 1) / kChunk;
    const uint32_t nsplit = min(nchunk, a.splits);
    if (split >= nsplit) return;  // fixed grids (replayed graphs) may exceed the causal range

    float m = -__builtin_inff(), l = 0.0f;
    df4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = df4{0.0f, 0.0f, 0.0f, 0.0f};
    const KVRsrc rs = kv_rsrc(kc, vc, kv_row, len);
    for (uint32_t c = split; c < nchunk; c += 2 * nsplit) {
        const uint32_t c1 = c + nsplit, c2 = c + 2 * nsplit;
        load_mchunk(rs, row_bytes, min(c1, nchunk), rb);
        if (c == split) {
            // the first chunk was read up to the context: zero V past the row (its weights
            // are 0, and 0 times a stale NaN would not be)
            const uint32_t pv0 = c * kChunk + wave * 16 + 4 * g;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (pv0 + (uint32_t)i >= len) ra.v[i] = make_uint4(0u, 0u, 0u, 0u);
        }
        if (c * kChunk + wave * 16 < len) mchunk_step(ra, qf, a.scale, c, len, m, l, acc);
        if (c1 >= nchunk) break;
        load_mchunk(rs, row_bytes, min(c2, nchunk), ra);
        if (c1 * kChunk + wave * 16 < len) mchunk_step(rb, qf, a.scale, c1, len, m, l, acc);
    }
    const float lt = rows_sum(l);
    if (n < (uint32_t)G) {
        if (g == 0) {
            sh.wm[wave][n] = m;
            sh.wl[wave][n] = lt;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int t = 0; t < 8; ++t) sh.wacc[wave][n][32 * g + 8 * i + t] = acc[t][i];
    }
    attn_finish<G, XL, MS>(a, hot, sh, id, nsplit);
}

}  // namespace

// heads = q_heads | kv_heads << 16, shape = rows | xcds << 16 (eight leading parameters are
// preloaded)
#define GH_ATTN_PARAMS                                                                          \
    uint64_t q, uint64_t kc, uint64_t vc, uint64_t pos_ptr, uint32_t layer, uint32_t context,     \
        uint32_t heads, uint32_t shape, GhAttnArgs a
#define GH_ATTN_HOT \
    AttnHot{q, kc, vc, pos_ptr, layer, context, heads & 0xFFFFu, heads >> 16, shape & 0xFFFFu, shape >> 16}
GH_KERNEL __launch_bounds__(256) void gh_attn_g1(GH_ATTN_PARAMS) { attn_body<1, false>(a, GH_ATTN_HOT); }
GH_KERNEL __launch_bounds__(256) void gh_attn_g2(GH_ATTN_PARAMS) { attn_body<2, false>(a, GH_ATTN_HOT); }
GH_KERNEL __launch_bounds__(256) void gh_attn_mfma_g4(GH_ATTN_PARAMS) { attn_mfma_body<4, false>(a, GH_ATTN_HOT); }
GH_KERNEL __launch_bounds__(256) void gh_attn_mfma_g8(GH_ATTN_PARAMS) { attn_mfma_body<8, false>(a, GH_ATTN_HOT); }
// launches of at most 16 splits: the merge reads 16 slots instead of 32
GH_KERNEL __launch_bounds__(256) void gh_attn_mfma_g4_s16(GH_ATTN_PARAMS) {
    attn_mfma_body<4, false, 16>(a, GH_ATTN_HOT);
}
// the XCD-local forms (grid (xcds, splits, pair groups))
GH_KERNEL __launch_bounds__(256) void gh_attn_g1_x(GH_ATTN_PARAMS) { attn_body<1, true>(a, GH_ATTN_HOT); }
GH_KERNEL __launch_bounds__(256) void gh_attn_g2_x(GH_ATTN_PARAMS) { attn_body<2, true>(a, GH_ATTN_HOT); }
GH_KERNEL __launch_bounds__(256) void gh_attn_mfma_g4_x(GH_ATTN_PARAMS) { attn_mfma_body<4, true>(a, GH_ATTN_HOT); }
GH_KERNEL __launch_bounds__(256) void gh_attn_mfma_g8_x(GH_ATTN_PARAMS) { attn_mfma_body<8, true>(a, GH_ATTN_HOT); }
GH_KERNEL __launch_bounds__(256) void gh_attn_mfma_g4_s16_x(GH_ATTN_PARAMS) {
    attn_mfma_body<4, true, 16>(a, GH_ATTN_HOT);
}

// The XCD each workgroup runs on (HW_REG_XCC_ID bits 3:0), at out[linear workgroup id]: the
// host's start-up check of the dispatcher's workgroup-to-XCD rule.
GH_KERNEL __launch_bounds__(64) void gh_xcd_probe(uint64_t out, uint32_t gx, uint32_t gy) {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    if (threadIdx.x == 0) gh_gpw<uint32_t>(out)[blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z)] = v & 0xFu;
}

// ---------------------------------------------------------------------------------------------
// Causal GQA prefill attention on the matrix cores (flash attention, G = 4 query heads per kv
// head, head_dim = value_dim = 128).
//
// Grid (query blocks of 16·QT rows, kv heads), 256 threads; wave w owns query head 4·kvh + w
// for the block's rows, so every K/V tile staged in LDS serves all four heads. Per tile of 64
// key positions, with v_mfma_f32_16x16x32_f16 and FP32 accumulators:
//   S^T = K · Q^T   A = K rows (LDS), B = the wave's FP16 query rows (registers); the output
//                   layout gives each lane one query row (lane % 16) and four key positions
//                   per 16 x 16 tile, so the row's running max/sum stay in that lane;
//   O^T += V^T · P^T  P goes to the B operand straight from the S^T registers (a lane's key
//                   positions name its k-slots; V^T is read from LDS in the same slot order,
//                   which leaves the product unchanged). P is split into FP16 hi + lo parts
//                   (two MFMAs), so P·V carries FP32-level accuracy.
// Softmax in base 2: scores are scaled by scale·log2(e), p = 2^(s - m), rescale 2^(m_old - m).
// Rows: query r at position base + r attends positions 0..base + r (the reference's prefill,
// attention/mod.rs:582-725). Query blocks run heaviest (latest) first.
namespace {
typedef _Float16 ah8 __attribute__((ext_vector_type(8)));
typedef float af4 __attribute__((ext_vector_type(4)));

constexpr int kPK = 64;          // key positions per tile
// K and V tiles share one layout: [64 keys][128 dims] in 256-byte rows, the 32-byte block b of
// row r holding dims 16 (b ^ sw(r)) .. + 16, sw(r) = r mod 8. Measured with
// SQ_LDS_BANK_CONFLICT on gfx950 (a probe running each fragment read pattern alone): the K
// fragment reads (ds_read_b128: 16 consecutive rows x 2 chunks of one block per 32 lanes) and
// the V transposing reads (ds_read_b64_tr_b16: 16 consecutive rows x one block) are free of
// conflicts with sw(r) = r mod 8, and conflicted with (r / 2) mod 8 (half the LDS cycles),
// (r / 4) mod 8 or no swizzle.
__device__ __forceinline__ uint32_t kv_sw(uint32_t r) { return r & 7u; }
// offset in halves of dims 16·blk .. + 16 of row r
__device__ __forceinline__ uint32_t kv_at(uint32_t r, uint32_t blk) { return r * 128 + 16 * (blk ^ kv_sw(r)); }

#define GH_LDS __attribute__((address_space(3)))

// Stage keys t0 .. t0+63 of K and V straight into their tiles by LDS DMA (global_load_lds_dwordx4:
// lane i of a load lands at byte 16 i of its 1 KiB destination, four 256-byte rows): wave w
// loads rows 16 w .. 16 w + 15, lane i of load q the 16-byte chunk of row r = 16 w + 4 q + i / 16
// that belongs in slot i mod 16. Keys past kv_end (masked; their weight is 0) re-read key
// kv_end - 1, so every value in the tile is a finite cache value and no load leaves the range.
// The loads are issued from inline assembly: the compiler does not count them, so it adds no
// wait before the reads of the other tile buffer; the caller waits (vmcnt(0)) before the
// barrier that hands the tile over. (Untracked loads can only make the compiler's own waits
// stricter, and the tile loop issues no tracked global loads.)
__device__ __forceinline__ void kv_dma(const uint16_t* kc, const uint16_t* vc, uint32_t kv_row,
                                       uint32_t t0, uint32_t kv_end, _Float16* kt, _Float16* vt) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, sl = lane & 15u;
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
        const uint32_t r = 16 * wave + 4 * q + (lane >> 4);
        const uint32_t c = ((((sl >> 1) ^ kv_sw(r)) << 1) | (sl & 1u));  // the row's chunk for this slot
        const size_t src = (size_t)min(t0 + r, kv_end - 1) * kv_row + 8 * c;
        const uint32_t at = (16 * wave + 4 * q) * 128;
        const uint32_t dk = (uint32_t)(uintptr_t)(GH_LDS void*)(kt + at);
        const uint32_t dv = (uint32_t)(uintptr_t)(GH_LDS void*)(vt + at);
        asm volatile("global_load_lds_dwordx4 %0, off" ::"v"((uint64_t)(uintptr_t)(kc + src)),
                     "{m0}"(__builtin_amdgcn_readfirstlane(dk))
                     : "memory");
        asm volatile("global_load_lds_dwordx4 %0, off" ::"v"((uint64_t)(uintptr_t)(vc + src)),
                     "{m0}"(__builtin_amdgcn_readfirstlane(dv))
                     : "memory");
    }
}

// A fragment of V^T for O^T += V^T·P^T: output row m = dims 16 j + m, k-slots = keys key0 + 0..3
// (elements 0-3) and key0 + 16 + 0..3 (elements 4-7), read from the [key][dim] tile with two
// ds_read_b64_tr_b16. Within each 16-lane group that instruction gives lane i the halves
// (i mod 4) of the 8-byte rows that lanes 4k + i / 4 address (k = 0..3, in order); so lane fr
// addresses key key0 + fr / 4, dims 16 j + 4 (fr mod 4), and lane i receives dim 16 j + i at
// the four keys. Rows r and r + 16 share sw(r).
typedef short as4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ ah8 v_frag(const _Float16* vb, uint32_t key0, uint32_t j, uint32_t fr) {
    typedef GH_LDS as4* lds_as4;
    _Float16* p = (_Float16*)vb + kv_at(key0 + (fr >> 2), j) + 4 * (fr & 3u);
    const as4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_as4)p);
    const as4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_as4)(p + 16 * 128));
    const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
    return __builtin_bit_cast(ah8, make_uint4(ua.x, ua.y, ub.x, ub.y));
}

// Reductions over the four lanes l, l^16, l^32, l^48 (one query row's lane group) with the
// gfx950 row-swap moves: v_permlane16_swap pairs rows 0/1 and 2/3, v_permlane32_swap pairs the
// wave halves; each swap leaves both partners' values in the two registers, in the same order
// in every lane, so all four lanes end with bit-identical results.
__device__ __forceinline__ float xor_max(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xor_sum(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <bool B>
struct Flag {
    static constexpr bool value = B;
};
typedef float af2 __attribute__((ext_vector_type(2)));
typedef _Float16 ah2 __attribute__((ext_vector_type(2)));

template <int QT>  // query tiles of 16 rows per wave
__device__ __forceinline__ void attn_prefill_g4(const GhAttnArgs& a) {
    constexpr uint32_t kPQ = 16 * QT;  // query rows per workgroup
    __shared__ __attribute__((aligned(16))) _Float16 kt[2][kPK * 128];
    __shared__ __attribute__((aligned(16))) _Float16 vt[2][kPK * 128];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t nqb = (a.rows + kPQ - 1) / kPQ;
    // Work order: L = 0 is the heaviest (latest) query block. Workgroup k of the first half of
    // the grid takes L = k, workgroup k + T/2 takes L = T - 1 - k: with the grid dispatched
    // round-robin over the CUs and two workgroups resident per CU, the pair that shares a CU
    // carries one heavy and one light causal block instead of two equal ones.
    const uint32_t T = nqb * a.kv_heads, k = blockIdx.x + nqb * blockIdx.y, half = (T + 1) / 2;
    const uint32_t L = k < half ? k : T - 1 - (k - half);  // grid: (nqb, kv_heads)
    const uint32_t qb = nqb - 1 - L / a.kv_heads, kvh = L % a.kv_heads, h = kvh * 4 + wave;
    const uint32_t q0 = qb * kPQ;
    const uint32_t kv_end = a.base + min(q0 + kPQ, a.rows);  // keys 0 .. kv_end-1 are visible
    const uint32_t ntiles = (kv_end + kPK - 1) / kPK;
    const size_t kv_row = (size_t)a.kv_heads * 128;
    const size_t cache0 = (size_t)a.layer * a.context * kv_row + (size_t)kvh * 128;
    const uint16_t* kc = (const uint16_t*)a.kc + cache0;
    const uint16_t* vc = (const uint16_t*)a.vc + cache0;
    const uint32_t fr = lane & 15u, fg = lane >> 4;  // fragment row / lane group
    const float sl2 = a.scale * 1.4426950408889634f;  // scores in base-2 units

    // this wave's query rows as B operands: [q tile t][k step ks] = dims 32 ks + 8 fg .. + 8
    ah8 qf[QT][4];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        const uint32_t r = min(q0 + 16 * t + fr, a.rows - 1);
        const GH_GLOBAL uint4* qp = gh_gp<uint4>(a.q + (((uint64_t)r * a.q_heads + h) * 128 + 8 * fg) * 2);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qf[t][ks] = __builtin_bit_cast(ah8, qp[4 * ks]);
    }
    uint32_t qpos[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) qpos[t] = a.base + q0 + 16 * t + fr;

    af4 o[8][QT];
    float m[QT], l[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j][t] = af4{0.0f, 0.0f, 0.0f, 0.0f};
        m[t] = -__builtin_inff();
        l[t] = 0.0f;
    }

    const uint32_t kv_row32 = (uint32_t)kv_row;
    kv_dma(kc, vc, kv_row32, 0, kv_end, kt[0], vt[0]);
    // the query fragments are taken here, so the compiler settles their loads before the tile
    // loop (it does not see the explicit wait below) and puts no load wait inside the loop
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) asm volatile("" ::"v"(qf[t][ks]));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's DMA has landed
    __syncthreads();
    // Tiles whose last key is at or before the block's first query position need no causal
    // mask (nor do they hold the clamped duplicates past kv_end); only the diagonal ones do.
    const uint32_t first_pos = a.base + q0;
    auto step = [&](uint32_t tile, auto masked) {
        constexpr bool kMask = decltype(masked)::value;
        const uint32_t cur = tile & 1u, t0 = tile * kPK;
        const bool more = tile + 1 < ntiles;
        // the next tile goes into the other buffers, whose reads ended before the last barrier
        if (more) kv_dma(kc, vc, kv_row32, t0 + kPK, kv_end, kt[cur ^ 1u], vt[cur ^ 1u]);
        const _Float16* kb = kt[cur];
        const _Float16* vb = vt[cur];
        // S^T tiles: [key tile kk][q tile t], lane holds keys 16 kk + 4 fg + e of query fr
        af4 s[4][QT];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
            for (int t = 0; t < QT; ++t) s[kk][t] = af4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const ah8 kf = *(const ah8*)(kb + kv_at(16 * kk + fr, 2 * ks + (fg >> 1)) + 8 * (fg & 1u));
#pragma unroll
                for (int t = 0; t < QT; ++t)
                    s[kk][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[t][ks], s[kk][t], 0, 0, 0);
            }
        }
        // online softmax per query row (lane), P as FP16 hi/lo B operands in key-slot order
        ah8 ph[2][QT], pl[2][QT];  // [k step (keys 32 ks2 ..)][q tile]
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            float v[4][4];
            float mx = -__builtin_inff();
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[kk][e] = s[kk][t][e];
                    if constexpr (kMask)
                        if (t0 + 16 * kk + 4 * fg + e > qpos[t]) v[kk][e] = -__builtin_inff();
                    mx = fmaxf(mx, v[kk][e]);
                }
            // sl2 > 0, so the row max of the scaled scores is sl2 · (row max of the raw ones);
            // finite: key 0 is in tile 0. v_exp_f32 directly: weights below 2^-126 (flushed
            // to zero) are far below the FP32 accumulation error of the sums they enter.
            const float m_new = fmaxf(m[t], xor_max(mx) * sl2);
            const float f = __builtin_amdgcn_exp2f(m[t] - m_new);
            m[t] = m_new;
            float sum = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[kk][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(v[kk][e], sl2, -m_new));
                    sum += v[kk][e];
                }
            l[t] = l[t] * f + sum;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j][t] *= f;
#pragma unroll
            for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const af2 pv = {v[2 * ks2 + (e >> 2)][e & 3], v[2 * ks2 + (e >> 2)][(e & 3) + 1]};
                    const ah2 hi = __builtin_convertvector(pv, ah2);  // round to nearest even
                    const ah2 lo = __builtin_convertvector(pv - __builtin_convertvector(hi, af2), ah2);
                    ph[ks2][t][e] = hi[0];
                    ph[ks2][t][e + 1] = hi[1];
                    pl[ks2][t][e] = lo[0];
                    pl[ks2][t][e + 1] = lo[1];
                }
        }
        // O^T += V^T P^T: A = V^T rows (dims 16 j + fr), k-slots = keys 32 ks2 + {4 fg .. +3,
        // 16 + 4 fg .. +3}, the keys the lane's P values hold
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int ks2 = 0; ks2 < 2; ++ks2) {
                const ah8 vf = v_frag(vb, 32 * ks2 + 4 * fg, j, fr);
#pragma unroll
                for (int t = 0; t < QT; ++t) {
                    o[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph[ks2][t], o[j][t], 0, 0, 0);
                    o[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl[ks2][t], o[j][t], 0, 0, 0);
                }
            }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's DMA of the next tile has landed
        __syncthreads();  // every wave's has, and every read of this tile is done
    };
    uint32_t tile = 0;
    for (; tile < ntiles && tile * kPK + kPK - 1 <= first_pos; ++tile) step(tile, Flag<false>{});
    for (; tile < ntiles; ++tile) step(tile, Flag<true>{});
    // O^T tile (j, t): lane holds dims 16 j + 4 fg + e of query row q0 + 16 t + fr
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        const uint32_t r = q0 + 16 * t + fr;
        const float inv = 1.0f / xor_sum(l[t]);
        if (r >= a.rows) continue;
        GH_GLOBAL uint16_t* op = gh_gpw<uint16_t>(a.out) + ((size_t)r * a.q_heads + h) * 128 + 4 * fg;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t w0 = (uint32_t)gh_f2h(o[j][t][0] * inv) | ((uint32_t)gh_f2h(o[j][t][1] * inv) << 16);
            const uint32_t w1 = (uint32_t)gh_f2h(o[j][t][2] * inv) | ((uint32_t)gh_f2h(o[j][t][3] * inv) << 16);
            *(GH_GLOBAL uint2*)(op + 16 * j) = make_uint2(w0, w1);
        }
    }
}
}  // namespace

GH_KERNEL __launch_bounds__(256) void gh_attn_prefill_g4(GhAttnArgs a) { attn_prefill_g4<2>(a); }
// 16 query rows per workgroup: twice the workgroups, for row counts whose 32-row blocks leave
// CUs idle
GH_KERNEL __launch_bounds__(256) void gh_attn_prefill_g4_r16(GhAttnArgs a) { attn_prefill_g4<1>(a); }

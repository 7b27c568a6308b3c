// Decode/prefill glue: RMSNorm, YaRN RoPE, SiLU·up, residual add, KV append, argmax.
#include "gh_common.h"

// rmsnorm_x (backend/cpu/kernels/elementwise/normalization.rs:12-40): one 1024-thread
// workgroup per row, 4 consecutive FP32 values per thread per step, Σx² reduced with DPP and
// LDS, inverse = 1/sqrt(Σx²/dim + eps), out = f16((x*inverse)*w). dim % 4 == 0.
GH_KERNEL __launch_bounds__(256) void gh_rmsnorm_x(GhRmsnormArgs a) {
#pragma clang fp contract(off)
    const uint32_t row = blockIdx.x;
    if (row >= a.rows) return;
    const GH_GLOBAL float4* x = gh_gp<float4>(a.x + (uint64_t)row * a.dim * 4);
    const GH_GLOBAL uint2* w = gh_gp<uint2>(a.w);
    GH_GLOBAL uint2* out = gh_gpw<uint2>(a.out + (uint64_t)row * a.dim * 2);
    __shared__ float red[4];
    const float inverse = gh_rms_inverse_256(x, a.dim, a.eps, red);
    for (uint32_t i = threadIdx.x; i < (a.dim >> 2); i += 256) {
        const float4 v = x[i];
        const uint2 wv = w[i];
        const uint32_t o0 = gh_f2h(v.x * inverse * gh_h2f(wv.x & 0xFFFFu));
        const uint32_t o1 = gh_f2h(v.y * inverse * gh_h2f(wv.x >> 16));
        const uint32_t o2 = gh_f2h(v.z * inverse * gh_h2f(wv.y & 0xFFFFu));
        const uint32_t o3 = gh_f2h(v.w * inverse * gh_h2f(wv.y >> 16));
        out[i] = make_uint2(o0 | (o1 << 16), o2 | (o3 << 16));
    }
}

// rope_yarn (cpu/kernels/elementwise/rope.rs:14-39): adjacent pairs rotated by the per
// (position, pair) YaRN (cos, sin) table, then the role's post-scale; FP16 in place.
// One thread per (row, head, pair).
GH_KERNEL __launch_bounds__(256) void gh_rope(GhRopeArgs a) {
#pragma clang fp contract(off)
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t total = (size_t)a.rows * a.heads * a.pairs;
    if (t >= total) return;
    const uint32_t pair = (uint32_t)(t % a.pairs);
    const size_t rh = t / a.pairs;
    const uint32_t head = (uint32_t)(rh % a.heads);
    const uint32_t row = (uint32_t)(rh / a.heads);
    const uint32_t pos = (a.pos_ptr ? *(const uint32_t*)a.pos_ptr : 0u) + a.base + row;
    const float2 cs = ((const float2*)a.table)[(size_t)pos * a.pairs + pair];
    const float scale = a.post ? ((const float*)a.post)[pos] : 1.0f;
    uint32_t* p = (uint32_t*)((uint16_t*)a.x + ((size_t)row * a.heads + head) * a.head_dim + 2 * pair);
    const uint32_t v = *p;
    const float x0 = gh_h2f(v & 0xFFFFu), x1 = gh_h2f(v >> 16);
    const float y0 = (x0 * cs.x - x1 * cs.y) * scale;
    const float y1 = (x0 * cs.y + x1 * cs.x) * scale;
    *p = (uint32_t)gh_f2h(y0) | ((uint32_t)gh_f2h(y1) << 16);
}

// silu_mul (cpu/kernels/elementwise/activation.rs:16-29): out = f16(f16(g/(1+exp(-g))) * u).
GH_KERNEL __launch_bounds__(256) void gh_silu_mul(GhEltArgs a) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n) return;
    ((uint16_t*)a.out)[i] = gh_silu_mul_h(((const uint16_t*)a.a)[i], ((const uint16_t*)a.b)[i]);
}

// residual_add (cpu/kernels/elementwise/residual.rs:12-22): x(f32) += f16 y.
GH_KERNEL __launch_bounds__(256) void gh_residual_add(GhEltArgs a) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n) return;
    float* x = (float*)a.out;
    x[i] = x[i] + gh_h2f(((const uint16_t*)a.b)[i]);
}

// Fill n u32 words at `out` with the value `pad`: a clear that a captured graph records as a
// kernel node, not a memset node.
GH_KERNEL __launch_bounds__(256) void gh_fill_u32(GhEltArgs a) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) gh_gpw<uint32_t>(a.out)[i] = a.pad;
}

// A plain streaming read, for measurement (no counterpart in the reference): the n 16-byte
// chunks at `a`, read with nontemporal loads (as the decode GEMVs read weights), four in
// flight per thread; thread i of the pad x 256 threads takes chunks i, i + 256 pad, ... . The
// chunks are XOR-folded and the fold is stored only if it equals 0xFFFFFFFF, so the loads stay
// live while the kernel writes (almost) nothing: its duration is what a pure weight stream of
// that size and launch shape takes on this chip.
GH_KERNEL __launch_bounds__(256) void gh_stream_probe(GhEltArgs a) {
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    const GH_GLOBAL u4v* src = (const GH_GLOBAL u4v*)a.a;
    const uint32_t stride = a.pad * 256;
    uint32_t i = blockIdx.x * 256 + threadIdx.x, acc = 0;
    for (; i + 3 * stride < a.n; i += 4 * stride) {
        u4v v[4];
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) v[k] = __builtin_nontemporal_load(src + i + k * stride);
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; i < a.n; i += stride) {
        const u4v v = __builtin_nontemporal_load(src + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0xFFFFFFFFu) gh_gpw<uint32_t>(a.out)[0] = blockIdx.x;
}

// kv_write f16 (cpu/kernels/attention/write.rs:50-63): raw FP16 copy of K and V into the
// caches at element offsets; with pos_ptr the offsets advance by stride * (*pos_ptr).
GH_KERNEL __launch_bounds__(256) void gh_kv_write(GhKvWriteArgs a) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t pos = a.pos_ptr ? *(const uint32_t*)a.pos_ptr : 0u;
    if (i < a.k_count)
        ((uint16_t*)a.kc)[a.k_off + pos * a.k_stride + i] = ((const uint16_t*)a.k)[i];
    if (i < a.v_count)
        ((uint16_t*)a.vc)[a.v_off + pos * a.v_stride + i] = ((const uint16_t*)a.v)[i];
}

// argmax_f32 (backend/cpu/readback.rs:45-55): first index of the maximum, NaN never wins;
// if no logit exceeds -inf the answer is 0. Stage 1: one (value, index) per workgroup.
__device__ __forceinline__ void argmax_merge(float& v, uint32_t& i, float ov, uint32_t oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__device__ __forceinline__ void argmax_block(float& v, uint32_t& i) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const uint32_t oi = __shfl_xor(i, off, 64);
        argmax_merge(v, i, ov, oi);
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = v;
        si[threadIdx.x >> 6] = i;
    }
    __syncthreads();
    v = sv[0];
    i = si[0];
    for (int w = 1; w < 4; ++w) argmax_merge(v, i, sv[w], si[w]);
}

GH_KERNEL __launch_bounds__(256) void gh_argmax_partial(GhArgmaxArgs a) {
    const float* l = (const float*)a.logits;
    float v = -__builtin_inff();
    uint32_t idx = 0xFFFFFFFFu;
    const uint32_t stride = a.blocks * 256;
    for (uint32_t j = blockIdx.x * 256 + threadIdx.x; j < a.n; j += stride) {
        const float x = l[j];
        if (x > v) {  // strict: the first (lowest) index of this thread's subset wins
            v = x;
            idx = j;
        }
    }
    argmax_block(v, idx);
    if (threadIdx.x == 0) {
        ((float*)a.part_v)[blockIdx.x] = v;
        ((uint32_t*)a.part_i)[blockIdx.x] = idx;
    }
}

GH_KERNEL __launch_bounds__(256) void gh_argmax_final(GhArgmaxArgs a) {
    float v = -__builtin_inff();
    uint32_t idx = 0xFFFFFFFFu;
    for (uint32_t j = threadIdx.x; j < a.blocks; j += 256)
        argmax_merge(v, idx, ((const float*)a.part_v)[j], ((const uint32_t*)a.part_i)[j]);
    argmax_block(v, idx);
    if (threadIdx.x == 0) {
        const uint32_t r = (idx == 0xFFFFFFFFu) ? 0u : idx;
        *(uint32_t*)a.out = r;
        if (a.out2) *(uint32_t*)a.out2 = r;
        if (a.step_scalars) {  // end of a replayed greedy decode step
            uint32_t* s = (uint32_t*)a.step_scalars;
            const uint32_t pos = s[0];
            ((uint32_t*)a.step_history)[pos] = r;
            s[1] = r;
            s[0] = pos + 1;
        }
    }
}

// ---- top-k: read_topk (backend/contract.rs:303-318, cpu/readback.rs:59-69) on the device ----
// The min(k, n) largest logits under (logit descending by f32 total order, i.e.
// f32::total_cmp, then index ascending). Each logit becomes one 64-bit key that sorts
// ascending in exactly that order:
//   key = (~ord(bits) << 32) | index,   ord(b) = b ^ (b >> 31 ? 0xFFFFFFFF : 0x80000000),
// ord mapping the total order of f32 bit patterns (-NaN < -inf < ... < -0 < +0 < ... < +inf <
// +NaN) onto unsigned order. The all-ones key pads short stripes and sorts after every real
// key. Both kernels sort with bitonic networks in LDS.
constexpr uint32_t kTopkChunk = 2048;  // keys sorted per step of the partial pass
constexpr uint32_t kTopkWidth = 128;   // largest list width (k <= 128 on the device path)
constexpr uint32_t kTopkStripes = 128; // largest stripe count

__device__ __forceinline__ uint64_t topk_key(uint32_t bits, uint32_t idx) {
    const uint32_t ord = bits ^ ((bits >> 31) ? 0xFFFFFFFFu : 0x80000000u);
    return ((uint64_t)~ord << 32) | idx;
}

// Ascending bitonic sort of s[0, n), n a power of 2, by the whole workgroup.
template <uint32_t NT>
__device__ void topk_sort(uint64_t* s, uint32_t n) {
    for (uint32_t size = 2; size <= n; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (uint32_t t = threadIdx.x; t < n / 2; t += NT) {
                const uint32_t i = 2 * t - (t & (stride - 1)), j = i + stride;
                const uint64_t x = s[i], y = s[j];
                if ((x > y) == ((i & size) == 0)) {
                    s[i] = y;
                    s[j] = x;
                }
            }
        }
    }
    __syncthreads();
}

// `lists` independent sorted lists of width w at s + l * w: sorts each bitonic list ascending
// (compare-exchanges at strides w/2 .. 1, all ascending).
template <uint32_t NT>
__device__ void topk_bitonic_merge(uint64_t* s, uint32_t lists, uint32_t w) {
    for (uint32_t stride = w >> 1; stride > 0; stride >>= 1) {
        __syncthreads();
        for (uint32_t t = threadIdx.x; t < lists * (w / 2); t += NT) {
            const uint32_t l = t / (w / 2), u = t % (w / 2);
            const uint32_t i = l * w + 2 * u - (u & (stride - 1)), j = i + stride;
            const uint64_t x = s[i], y = s[j];
            if (x > y) {
                s[i] = y;
                s[j] = x;
            }
        }
    }
    __syncthreads();
}

GH_KERNEL __launch_bounds__(512) void gh_topk_partial(GhTopkArgs a) {
    __shared__ uint64_t s[kTopkChunk];
    __shared__ uint64_t r[kTopkWidth];
    const uint32_t w = a.width;
    const uint64_t b0 = (uint64_t)blockIdx.x * a.per, e = min((uint64_t)a.n, b0 + a.per);
    const uint32_t* bits = (const uint32_t*)a.logits;
    for (uint32_t t = threadIdx.x; t < w; t += 512) r[t] = ~0ull;
    for (uint64_t c = b0; c < e; c += kTopkChunk) {
        __syncthreads();
        for (uint32_t t = threadIdx.x; t < kTopkChunk; t += 512)
            s[t] = c + t < e ? topk_key(bits[c + t], (uint32_t)(c + t)) : ~0ull;
        topk_sort<512>(s, kTopkChunk);
        // the w smallest of (r, s[0, w)): r[i] = min(r[i], s[w - 1 - i]) is bitonic; sort it
        for (uint32_t t = threadIdx.x; t < w; t += 512) r[t] = min(r[t], s[w - 1 - t]);
        topk_bitonic_merge<512>(r, 1, w);
    }
    for (uint32_t t = threadIdx.x; t < w; t += 512)
        ((uint64_t*)a.part)[(size_t)blockIdx.x * w + t] = r[t];
}

// One workgroup: the stripes' lists (padded to a power of 2 with all-ones lists) are merged
// pairwise, halving the list count per level, keeping the w smallest keys of each pair.
GH_KERNEL __launch_bounds__(1024) void gh_topk_final(GhTopkArgs a) {
    __shared__ uint64_t s[kTopkStripes * kTopkWidth];
    const uint32_t w = a.width;
    uint32_t lists = 1;
    while (lists < a.stripes) lists <<= 1;
    for (uint32_t t = threadIdx.x; t < lists * w; t += 1024)
        s[t] = t < a.stripes * w ? ((const uint64_t*)a.part)[t] : ~0ull;
    for (uint32_t half = lists >> 1; half > 0; half >>= 1) {
        __syncthreads();
        // list l (< half) takes the w smallest of itself and list l + half
        for (uint32_t t = threadIdx.x; t < half * w; t += 1024) {
            const uint32_t l = t / w, i = t % w;
            s[t] = min(s[t], s[(l + half) * w + (w - 1 - i)]);
        }
        topk_bitonic_merge<1024>(s, half, w);
    }
    for (uint32_t t = threadIdx.x; t < a.k; t += 1024) {
        const uint64_t key = s[t];
        const uint32_t ord = ~(uint32_t)(key >> 32);
        ((uint32_t*)a.out)[t] = (uint32_t)key;
        ((uint32_t*)a.out)[a.k + t] = ord ^ ((ord >> 31) ? 0x80000000u : 0xFFFFFFFFu);
    }
}

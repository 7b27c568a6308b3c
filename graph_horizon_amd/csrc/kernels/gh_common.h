// Device helpers shared by the gfx950 kernels.
#ifndef GH_COMMON_H
#define GH_COMMON_H
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gh_kargs.h"

typedef _Float16 gh_h2 __attribute__((ext_vector_type(2)));

#define GH_KERNEL extern "C" __global__

__device__ __forceinline__ float gh_h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ uint16_t gh_f2h(float v) {
    // v_cvt_f16_f32 under the default round-to-nearest-even mode (f16 denormals preserved).
    // A NaN keeps its sign and the top bits of its payload, quieted — as the reference's
    // buffer writes narrow through F16C vcvtps2ph (backend/cpu/f16.rs:86-102).
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}

__device__ __forceinline__ gh_h2 gh_as_h2(uint32_t v) { return __builtin_bit_cast(gh_h2, v); }

// D = a.lo*b.lo + a.hi*b.hi + c in FP32 (v_dot2_f32_f16).
__device__ __forceinline__ float gh_dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(gh_as_h2(a), gh_as_h2(b), c, false);
}

// Workgroup barrier that orders LDS accesses only: unlike __syncthreads() (whose workgroup
// fence waits for every outstanding global load and store, vmcnt(0)), global accesses stay
// in flight across it.
__device__ __forceinline__ void gh_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}


#define GH_GLOBAL __attribute__((address_space(1)))

// Global-address-space views of a device address (global_load/global_store, not flat).
template <class T>
__device__ __forceinline__ const GH_GLOBAL T* gh_gp(uint64_t a) {
    return (const GH_GLOBAL T*)a;
}
template <class T>
__device__ __forceinline__ GH_GLOBAL T* gh_gpw(uint64_t a) {
    return (GH_GLOBAL T*)a;
}

#define GH_DPP(v, ctrl, rmask) \
    __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, rmask, 0xF, false))

// Sum across a wavefront with DPP (quad perms, half-row/row mirrors, row broadcasts); the
// total lands in lanes 48..63 (read it from lane 63).
__device__ __forceinline__ float gh_wave_sum63(float v) {
    v += GH_DPP(v, 0xB1, 0xF);   // quad_perm [1,0,3,2]
    v += GH_DPP(v, 0x4E, 0xF);   // quad_perm [2,3,0,1]
    v += GH_DPP(v, 0x141, 0xF);  // row_half_mirror
    v += GH_DPP(v, 0x140, 0xF);  // row_mirror
    v += GH_DPP(v, 0x142, 0xA);  // row_bcast:15 into rows 1 and 3
    v += GH_DPP(v, 0x143, 0xC);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Maximum across a wavefront with the same DPP steps (lanes a step does not write keep their
// own value); the maximum lands in lane 63.
#define GH_DPP_KEEP(v, ctrl, rmask) \
    __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), ctrl, rmask, 0xF, false))
__device__ __forceinline__ float gh_wave_max63(float v) {
    v = fmaxf(v, GH_DPP_KEEP(v, 0xB1, 0xF));
    v = fmaxf(v, GH_DPP_KEEP(v, 0x4E, 0xF));
    v = fmaxf(v, GH_DPP_KEEP(v, 0x141, 0xF));
    v = fmaxf(v, GH_DPP_KEEP(v, 0x140, 0xF));
    v = fmaxf(v, GH_DPP_KEEP(v, 0x142, 0xA));
    v = fmaxf(v, GH_DPP_KEEP(v, 0x143, 0xC));
    return v;
}

__device__ __forceinline__ float gh_lane63(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum / maximum across the 64 lanes of a wavefront, returned to every lane (DPP steps, then
// lane 63 read into a scalar: no LDS round trips, unlike lane shuffles through ds_bpermute).
__device__ __forceinline__ float gh_wave_sum(float v) { return gh_lane63(gh_wave_sum63(v)); }
__device__ __forceinline__ float gh_wave_max(float v) { return gh_lane63(gh_wave_max63(v)); }

// silu_mul of one FP16 gate/up pair (cpu/kernels/elementwise/activation.rs:16-29):
// f16(f16(g / (1 + e^-g)) · u) in FP32, contraction off.
__device__ __forceinline__ uint16_t gh_silu_mul_h(uint32_t g16, uint32_t u16) {
#pragma clang fp contract(off)
    const float g = gh_h2f(g16), u = gh_h2f(u16);
    const float silu = g / (1.0f + expf(-g));
    return gh_f2h(gh_h2f(gh_f2h(silu)) * u);
}

// RMSNorm scale of one FP32 row over a 256-thread workgroup, in one fixed order (each thread
// sums its float4 chunks tid, tid + 256, ... as (x²+y²)+(z²+w²); DPP wave sums; the four wave
// sums added in wave order), so every kernel that uses it gets the same bits:
// 1 / sqrt(Σx²/dim + eps) (normalization.rs:12-40). `red` is 4 floats of LDS; `s` is the
// thread's own partial. Ends with a workgroup barrier.
__device__ __forceinline__ float gh_rms_add(float s, const float4& v) {
#pragma clang fp contract(off)
    return s + ((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w));
}

__device__ __forceinline__ float gh_rms_finish_256(float s, uint32_t dim, float eps, float* red) {
#pragma clang fp contract(off)
    s = gh_wave_sum63(s);
    if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float sum = ((red[0] + red[1]) + red[2]) + red[3];
    return 1.0f / __builtin_sqrtf(sum / (float)dim + eps);
}

// Σx² order: thread t adds the float4 chunks of the 16-value items j = t, t + 256, ... (chunks
// 4j .. 4j + 3 in turn), then the wave sums and the four waves' sums in order — the order the
// fused RMSNorm GEMVs use, so both produce the same inverse.
__device__ __forceinline__ float gh_rms_inverse_256(const __attribute__((address_space(1))) float4* x,
                                                   uint32_t dim, float eps, float* red) {
    float s = 0.0f;
    const uint32_t n4 = dim >> 2;
    for (uint32_t j = threadIdx.x; 4 * j < n4; j += 256)
        for (uint32_t q = 0; q < 4 && 4 * j + q < n4; ++q) s = gh_rms_add(s, x[4 * j + q]);
    return gh_rms_finish_256(s, dim, eps, red);
}

// get_scale_min_k4 on the 12 scale bytes held in bytes 4..15 of the Q4_K header chunk
// (backend/cpu/dequant.rs:78-89): 6-bit (sc, mn) of sub-block j.
// Branch-free (j differs across the lanes of a wave): the scale bytes sit in hd.y (scales[0..3]),
// hd.z ([4..7]) and hd.w ([8..11]); sub-block j and j + 4 use byte j & 3 of each word, so three
// shifts by 8·(j & 3) serve both forms and a mask selects one.
__device__ __forceinline__ void gh_q4k_scale_min(const uint4& hd, uint32_t j, uint32_t& sc,
                                                 uint32_t& mn) {
    const uint32_t sh = (j & 3u) * 8u;
    const uint32_t ys = hd.y >> sh, zs = hd.z >> sh, ws = hd.w >> sh;
    const uint32_t hi = 0u - ((j >> 2) & 1u);  // all ones for j >= 4
    sc = ((ys & 63u) & ~hi) | (((ws & 15u) | ((ys >> 2) & 48u)) & hi);
    mn = ((zs & 63u) & ~hi) | ((((ws >> 4) & 15u) | ((zs >> 2) & 48u)) & hi);
}

#endif

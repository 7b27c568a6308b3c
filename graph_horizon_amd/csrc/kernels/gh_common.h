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
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}

__device__ __forceinline__ gh_h2 gh_as_h2(uint32_t v) { return __builtin_bit_cast(gh_h2, v); }

// D = a.lo*b.lo + a.hi*b.hi + c in FP32 (v_dot2_f32_f16).
__device__ __forceinline__ float gh_dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(gh_as_h2(a), gh_as_h2(b), c, false);
}

// Sum across the 64 lanes of a wavefront (every lane receives the total).
__device__ __forceinline__ float gh_wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float gh_wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Byte `i` (runtime, 0..15) of a 16-byte register block.
__device__ __forceinline__ uint32_t gh_byte(const uint4& v, uint32_t i) {
    uint32_t w = (i < 4) ? v.x : (i < 8) ? v.y : (i < 12) ? v.z : v.w;
    return (w >> ((i & 3) * 8)) & 0xFFu;
}

// get_scale_min_k4 on the 12 scale bytes held in bytes 4..15 of the Q4_K header chunk
// (backend/cpu/dequant.rs:78-89): 6-bit (sc, mn) of sub-block j.
__device__ __forceinline__ void gh_q4k_scale_min(const uint4& hd, uint32_t j, uint32_t& sc,
                                                 uint32_t& mn) {
    if (j < 4) {
        sc = gh_byte(hd, 4 + j) & 63u;
        mn = gh_byte(hd, 8 + j) & 63u;
    } else {
        uint32_t hi = gh_byte(hd, 8 + j);
        uint32_t lo = gh_byte(hd, j);
        sc = (hi & 0xFu) | ((lo >> 6) << 4);
        mn = (hi >> 4) | ((gh_byte(hd, 4 + j) >> 6) << 4);
    }
}

#endif

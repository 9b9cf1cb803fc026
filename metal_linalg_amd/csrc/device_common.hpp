// Device helpers shared by the kernels: lane-group reductions within a
// wave64, the non-finite test and the quiet-NaN fill value.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

namespace mla {

// The quiet NaN the reference writes for a non-finite matrix (0x7FC00000).
__device__ __forceinline__ float qnan() { return __uint_as_float(0x7FC00000u); }

// |v| <= FLT_MAX fails for NaN and for the infinities (the reference's scan,
// src/metal_runtime.mm:161-162).
__device__ __forceinline__ bool finite_f(float v) { return fabsf(v) <= FLT_MAX; }

// Sum, max and or over an aligned group of G lanes (G a power of two <= 64),
// the result on every lane of the group.
template <int G>
__device__ __forceinline__ float group_sum(float x) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) x += __shfl_xor(x, off, G);
    return x;
}

template <int G>
__device__ __forceinline__ float group_max(float x) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, G));
    return x;
}

template <int G>
__device__ __forceinline__ int group_or(int x) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) x |= __shfl_xor(x, off, G);
    return x;
}

// DPP sums within a wave64 (row = 16 lanes): quad_sum leaves every lane of
// each group of 4 with the group's sum, half_row_sum groups of 8, row_sum
// rows of 16; wave_sum returns the wave's sum (uniform, from lane 63 after
// the row_bcast15 / row_bcast31 steps).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float quad_sum(float v) {
    v = dpp_add<0xB1>(v);      // quad_perm [1,0,3,2]
    return dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
}

__device__ __forceinline__ float half_row_sum(float v) { return dpp_add<0x141>(quad_sum(v)); }   // row_half_mirror

__device__ __forceinline__ float dpp_row_sum(float v) { return dpp_add<0x140>(half_row_sum(v)); }   // row_mirror

__device__ __forceinline__ float wave_sum_f(float v) {
    v = dpp_row_sum(v);
    v = dpp_add<0x142, 0xa>(v);   // row_bcast15 into rows 1 and 3
    v = dpp_add<0x143, 0xc>(v);   // row_bcast31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over an aligned group of G lanes (G = 8, 16, 32 or 64) on every lane of
// the group, by DPP (one cross-lane permute for G = 32).
template <int G>
__device__ __forceinline__ float group_sum_dpp(float v) {
    if constexpr (G == 64) return wave_sum_f(v);
    else if constexpr (G == 32) {
        v = dpp_row_sum(v);
        return v + __shfl_xor(v, 16, 32);
    } else if constexpr (G == 16) return dpp_row_sum(v);
    else if constexpr (G == 8) return half_row_sum(v);
    else return group_sum<G>(v);
}

// Power-of-two exponent e with amax * 2^-e in [0.5, 1) (frexp's), 0 for a
// zero or non-finite amax: the reference's scaled_input rule
// (src/metal_runtime.mm:179-215).
__device__ __forceinline__ int scale_exponent(float amax) {
    if (!(amax > 0.0f) || !(amax <= FLT_MAX)) return 0;
    int e = 0;
    (void)frexpf(amax, &e);
    return e;
}

// A reproducible pseudo-random value in (-1, 1) from two integers (an
// integer hash: xor-shift-multiply rounds).  Start vectors of inverse
// iteration.
__device__ __forceinline__ float hash_uniform(unsigned a, unsigned b) {
    unsigned x = a * 0x9E3779B1u ^ (b + 0x7F4A7C15u) * 0x85EBCA77u;
    x ^= x >> 15;
    x *= 0x2C1B3C6Du;
    x ^= x >> 12;
    x *= 0x297A2D39u;
    x ^= x >> 15;
    return (float)(x >> 8) * (2.0f / 16777216.0f) - 1.0f;
}

// 1/x: the hardware estimate (about 1 ulp) refined by one Newton step.
__device__ __forceinline__ float rcp_refined(float x) {
    const float y = __builtin_amdgcn_rcpf(x);
    return fmaf(y, fmaf(-x, y, 1.0f), y);
}

// A wave-level fence for LDS traffic between lanes of one wavefront: the
// kernels that use it launch one wave per workgroup.
__device__ __forceinline__ void wave_lds_sync() { __syncthreads(); }

}  // namespace mla

/* Shared device helpers for the gfx950 kernels (wave64, CDNA4). */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../qw_kernel_args.h"

typedef uint16_t u16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define QW_KERNEL extern "C" __global__

__device__ __forceinline__ float bf2f(u16 b) {
    return __uint_as_float((uint32_t)b << 16);
}

/* Round-to-nearest-even to bf16 (v_cvt_pk_bf16_f32): for finite inputs,
 * subnormals included, the same rounding as the reference's
 * h3_f32_to_bf16 (h3_shaders.metal:15: bias 0x7fff + lsb, then
 * truncate). */
typedef float qw_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 qw_b2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(qw_f2{lo, hi}, qw_b2));
}
__device__ __forceinline__ u16 f2bf(float f) { return (u16)pack_bf(f, 0.0f); }

__device__ __forceinline__ u16 f2bf_trunc(float f) {
    return (u16)(__float_as_uint(f) >> 16);
}

/* Low/high bf16 halves of a packed 32-bit word. */
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

/* Sum over each 16-lane row of the wave, in every lane of the row: adds of
 * the row rotated by 8, 4, 2 and 1 lanes (DPP row_ror: VALU, not the LDS
 * crossbar a shuffle uses). The same bits as the xor-shuffle tree over
 * 8, 4, 2, 1: after each step the partial sums repeat with that step's
 * period, so lane i + n (mod 16) holds what lane i ^ n would, and every
 * add pairs the same two operands. */
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xF, 0xF, false));
    return v;
}

/* The per-head RMS-norm factor 1 / sqrt(mean of squares + eps) as the
 * reference's kernel takes it (h3_shaders.metal:4323, Metal rsqrt): the
 * hardware reciprocal square root, not a correctly rounded divide of a
 * correctly rounded square root. */
__device__ __forceinline__ float head_rms_inv(float sum_sq, float eps) {
    return __builtin_amdgcn_rsqf(sum_sq * (1.0f / 128.0f) + eps);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

/* Block-wide sum; red must hold blockDim.x / 64 floats. Result in all lanes. */
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int waves = (blockDim.x + 63) >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < waves; i++) s += red[i];
    return s;
}

/* h3_shaders.metal:3385-3408 (approximate = 1): GELU with the tanh form,
 * saturating outside |inner| < 10. Evaluated through the identity
 * 0.5 (1 + tanh u) = 1 / (1 + e^(-2u)): one v_exp_f32 and one v_rcp_f32,
 * no cancellation for negative u (the 1 + tanh form loses bits there). */
__device__ __forceinline__ float gelu_tanh_f(float v) {
    /* x = -2 u log2(e) = v (C1 + C2 v^2); the reference's saturation
     * u <= -10 (result +0) is x >= 28.85...; for u >= 10, 1 + 2^x rounds to
     * 1 and the result is v exactly */
    const float C1 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
    const float C2 = C1 * 0.044715f;
    const float x = v * __builtin_fmaf(v * v, C2, C1);
    const float y = v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x));
    return x >= 28.853900817779268f ? 0.0f : y;
}

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

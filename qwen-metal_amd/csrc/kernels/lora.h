/* LoRA weight fusion (qwen_dit.m:535-1010): W' = RNE_bf16(fp32(W) +
 * sum_t scale_t * (B_t @ A_t)) over the terms that cover each row, in term
 * order, with one rounding. A term's product is fp32: the rank sum
 * accumulated with fma, then multiplied by its scale and added to the
 * running fp32 sum, the operation order of the reference's
 * sgemm(alpha = scale) plus accumulate. */
#pragma once
#include "common.h"

#define LORA_TILE 64 /* output rows and columns per workgroup */

QW_KERNEL void __launch_bounds__(256) qw_lora_fuse_bf16(qw_lora_args a) {
#pragma clang fp contract(off)
    __shared__ float bs[LORA_TILE][QW_LORA_MAX_RANK + 1]; /* B rows of the tile */
    __shared__ float as[QW_LORA_MAX_RANK][LORA_TILE + 4];   /* A columns of the tile */
    const uint32_t tid = threadIdx.x;
    const uint32_t r0 = blockIdx.y * LORA_TILE, c0 = blockIdx.x * LORA_TILE;
    const uint32_t tr = (tid / 16) * 4, tc = (tid % 16) * 4; /* this thread's 4 x 4 */
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t r = r0 + tr + i, c = c0 + tc + j;
            acc[i][j] = r < a.rows && c < a.cols ? bf2f(a.base[(size_t)r * a.cols + c]) : 0.0f;
        }
    for (uint32_t t = 0; t < a.nterms; t++) {
        const qw_lora_term T = a.terms[t];
        /* tile rows outside this term's segment take no contribution */
        if (r0 + LORA_TILE <= T.row0 || r0 >= T.row0 + T.rows) continue;
        __syncthreads(); /* the previous term's LDS reads are done */
        for (uint32_t e = tid; e < LORA_TILE * T.rank; e += 256) {
            const uint32_t i = e / T.rank, k = e % T.rank, r = r0 + i;
            bs[i][k] = r >= T.row0 && r < T.row0 + T.rows
                           ? bf2f(T.b[(size_t)(r - T.row0) * T.rank + k]) : 0.0f;
        }
        for (uint32_t e = tid; e < LORA_TILE * T.rank; e += 256) {
            const uint32_t k = e / LORA_TILE, j = e % LORA_TILE, c = c0 + j;
            as[k][j] = c < a.cols ? bf2f(T.a[(size_t)k * a.cols + c]) : 0.0f;
        }
        __syncthreads();
        float d[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) d[i][j] = 0.0f;
        for (uint32_t k = 0; k < T.rank; k++)
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    d[i][j] = __builtin_fmaf(bs[tr + i][k], as[k][tc + j], d[i][j]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t r = r0 + tr + i;
            if (r < T.row0 || r >= T.row0 + T.rows) continue;
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] += T.scale * d[i][j];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t r = r0 + tr + i, c = c0 + tc + j;
            if (r < a.rows && c < a.cols) a.out[(size_t)r * a.cols + c] = f2bf(acc[i][j]);
        }
}

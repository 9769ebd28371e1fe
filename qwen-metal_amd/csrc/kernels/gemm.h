/* bf16 / int8-weight GEMM on CDNA4 matrix cores:
 *   out[m, n] = epilogue( sum_k A[m, k] * W[n, k] )
 * A bf16 row-major (row stride lda), W in the checkpoint's native [out, in]
 * layout (bf16, or int8 with one fp32 scale per output row), fp32
 * accumulation in v_mfma_f32_32x32x16_bf16.
 *
 * Tiling: 256 x 256 x 64 macro-tile per workgroup of 4 waves (2 x 2, each
 * wave 128 x 128 = 4 x 4 MFMA blocks of 32 x 32, 256 fp32 accumulators per
 * lane). A and W tiles are staged through LDS, double-buffered (2 x 64 KB),
 * with the next K-slice's global loads in flight while the current one is
 * multiplied. LDS rows are 128 B; 16-byte chunks are XOR-swizzled by
 * (row / 2) % 8 so the 32 rows one MFMA operand read touches spread over
 * all banks. int8 weights are widened to bf16 (exact for |q| <= 127) on the
 * way into LDS, and the per-row scale multiplies the fp32 sum in the
 * epilogue, so the contraction equals the dequantised product.
 *
 * Tile order: workgroup ids are dealt round-robin to the 8 XCDs; the id is
 * remapped so each XCD owns a contiguous range of tiles, walked in groups
 * of 8 tile-rows, keeping the A panels and W panels an XCD touches hot in
 * its own L2. */
#pragma once
#include "common.h"

#define GBM 256
#define GBN 256
#define GBK 64
#define G_LDS_BUF 65536 /* A (32 KB) + W (32 KB) per stage */

__device__ __forceinline__ uint32_t g_swz(uint32_t row, uint32_t chunk) {
    return row * 128u + ((chunk ^ ((row >> 1) & 7u)) << 4);
}

/* int8 x16 -> bf16 x16 (exact), as two 16-byte LDS chunks. */
__device__ __forceinline__ void i8x16_to_bf16(u32x4 q, u32x4 &lo, u32x4 &hi) {
    uint32_t o[8];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        int32_t x = (int32_t)q[w];
        float f0 = (float)((x << 24) >> 24);
        float f1 = (float)((x << 16) >> 24);
        float f2 = (float)((x << 8) >> 24);
        float f3 = (float)(x >> 24);
        o[2 * w] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
        o[2 * w + 1] = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xffff0000u);
    }
    lo = u32x4{o[0], o[1], o[2], o[3]};
    hi = u32x4{o[4], o[5], o[6], o[7]};
}

template <int EPI, int INT8>
__device__ __forceinline__ void qw_gemm_impl(const qw_gemm_args &a, unsigned char *lds) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t h = lane >> 5, i32 = lane & 31;

    /* ---- tile id -> (tm, tn), XCD-contiguous, grouped by 8 tile-rows ---- */
    const uint32_t nt = a.tiles_m * a.tiles_n;
    uint32_t pid = blockIdx.x;
    if ((nt & 7u) == 0) pid = (pid & 7u) * (nt >> 3) + (pid >> 3);
    const uint32_t G = 8;
    const uint32_t per_group = G * a.tiles_n;
    const uint32_t first_m = (pid / per_group) * G;
    const uint32_t gsize = min(a.tiles_m - first_m, G);
    const uint32_t inner = pid % per_group;
    const uint32_t tm = first_m + inner % gsize, tn = inner / gsize;
    const uint32_t m0 = tm * GBM, n0 = tn * GBN;

    /* ---- global load coordinates (row-clamped at the edges) ------------- */
    const u16 *A = (const u16 *)a.a;
    const uint32_t ac = tid & 7, ar = tid >> 3; /* A: 8 chunks x 32 rows per pass */
    uint32_t a_off[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t r = min(m0 + ar + 32 * j, a.m - 1);
        a_off[j] = r * a.lda + ac * 8;
    }
    constexpr int WLD = INT8 ? 4 : 8;
    const uint32_t wc = INT8 ? (tid & 3) : (tid & 7);
    const uint32_t wr = INT8 ? (tid >> 2) : (tid >> 3);
    uint32_t w_off[WLD];
#pragma unroll
    for (int j = 0; j < WLD; j++) {
        uint32_t r = min(n0 + wr + (INT8 ? 64 : 32) * j, a.n - 1);
        w_off[j] = r * a.k + wc * (INT8 ? 16 : 8);
    }

    u32x4 ra[8], rw[WLD];
    auto load_global = [&](uint32_t k0) {
#pragma unroll
        for (int j = 0; j < 8; j++) ra[j] = *(const u32x4 *)(A + a_off[j] + k0);
        if (INT8) {
            const int8_t *W = (const int8_t *)a.w;
#pragma unroll
            for (int j = 0; j < WLD; j++) rw[j] = *(const u32x4 *)(W + w_off[j] + k0);
        } else {
            const u16 *W = (const u16 *)a.w;
#pragma unroll
            for (int j = 0; j < WLD; j++) rw[j] = *(const u32x4 *)(W + w_off[j] + k0);
        }
    };
    auto store_lds = [&](uint32_t buf) {
        unsigned char *As = lds + buf * G_LDS_BUF;
        unsigned char *Ws = As + 32768;
#pragma unroll
        for (int j = 0; j < 8; j++) *(u32x4 *)(As + g_swz(ar + 32 * j, ac)) = ra[j];
        if (INT8) {
#pragma unroll
            for (int j = 0; j < WLD; j++) {
                u32x4 lo, hi;
                i8x16_to_bf16(rw[j], lo, hi);
                const uint32_t r = wr + 64 * j;
                *(u32x4 *)(Ws + g_swz(r, 2 * wc)) = lo;
                *(u32x4 *)(Ws + g_swz(r, 2 * wc + 1)) = hi;
            }
        } else {
#pragma unroll
            for (int j = 0; j < WLD; j++) *(u32x4 *)(Ws + g_swz(wr + 32 * j, wc)) = rw[j];
        }
    };

    floatx16 acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int ni = 0; ni < 4; ni++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[mi][ni][v] = 0.0f;

    const uint32_t KT = a.k / GBK;
    load_global(0);
    store_lds(0);
    __syncthreads();
    for (uint32_t kt = 0; kt < KT; kt++) {
        const uint32_t cur = kt & 1;
        if (kt + 1 < KT) load_global((kt + 1) * GBK);
        const unsigned char *As = lds + cur * G_LDS_BUF;
        const unsigned char *Ws = As + 32768;
#pragma unroll
        for (uint32_t ks = 0; ks < 4; ks++) {
            bf16x8 af[4], bw[4];
#pragma unroll
            for (int mi = 0; mi < 4; mi++)
                af[mi] = *(const bf16x8 *)(As + g_swz(wm * 128 + mi * 32 + i32, 2 * ks + h));
#pragma unroll
            for (int ni = 0; ni < 4; ni++)
                bw[ni] = *(const bf16x8 *)(Ws + g_swz(wn * 128 + ni * 32 + i32, 2 * ks + h));
#pragma unroll
            for (int mi = 0; mi < 4; mi++)
#pragma unroll
                for (int ni = 0; ni < 4; ni++)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mi], bw[ni],
                                                                          acc[mi][ni], 0, 0, 0);
        }
        if (kt + 1 < KT) store_lds(cur ^ 1);
        __syncthreads();
    }

    /* ---- epilogue: lane holds column i32 of each 32x32 block, rows
     *      8 * (v / 4) + 4 * h + v % 4 -------------------------------------- */
    {
#pragma clang fp contract(off)
#pragma unroll
    for (int ni = 0; ni < 4; ni++) {
        const uint32_t col = n0 + wn * 128 + ni * 32 + i32;
        if (col >= a.n) continue;
        const float sc = INT8 ? a.wscale[col] : 1.0f;
        const float bias = a.bias ? bf2f(a.bias[col]) : 0.0f;
#pragma unroll
        for (int mi = 0; mi < 4; mi++) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const uint32_t row = m0 + wm * 128 + mi * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (row >= a.m) continue;
                float y = acc[mi][ni][v];
                if (INT8) y *= sc;
                y += bias;
                u16 *dst = a.out + (size_t)row * a.ldc + col;
                if (EPI == QW_EPI_STORE) {
                    *dst = f2bf(y);
                } else if (EPI == QW_EPI_GELU) {
                    *dst = f2bf(gelu_tanh_f(bf2f(f2bf(y))));
                } else {
                    const float g = bf2f(a.gate[(size_t)a.row_map[row] * a.gate_row_stride + col]);
                    *dst = f2bf(bf2f(*dst) + bf2f(f2bf(y)) * g);
                }
            }
        }
    }
    }
}

#define QW_GEMM_ENTRY(name, EPI, INT8)                                   \
    QW_KERNEL void __launch_bounds__(256, 1) name(qw_gemm_args a) {      \
        __shared__ __attribute__((aligned(16))) unsigned char lds[2 * G_LDS_BUF]; \
        qw_gemm_impl<EPI, INT8>(a, lds);                                  \
    }

QW_GEMM_ENTRY(qw_gemm_bf16_store, QW_EPI_STORE, 0)
QW_GEMM_ENTRY(qw_gemm_bf16_gelu, QW_EPI_GELU, 0)
QW_GEMM_ENTRY(qw_gemm_bf16_gate, QW_EPI_GATE, 0)
QW_GEMM_ENTRY(qw_gemm_i8_store, QW_EPI_STORE, 1)
QW_GEMM_ENTRY(qw_gemm_i8_gelu, QW_EPI_GELU, 1)
QW_GEMM_ENTRY(qw_gemm_i8_gate, QW_EPI_GATE, 1)

/* bf16 / int8-weight GEMM on CDNA4 matrix cores:
 *   out[m, n] = epilogue( sum_k A[m, k] * W[n, k] )
 * A bf16 row-major (row stride lda), W in the checkpoint's native [out, in]
 * layout (bf16, or int8 with one fp32 scale per output row), fp32
 * accumulation on the matrix cores.
 *
 * Tiling (template): a workgroup of WM x WN waves computes a BM x BN tile,
 * BM = WM * MI * 32, BN = WN * NI * 32, each wave an (MI*32) x (NI*32) block
 * of MI x NI MFMA tiles, stepping K by 64. One geometry is built: 4 x 2
 * waves of 2 x 4 blocks (256 x 256, two waves per SIMD, 128 accumulators
 * each: one wave's MFMAs cover the other's LDS/global latency), with
 * v_mfma_f32_32x32x16_bf16, for int8 weights widened in the loop (the
 * "_w8" kernels). bf16 weights run on the 4-wave kernels of gemm_q.h,
 * which share this file's LDS layout, direct loads, tile order and
 * epilogue.
 * A and W tiles are staged through LDS, double-buffered (2 x 64 KB at
 * 256 x 256), with the next K-slice's global loads in flight while the
 * current one is multiplied; within a K-slice the operand fragments of
 * sub-step s + 1 are read from LDS while the MFMAs of sub-step s run. LDS
 * rows are 128 B; 16-byte chunks are XOR-swizzled by (row / 2) % 8: the
 * 64 banks (256 B) serve 16 lanes of a ds_read_b128 per pass, and 16
 * consecutive rows then land on 16 distinct (bank half, chunk) slots (an
 * earlier row % 8 swizzle measured 2.3x more bank-conflict cycles). int8
 * weights are widened to bf16 (exact for |q| <= 127) on the way into LDS and the
 * per-row scale multiplies the fp32 sum in the epilogue, so the contraction
 * equals the dequantised product.
 *
 * The MFMA is issued as C^T = W A^T (W fragment as the A operand). The
 * epilogue (scale, bias, GELU, residual gate, q/k norm + RoPE) stages the
 * fp32 sums through LDS and writes whole 256-byte row runs.
 */
#pragma once
#include "common.h"

#define GBK 64
/* epilogue rows per pass: 8-wave kernels (two waves per SIMD share its registers) */
#ifndef QW_EPI_RP_D
#define QW_EPI_RP_D 2
#endif
/* End of a K-slice of the 16x16x32 pipeline: its direct loads landed
 * (vmcnt(0)) and this wave's LDS reads done, then a bare s_barrier. The
 * direct loads are issued from inline assembly, so the compiler's own wait
 * insertion does not know them; this wait is the one that covers them. */
#define QW_SLICE_END() asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory")
/* floats per split-tile partial (one 256 x 256 tile) */
#define QW_SPLIT_PART (256u * 256u)
/* buffer cache policy sc0 | sc1: coherent at device scope */
#define QW_CPOL_COHERENT 17
/* buffer cache policy nt: non-temporal */
#define QW_CPOL_NT 2

__device__ __forceinline__ uint32_t g_swz(uint32_t row, uint32_t chunk) {
    return row * 128u + ((chunk ^ ((row >> 1) & 7u)) << 4);
}

/* int8 x16 -> bf16 x16 (exact: bf16 holds every 8-bit integer), as two
 * 16-byte chunks: byte-select conversions to fp32, packed pairwise. */
__device__ __forceinline__ void i8x16_to_bf16(u32x4 q, u32x4 &lo, u32x4 &hi) {
    uint32_t o[8];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        int32_t x = (int32_t)q[w];
        o[2 * w] = pack_bf((float)((x << 24) >> 24), (float)((x << 16) >> 24));
        o[2 * w + 1] = pack_bf((float)((x << 8) >> 24), (float)(x >> 24));
    }
    lo = u32x4{o[0], o[1], o[2], o[3]};
    hi = u32x4{o[4], o[5], o[6], o[7]};
}

/* out[i] = bf16(q[i]) for count int8 weights (count % 16 == 0): the
 * unscaled widening that lets int8 linears run on the bf16 GEMM, whose
 * epilogue then applies the per-row scale to the fp32 sums. */
QW_KERNEL void __launch_bounds__(256) qw_widen_i8_bf16(qw_widen_args a) {
    const uint64_t n16 = a.count / 16;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
         i += (uint64_t)gridDim.x * blockDim.x) {
        u32x4 lo, hi;
        i8x16_to_bf16(((const u32x4 *)a.in)[i], lo, hi);
        ((u32x4 *)a.out)[2 * i] = lo;
        ((u32x4 *)a.out)[2 * i + 1] = hi;
    }
}

/* Linears with at most QW_GEMV_MAX_ROWS rows (the timestep / modulation
 * MLP runs on 1-2 rows): a 256 x 256 tile would be almost all padding and
 * its K loop latency-bound, so each wave instead streams QW_GEMV_COLS weight
 * rows (bf16, or int8 widened in registers) once, 16 bytes per lane, against
 * the same k chunks of every input row, with fp32 FMAs and a wave-shuffle
 * sum. The epilogue is the GEMM's: y = bf16(acc * wscale + bias) (the int8
 * scale multiplies the finished sum, as in the tiled kernels), then GELU or
 * a plain store. */
#define QW_GEMV_MAX_ROWS 8
#define QW_GEMV_COLS 2
template <int INT8, int EPI>
__device__ __forceinline__ void qw_gemv_impl(const qw_gemm_args &a) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t c0 = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * QW_GEMV_COLS;
    if (c0 >= a.n) return; /* whole waves */
    const uint32_t m = a.m, kc = a.k / 8;
    const u16 *A = (const u16 *)a.a;
    float acc[QW_GEMV_MAX_ROWS][QW_GEMV_COLS];
#pragma unroll
    for (int r = 0; r < QW_GEMV_MAX_ROWS; r++)
#pragma unroll
        for (int c = 0; c < QW_GEMV_COLS; c++) acc[r][c] = 0.0f;
    for (uint32_t j = lane; j < kc; j += 64) {
        float w[QW_GEMV_COLS][8];
#pragma unroll
        for (int c = 0; c < QW_GEMV_COLS; c++) {
            const uint32_t col = min(c0 + c, a.n - 1);
            if (INT8) {
                const u32x2 q = *(const u32x2 *)((const int8_t *)a.w + (size_t)col * a.k + 8 * j);
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int32_t x = (int32_t)q[h];
                    w[c][4 * h] = (float)((x << 24) >> 24);
                    w[c][4 * h + 1] = (float)((x << 16) >> 24);
                    w[c][4 * h + 2] = (float)((x << 8) >> 24);
                    w[c][4 * h + 3] = (float)(x >> 24);
                }
            } else {
                const u32x4 q = *(const u32x4 *)((const u16 *)a.w + (size_t)col * a.k + 8 * j);
#pragma unroll
                for (int i = 0; i < 4; i++) w[c][2 * i] = lo_bf(q[i]), w[c][2 * i + 1] = hi_bf(q[i]);
            }
        }
#pragma unroll
        for (int r = 0; r < QW_GEMV_MAX_ROWS; r++) {
            if ((uint32_t)r >= m) break;
            const u32x4 x = *(const u32x4 *)(A + (size_t)r * a.lda + 8 * j);
            float xf[8];
#pragma unroll
            for (int i = 0; i < 4; i++) xf[2 * i] = lo_bf(x[i]), xf[2 * i + 1] = hi_bf(x[i]);
#pragma unroll
            for (int c = 0; c < QW_GEMV_COLS; c++)
#pragma unroll
                for (int i = 0; i < 8; i++) acc[r][c] = fmaf(xf[i], w[c][i], acc[r][c]);
        }
    }
#pragma unroll
    for (int r = 0; r < QW_GEMV_MAX_ROWS; r++) {
        if ((uint32_t)r >= m) break;
#pragma unroll
        for (int c = 0; c < QW_GEMV_COLS; c++) {
            float t = wave_sum(acc[r][c]);
            const uint32_t col = c0 + c;
            if (lane != 0 || col >= a.n) continue;
            if (a.wscale) t *= a.wscale[col];
            float y = bf2f(f2bf(t + (a.bias ? bf2f(a.bias[col]) : 0.0f)));
            if (EPI == QW_EPI_GELU) y = gelu_tanh_f(y);
            a.out[(size_t)r * a.ldc + col] = f2bf(y);
        }
    }
}
QW_KERNEL void __launch_bounds__(256) qw_gemv_bf16_store(qw_gemm_args a) {
    qw_gemv_impl<0, QW_EPI_STORE>(a);
}
QW_KERNEL void __launch_bounds__(256) qw_gemv_bf16_gelu(qw_gemm_args a) {
    qw_gemv_impl<0, QW_EPI_GELU>(a);
}
QW_KERNEL void __launch_bounds__(256) qw_gemv_i8_store(qw_gemm_args a) {
    qw_gemv_impl<1, QW_EPI_STORE>(a);
}
QW_KERNEL void __launch_bounds__(256) qw_gemv_i8_gelu(qw_gemm_args a) {
    qw_gemv_impl<1, QW_EPI_GELU>(a);
}

/* Workgroup id -> (tile row, tile column). Ids are dealt round-robin to the
 * 8 XCDs; the id is remapped so each XCD owns a contiguous range of tiles,
 * walked in groups of 8 tile-rows (column-major inside a group), so the A
 * and W panels an XCD touches stay hot in its L2. */
__device__ __forceinline__ void gemm_tile_at(const qw_gemm_args &a, uint32_t pid, uint32_t &tm,
                                             uint32_t &tn) {
#ifndef QW_GEMM_GROUP
#define QW_GEMM_GROUP 8
#endif
    const uint32_t G = QW_GEMM_GROUP;
    const uint32_t per_group = G * a.tiles_n;
    const uint32_t first_m = (pid / per_group) * G;
    const uint32_t gsize = min(a.tiles_m - first_m, G);
    const uint32_t inner = pid % per_group;
    tm = first_m + inner % gsize;
    tn = inner / gsize;
}
__device__ __forceinline__ void gemm_tile(const qw_gemm_args &a, uint32_t &tm, uint32_t &tn) {
    const uint32_t nt = a.tiles_m * a.tiles_n;
    uint32_t pid = blockIdx.x;
    if ((nt & 7u) == 0) pid = (pid & 7u) * (nt >> 3) + (pid >> 3);
    gemm_tile_at(a, pid, tm, tn);
}

/* Epilogue through LDS: the fp32 sums of each 32-row slab of the wave's
 * block are first written to a wave-private LDS region (row stride
 * NI*32 + 4 floats: the 16 lanes of a ds_write_b128 pass land on 16
 * distinct 4-bank groups), then read back row-contiguous: 16 lanes per row,
 * 8 columns (one 16-byte store) per lane, so every output row segment is
 * written by whole 256-byte runs, and the residual/gate reads of the GATE
 * epilogue are coalesced the same way. A lane keeps the same 8 columns for
 * every row, so it loads their scale and bias once.
 *
 * Rows are processed RP at a time without branches: a lane outside the
 * output (row >= m, or its columns >= n) addresses its output and residual
 * past the end of a buffer resource, so its loads return zeros and its
 * stores are dropped. The per-row operands of the RP rows (residual, gate,
 * RoPE table rows) are issued before their LDS reads, so the rows' memory
 * latencies overlap each other instead of adding up row by row.
 *
 * MODE 0: a finished tile. MODE 1: a piece of a split tile, whose fp32 sums
 * are stored to its partial slot. MODE 2: the last piece of a split tile,
 * which adds all pieces' sums in piece order (its own from LDS) and runs
 * the epilogue. */
template <int EPI, int INT8, int MI, int NI, int RP, int MODE, class SlabWriter>
__device__ __forceinline__ void gemm_epilogue_mode(const qw_gemm_args &a, SlabWriter write_slab,
                                                   float *region, uint32_t row0, uint32_t col0,
                                                   uint32_t lane, float *pst, const float *pld,
                                                   uint32_t npart, uint32_t own) {
#pragma clang fp contract(off)
    constexpr uint32_t LDF = NI * 32 + 4; /* floats per staged row */
    static_assert(8 % RP == 0, "rows per pass");
    const bool scaled = INT8 || a.wscale != nullptr;
    /* split-tile partials go through device-coherent buffer accesses (write
     * through / read past the XCD's L2), so pieces on different XCDs see
     * each other's sums without any L2 write-back or invalidate */
    const __amdgpu_buffer_rsrc_t part_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.sk_part, (short)0, (int)0x7FFFFFF0, 0x00020000);
    const __amdgpu_buffer_rsrc_t out_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.out, (short)0, (int)a.out_bytes, 0x00020000);
    /* read-back geometry: lane -> (row within a 4-row group, 8-column chunk) */
    const uint32_t rr = lane >> 4, cc = lane & 15;
    constexpr uint32_t CHUNKS = NI * 32 / 8; /* 16 for NI = 4 */
    static_assert(CHUNKS == 16, "read-back maps 16 lanes to one row");
    const uint32_t col = col0 + cc * 8;
    const bool col_ok = col < a.n;                 /* n % 8 == 0 */
    const uint32_t colc = col_ok ? col : a.n - 8;  /* in-range column for operand loads */
    float sc[8], bias[8];
#pragma unroll
    for (int j = 0; j < 8; j++) sc[j] = 1.0f, bias[j] = 0.0f;
    if (MODE != 1) {
        if (scaled) {
            const floatx4 s0 = *(const floatx4 *)(a.wscale + colc);
            const floatx4 s1 = *(const floatx4 *)(a.wscale + colc + 4);
#pragma unroll
            for (int j = 0; j < 4; j++) sc[j] = s0[j], sc[4 + j] = s1[j];
        }
        if (a.bias) {
            const u32x4 bb = *(const u32x4 *)(a.bias + colc);
#pragma unroll
            for (int j = 0; j < 4; j++) bias[2 * j] = lo_bf(bb[j]), bias[2 * j + 1] = hi_bf(bb[j]);
        }
    }
    /* QW_EPI_QKNORM: this wave's 128 columns are one head (tiles start at
     * multiples of 256); q or k heads get the norm weight of their kind */
    const bool qk_head = EPI == QW_EPI_QKNORM && MODE != 1 && col0 < a.qk_cols;
    float nw[8];
    if (EPI == QW_EPI_QKNORM && qk_head) {
        const u32x4 wn = *(const u32x4 *)((col0 < a.qk_cols / 2 ? a.norm_q : a.norm_k) + 8 * cc);
#pragma unroll
        for (int i = 0; i < 4; i++) nw[2 * i] = lo_bf(wn[i]), nw[2 * i + 1] = hi_bf(wn[i]);
    }
    /* first/second 16-byte halves of the lane's 32 read-back bytes:
     * lanes 8-15 of a row start with the upper half, so one ds_read_b128
     * pass covers all 64 banks */
    const uint32_t swap = (cc >> 3) & 1;
    auto lds_row = [&](uint32_t lr, float (&v)[8]) __attribute__((always_inline)) {
        const floatx4 v0 = *(const floatx4 *)(region + lr * LDF + cc * 8 + 4 * swap);
        const floatx4 v1 = *(const floatx4 *)(region + lr * LDF + cc * 8 + 4 * (swap ^ 1));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[j] = swap ? v1[j] : v0[j];
            v[4 + j] = swap ? v0[j] : v1[j];
        }
    };
#pragma unroll
    for (int mi = 0; mi < MI; mi++) {
        write_slab(mi); /* fp32 sums of rows [32 mi, 32 mi + 32) into region */
#pragma unroll
        for (int p0 = 0; p0 < 8; p0 += RP) {
            uint32_t ooff[RP];
            u32x4 gv[RP], rv[RP];
            floatx4 rc[RP], rs[RP];
#pragma unroll
            for (int i = 0; i < RP; i++) {
                const uint32_t row = row0 + mi * 32 + 4 * (p0 + i) + rr;
                ooff[i] = col_ok && row < a.m ? (row * a.ldc + col) * 2 : 0x80000000u;
                if (EPI == QW_EPI_GATE && MODE != 1) {
                    const uint32_t mrow = a.row_map[min(row, a.m - 1)];
                    gv[i] = *(const u32x4 *)(a.gate + (size_t)mrow * a.gate_row_stride + colc);
                    rv[i] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(out_rsrc, ooff[i], 0, 0));
                }
            }
            if (EPI == QW_EPI_QKNORM && qk_head) {
#pragma unroll
                for (int i = 0; i < RP; i++) {
                    const uint32_t row = min(row0 + mi * 32 + 4 * (p0 + i) + rr, a.m - 1);
                    const size_t t = (size_t)(row % a.rope_rows) * 64 + 4 * cc;
                    rc[i] = *(const floatx4 *)(a.rope_cos + t);
                    rs[i] = *(const floatx4 *)(a.rope_sin + t);
                }
            }
            float y[RP][8];
            if (MODE == 2) { /* all pieces of a split tile, summed in piece order */
#pragma unroll
                for (int i = 0; i < RP; i++)
#pragma unroll
                    for (int j = 0; j < 8; j++) y[i][j] = 0.0f;
                for (uint32_t pc = 0; pc < npart; pc++) {
                    if (pc == own) {
#pragma unroll
                        for (int i = 0; i < RP; i++) {
                            float v[8];
                            lds_row(4 * (p0 + i) + rr, v);
#pragma unroll
                            for (int j = 0; j < 8; j++) y[i][j] += v[j];
                        }
                    } else {
#pragma unroll
                        for (int i = 0; i < RP; i++) {
                            const uint32_t poff = (mi * 32 + 4 * (p0 + i) + rr) * 256 + cc * 8;
                            const uint32_t bo =
                                (uint32_t)((pld - a.sk_part) + pc * QW_SPLIT_PART + poff) * 4;
                            const floatx4 q0 = __builtin_bit_cast(
                                floatx4, __builtin_amdgcn_raw_buffer_load_b128(part_rsrc, bo, 0,
                                                                               QW_CPOL_COHERENT));
                            const floatx4 q1 = __builtin_bit_cast(
                                floatx4, __builtin_amdgcn_raw_buffer_load_b128(
                                             part_rsrc, bo + 16, 0, QW_CPOL_COHERENT));
#pragma unroll
                            for (int j = 0; j < 4; j++) y[i][j] += q0[j], y[i][4 + j] += q1[j];
                        }
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < RP; i++) lds_row(4 * (p0 + i) + rr, y[i]);
            }
            if constexpr (MODE == 1) { /* piece of a split tile: keep the fp32 sums */
#pragma unroll
                for (int i = 0; i < RP; i++) {
                    const uint32_t poff = (mi * 32 + 4 * (p0 + i) + rr) * 256 + cc * 8;
                    const uint32_t bo = (uint32_t)((pst - a.sk_part) + poff) * 4;
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4, floatx4{y[i][0], y[i][1], y[i][2], y[i][3]}),
                        part_rsrc, bo, 0, QW_CPOL_COHERENT);
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4, floatx4{y[i][4], y[i][5], y[i][6], y[i][7]}),
                        part_rsrc, bo + 16, 0, QW_CPOL_COHERENT);
                }
                continue;
            }
#pragma unroll
            for (int i = 0; i < RP; i++)
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    float t = y[i][j];
                    if (scaled) t *= sc[j];
                    y[i][j] = bf2f(f2bf(t + bias[j]));
                }
            if (EPI == QW_EPI_QKNORM && qk_head) {
                /* the 16 lanes of a row hold one head, 8 elements each
                 * (lane cc: elements 8 cc..8 cc + 7), as qw_qk_norm_rope_bf16
                 * holds it: the same sum order, shuffles and roundings */
                float ss[RP];
#pragma unroll
                for (int i = 0; i < RP; i++) {
                    ss[i] = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; j++) ss[i] = fmaf(y[i][j], y[i][j], ss[i]);
                }
#pragma unroll
                for (int o = 8; o > 0; o >>= 1)
#pragma unroll
                    for (int i = 0; i < RP; i++) ss[i] += __shfl_xor(ss[i], o, 64);
#pragma unroll
                for (int i = 0; i < RP; i++) {
                    const float inv = 1.0f / sqrtf(ss[i] / 128.0f + a.eps);
#pragma unroll
                    for (int j = 0; j < 8; j++) y[i][j] = bf2f(f2bf(y[i][j] * inv * nw[j]));
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float y0 = y[i][2 * q] * rc[i][q] - y[i][2 * q + 1] * rs[i][q];
                        const float y1 = y[i][2 * q] * rs[i][q] + y[i][2 * q + 1] * rc[i][q];
                        y[i][2 * q] = y0;
                        y[i][2 * q + 1] = y1;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < RP; i++) {
                if (EPI == QW_EPI_GELU) {
#pragma unroll
                    for (int j = 0; j < 8; j++) y[i][j] = gelu_tanh_f(y[i][j]);
                } else if (EPI == QW_EPI_GATE) {
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        y[i][2 * j] = lo_bf(rv[i][j]) + y[i][2 * j] * lo_bf(gv[i][j]);
                        y[i][2 * j + 1] = hi_bf(rv[i][j]) + y[i][2 * j + 1] * hi_bf(gv[i][j]);
                    }
                }
                /* non-temporal store (cache policy NT): measured 3% faster
                 * on the up projection and 8% on 8192^3 than a
                 * default-policy store */
                __builtin_amdgcn_raw_buffer_store_b128(
                    u32x4{pack_bf(y[i][0], y[i][1]), pack_bf(y[i][2], y[i][3]),
                          pack_bf(y[i][4], y[i][5]), pack_bf(y[i][6], y[i][7])},
                    out_rsrc, ooff[i], 0, QW_CPOL_NT);
            }
        }
    }
}

template <int EPI, int INT8, int MI, int NI, int RP, class SlabWriter>
__device__ __forceinline__ void gemm_epilogue_lds(const qw_gemm_args &a, SlabWriter write_slab,
                                                  float *region, uint32_t row0, uint32_t col0,
                                                  uint32_t lane, float *pst, const float *pld,
                                                  uint32_t npart, uint32_t own) {
    if (pst)
        gemm_epilogue_mode<EPI, INT8, MI, NI, RP, 1>(a, write_slab, region, row0, col0, lane, pst,
                                                     pld, npart, own);
    else if (pld)
        gemm_epilogue_mode<EPI, INT8, MI, NI, RP, 2>(a, write_slab, region, row0, col0, lane, pst,
                                                     pld, npart, own);
    else
        gemm_epilogue_mode<EPI, INT8, MI, NI, RP, 0>(a, write_slab, region, row0, col0, lane, pst,
                                                     pld, npart, own);
}

template <int WM, int WN, int MI, int NI>
struct GemmShape {
    static constexpr int NT = 64 * WM * WN;
    static constexpr int BM = WM * MI * 32;
    static constexpr int BN = WN * NI * 32;
    static constexpr int A_BYTES = BM * 128; /* BM rows x 64 bf16 */
    static constexpr int W_BYTES = BN * 128;
    static constexpr int STAGE = A_BYTES + W_BYTES;
    static constexpr int A_LD = BM * 8 / NT;        /* 16-byte A chunks per thread */
    static constexpr int W_LD_BF16 = BN * 8 / NT;   /* 16-byte bf16 W chunks */
    static constexpr int W_LD_I8 = BN * 4 / NT;     /* 16-byte int8 W chunks */
};

/* Operands of one pipelined K-slice (direct-to-LDS path). */
template <int A_DL, int W_DL, int WLD>
struct PipeCtx {
    __amdgpu_buffer_rsrc_t a_rsrc, w_rsrc;
    uint32_t a_dvoff[A_DL];
    uint32_t w_dvoff[W_DL > 0 ? W_DL : 1];
    uint32_t w_off[WLD];
    uint32_t a_row0, w_row0, swz, h, a_dst0, w_dst0, wr, wc;
    u32x4 a_rs4, w_rs4; /* the rsrcs as plain words, for the inline-assembly loads */
};

/* buffer_load_dwordx4 ... lds from inline assembly: M0 = LDS address,
 * lane l writes M0 + 16 l */
__device__ __forceinline__ void gemm_dma16(u32x4 rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
                 : "m0");
}
__device__ __forceinline__ u32x4 gemm_rs4(const void *p, uint32_t bytes) {
    const uint64_t b = (uint64_t)p;
    return u32x4{(uint32_t)b, (uint32_t)(b >> 32) & 0xffffu, bytes, 0x00020000u};
}

/* One K-slice: multiply the stage `cur` while slice k_next streams into the
 * stage `nxt`. The two stages are distinct (restrict) so the scheduler may
 * interleave the LDS fragment reads of one with the direct loads into the
 * other. The last sub-step's MFMAs are held back: they run at the start of
 * the next slice (PREV), after the barrier, under the LDS reads of that
 * slice's first fragments, so the matrix pipe does not drain at each
 * barrier. pa / pw carry those fragments from one slice to the next.
 * sched_group_barrier lays out the pipeline: fragment reads of sub-step
 * s + 1, the slice loads and the int8 LDS writes between MFMAs. */
template <int INT8, int MI, int NI, int A_BYTES, int A_DL, int W_DL, int WLD, int WROWS,
          bool PREV>
__device__ __forceinline__ void gemm_pipe_slice(const PipeCtx<A_DL, W_DL, WLD> &c,
                                                floatx16 (&acc)[NI][MI], bf16x8 (&pa)[MI],
                                                bf16x8 (&pw)[NI],
                                                const unsigned char *__restrict__ cur,
                                                unsigned char *__restrict__ nxt,
                                                uint32_t k_next) {
    typedef __attribute__((address_space(3))) void lds_void;
    /* slice k_next: A (and bf16 W) straight into LDS; the k advance rides
     * in the scalar offset, so the lane offsets need no per-slice VALU */
#pragma unroll
    for (int j = 0; j < A_DL; j++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(c.a_rsrc, (lds_void *)(nxt + c.a_dst0 + j * 1024),
                                                 16, c.a_dvoff[j], k_next * 2, 0, 0);
#pragma unroll
    for (int j = 0; j < W_DL; j++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(c.w_rsrc,
                                                 (lds_void *)(nxt + A_BYTES + c.w_dst0 + j * 1024),
                                                 16, c.w_dvoff[j], k_next * 2, 0, 0);
    u32x4 rw[WLD];
    if (INT8) {
#pragma unroll
        for (int j = 0; j < WLD; j++)
            rw[j] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(c.w_rsrc, c.w_off[j], k_next, 0));
    }
    const unsigned char *As = cur, *Ws = cur + A_BYTES;
#define QW_FR(row, ks) ((row) * 128u + (((2 * (ks) + c.h) ^ c.swz) << 4))
    bf16x8 af[2][MI], bw[2][NI];
#pragma unroll
    for (int i = 0; i < MI; i++) af[0][i] = *(const bf16x8 *)(As + QW_FR(c.a_row0 + 32 * i, 0));
#pragma unroll
    for (int i = 0; i < NI; i++) bw[0][i] = *(const bf16x8 *)(Ws + QW_FR(c.w_row0 + 32 * i, 0));
    if (PREV) { /* the previous slice's last sub-step */
#pragma unroll
        for (int ni = 0; ni < NI; ni++)
#pragma unroll
            for (int mi = 0; mi < MI; mi++)
                acc[ni][mi] =
                    __builtin_amdgcn_mfma_f32_32x32x16_bf16(pw[ni], pa[mi], acc[ni][mi], 0, 0, 0);
    }
#pragma unroll
    for (uint32_t ks = 0; ks < 3; ks++) {
        const int b = ks & 1;
#pragma unroll
        for (int i = 0; i < MI; i++)
            af[b ^ 1][i] = *(const bf16x8 *)(As + QW_FR(c.a_row0 + 32 * i, ks + 1));
#pragma unroll
        for (int i = 0; i < NI; i++)
            bw[b ^ 1][i] = *(const bf16x8 *)(Ws + QW_FR(c.w_row0 + 32 * i, ks + 1));
#pragma unroll
        for (int ni = 0; ni < NI; ni++)
#pragma unroll
            for (int mi = 0; mi < MI; mi++)
                acc[ni][mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw[b][ni], af[b][mi],
                                                                      acc[ni][mi], 0, 0, 0);
    }
#undef QW_FR
#pragma unroll
    for (int i = 0; i < MI; i++) pa[i] = af[1][i];
#pragma unroll
    for (int i = 0; i < NI; i++) pw[i] = bw[1][i];
    if (INT8) {
        unsigned char *Wn = nxt + A_BYTES;
#pragma unroll
        for (int j = 0; j < WLD; j++) {
            u32x4 lo, hi;
            i8x16_to_bf16(rw[j], lo, hi);
            const uint32_t r = c.wr + WROWS * j;
            *(u32x4 *)(Wn + g_swz(r, 2 * c.wc)) = lo;
            *(u32x4 *)(Wn + g_swz(r, 2 * c.wc + 1)) = hi;
        }
    }
    constexpr int NMF = MI * NI, NRD = MI + NI;
    constexpr int NV = A_DL + W_DL + (INT8 ? WLD : 0);
    constexpr int NW = INT8 ? 2 * WLD : 0;
    static_assert(NV <= NMF && NW <= NMF && NRD <= NMF, "pipeline pattern");
    if (PREV) {
#pragma unroll
        for (int i = 0; i < NMF; i++) { /* held-back MFMAs: slice loads + fragments of step 0 */
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i < NV) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            if (i < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    } else {
        __builtin_amdgcn_sched_group_barrier(0x020, NV, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);
    }
#pragma unroll
    for (int st = 0; st < 3; st++)
#pragma unroll
        for (int i = 0; i < NMF; i++) { /* steps 0-2: fragments of the next step */
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (st == 2 && i < NW) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
        }
}

/* Sums of tile (tm, tn) over k-steps [kb, ke) (64 k each) into acc; the
 * Ends with the LDS
 * stages free (after a barrier). */
template <int INT8, int WM, int WN, int MI, int NI>
__device__ __forceinline__ void gemm_mainloop(const qw_gemm_args &a, unsigned char *lds,
                                              unsigned char *lds_b, uint32_t tm, uint32_t tn,
                                              uint32_t kb, uint32_t ke,
                                              floatx16 (&acc)[NI][MI]) {
    typedef GemmShape<WM, WN, MI, NI> S;
    /* wave index in a scalar register: the LDS destinations of the direct
     * loads (M0) and the fragment bases then need no per-slice
     * vector-to-scalar moves */
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WN, wn = wave % WN;
    const uint32_t h = lane >> 5, i32 = lane & 31;
    const uint32_t m0 = tm * S::BM, n0 = tn * S::BN;

    /* ---- global loads: raw buffer loads with 32-bit byte offsets (one
     *      VGPR per load address), rows clamped at the edges ------------- */
    const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.a, (short)0, (int)a.a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.w, (short)0, (int)a.w_bytes, 0x00020000);
    const uint32_t ac = tid & 7, ar = tid >> 3; /* 8 chunks per 64-wide row */
    constexpr int AROWS = S::NT / 8;             /* rows per load pass */
    uint32_t a_off[S::A_LD];
#pragma unroll
    for (int j = 0; j < S::A_LD; j++) {
        uint32_t r = min(m0 + ar + AROWS * j, a.m - 1);
        a_off[j] = (r * a.lda + ac * 8) * 2;
    }
    constexpr int WLD = INT8 ? S::W_LD_I8 : S::W_LD_BF16;
    constexpr int WROWS = INT8 ? S::NT / 4 : S::NT / 8;
    constexpr uint32_t WES = INT8 ? 1 : 2; /* weight element bytes */
    const uint32_t wc = INT8 ? (tid & 3) : (tid & 7);
    const uint32_t wr = INT8 ? (tid >> 2) : (tid >> 3);
    uint32_t w_off[WLD];
#pragma unroll
    for (int j = 0; j < WLD; j++) {
        uint32_t r = min(n0 + wr + WROWS * j, a.n - 1);
        w_off[j] = (r * a.k + wc * (INT8 ? 16 : 8)) * WES;
    }

    /* staging registers of the int8 W prologue (widened on the way into LDS) */
    u32x4 ra[1][S::A_LD], rw[1][WLD];
#define QW_LOAD(SET, k0)                                                                      \
    do {                                                                                       \
        _Pragma("unroll") for (int j = 0; j < S::A_LD; j++) ra[SET][j] = __builtin_bit_cast(   \
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_off[j] + (k0) * 2, 0, 0));  \
        _Pragma("unroll") for (int j = 0; j < WLD; j++) rw[SET][j] = __builtin_bit_cast(       \
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_off[j] + (k0) * WES, 0, 0)); \
    } while (0)
    auto store_lds = [&](const u32x4 *sa, const u32x4 *sw, uint32_t buf)
                         __attribute__((always_inline)) {
        unsigned char *As = lds + buf * S::STAGE;
        unsigned char *Ws = As + S::A_BYTES;
#pragma unroll
        for (int j = 0; j < S::A_LD; j++) *(u32x4 *)(As + g_swz(ar + AROWS * j, ac)) = sa[j];
        if (INT8) {
#pragma unroll
            for (int j = 0; j < WLD; j++) {
                u32x4 lo, hi;
                i8x16_to_bf16(sw[j], lo, hi);
                const uint32_t r = wr + WROWS * j;
                *(u32x4 *)(Ws + g_swz(r, 2 * wc)) = lo;
                *(u32x4 *)(Ws + g_swz(r, 2 * wc + 1)) = hi;
            }
        } else {
#pragma unroll
            for (int j = 0; j < WLD; j++) *(u32x4 *)(Ws + g_swz(wr + WROWS * j, wc)) = sw[j];
        }
    };

#pragma unroll
    for (int ni = 0; ni < NI; ni++)
#pragma unroll
        for (int mi = 0; mi < MI; mi++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[ni][mi][v] = 0.0f;

    /* fragment rows: this lane's row within each 32-row block; the swizzle
     * term (row / 2) % 8 only depends on i32 (blocks are 32-aligned) */
    const uint32_t a_row0 = wm * (MI * 32) + i32, w_row0 = wn * (NI * 32) + i32;
    const uint32_t swz = (i32 >> 1) & 7u;

    const uint32_t KT = ke;
    {
        /* Direct-to-LDS pipeline. The A tile (and a bf16 W tile) are loaded
         * with buffer_load_dwordx4 ... lds: each instruction writes 1 KB
         * (8 rows) of a wave's share of the tile straight into LDS, lane l
         * landing on row l / 8, physical chunk l % 8; the lane therefore
         * fetches logical chunk (l % 8) ^ ((row / 2) % 8), which realises
         * the swizzle with no staging registers and no ds_write. int8 W is
         * still widened through registers. The last slice re-loads itself
         * into the idle stage, which nobody reads afterwards. */
        constexpr int NWAVE = WM * WN;
        constexpr int A_DL = S::BM / 8 / NWAVE;  /* direct loads per wave, A */
        constexpr int W_DL = INT8 ? 0 : S::BN / 8 / NWAVE;
        PipeCtx<A_DL, W_DL, WLD> c;
        c.a_rsrc = a_rsrc;
        c.w_rsrc = w_rsrc;
        const uint32_t lrow = lane >> 3, lp = lane & 7;
#pragma unroll
        for (int j = 0; j < A_DL; j++) {
            const uint32_t r = wave * (S::BM / NWAVE) + j * 8 + lrow;
            c.a_dvoff[j] = (min(m0 + r, a.m - 1) * a.lda + (lp ^ ((r >> 1) & 7u)) * 8) * 2;
        }
#pragma unroll
        for (int j = 0; j < W_DL; j++) {
            const uint32_t r = wave * (S::BN / NWAVE) + j * 8 + lrow;
            c.w_dvoff[j] = (min(n0 + r, a.n - 1) * a.k + (lp ^ ((r >> 1) & 7u)) * 8) * 2;
        }
#pragma unroll
        for (int j = 0; j < WLD; j++) c.w_off[j] = w_off[j];
        c.a_row0 = a_row0;
        c.w_row0 = w_row0;
        c.swz = swz;
        c.h = h;
        c.a_dst0 = wave * (S::BM / NWAVE) * 128;
        c.w_dst0 = wave * (S::BN / NWAVE) * 128;
        c.wr = wr;
        c.wc = wc;
        c.a_rs4 = gemm_rs4(a.a, a.a_bytes);
        c.w_rs4 = gemm_rs4(a.w, a.w_bytes);
        /* prologue: slice 0 into stage lds (A/W direct; int8 W via regs) */
        {
            typedef __attribute__((address_space(3))) void lds_void;
            const uint32_t k0 = kb * GBK;
#pragma unroll
            for (int j = 0; j < A_DL; j++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_void *)(lds + c.a_dst0 + j * 1024),
                                                         16, c.a_dvoff[j] + k0 * 2, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < W_DL; j++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    w_rsrc, (lds_void *)(lds + S::A_BYTES + c.w_dst0 + j * 1024), 16,
                    c.w_dvoff[j] + k0 * 2, 0, 0, 0);
            if (INT8) {
                QW_LOAD(0, k0);
                store_lds(ra[0], rw[0], 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0): direct loads landed */
        __syncthreads();
        {
            bf16x8 pa[MI], pw[NI]; /* last sub-step's fragments, multiplied one slice late */
            {
                const uint32_t nk = (kb + 1 < KT ? kb + 1 : kb) * GBK;
                gemm_pipe_slice<INT8, MI, NI, S::A_BYTES, A_DL, W_DL, WLD, WROWS, false>(
                    c, acc, pa, pw, lds, lds_b, nk);
                __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();
            }
            /* two slices per trip, so each one's stages are fixed at compile
             * time and their LDS bases fold into the instructions' offsets */
            uint32_t kt = kb + 1;
            for (; kt + 1 < KT; kt += 2) {
                gemm_pipe_slice<INT8, MI, NI, S::A_BYTES, A_DL, W_DL, WLD, WROWS, true>(
                    c, acc, pa, pw, lds_b, lds, (kt + 1) * GBK);
                __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();
                gemm_pipe_slice<INT8, MI, NI, S::A_BYTES, A_DL, W_DL, WLD, WROWS, true>(
                    c, acc, pa, pw, lds, lds_b, (kt + 2 < KT ? kt + 2 : kt + 1) * GBK);
                __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();
            }
            if (kt < KT) { /* the last slice, from stage lds_b */
                gemm_pipe_slice<INT8, MI, NI, S::A_BYTES, A_DL, W_DL, WLD, WROWS, true>(
                    c, acc, pa, pw, lds_b, lds, kt * GBK);
                __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();
            }
    #pragma unroll
            for (int ni = 0; ni < NI; ni++)
    #pragma unroll
                for (int mi = 0; mi < MI; mi++)
                    acc[ni][mi] =
                        __builtin_amdgcn_mfma_f32_32x32x16_bf16(pw[ni], pa[mi], acc[ni][mi], 0, 0, 0);
        }
    }
#undef QW_LOAD
}

/* Epilogue of a finished tile (bf16 output plus the EPI op), or with pst the
 * fp32 sums of one piece of a split tile, or with pld the sum of all its
 * pieces followed by the epilogue */
template <int EPI, int INT8, int WM, int WN, int MI, int NI>
__device__ __forceinline__ void gemm_finish(const qw_gemm_args &a, unsigned char *lds,
                                            unsigned char *lds_b, uint32_t tm, uint32_t tn,
                                            floatx16 (&acc)[NI][MI], float *pst = nullptr,
                                            const float *pld = nullptr, uint32_t npart = 0,
                                            uint32_t own = 0) {
    typedef GemmShape<WM, WN, MI, NI> S;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave / WN, wn = wave % WN;
    const uint32_t h = lane >> 5, i32 = lane & 31;
    const uint32_t row0 = tm * S::BM + wm * (MI * 32), col0 = tn * S::BN + wn * (NI * 32);
    static_assert(NI == 4, "the LDS epilogue maps 16 lanes to one 128-column row");
    {
        /* the stages are free after the loop's last barrier: the first half
         * of the waves stage through `lds`, the second through `lds_b`, one
         * 32-row slab (16.5 KB) per wave at a time */
        constexpr int NW = WM * WN, REG = 32 * (NI * 32 + 4) * 4;
        float *region = (float *)((wave < NW / 2 ? lds : lds_b) + (wave % (NW / 2)) * REG);
        /* split-tile partials: row-major 256 x 256 fp32 */
        static_assert(S::BN == 256 && S::BM * S::BN <= QW_SPLIT_PART, "partial tile size");
        const uint32_t poff = wm * (MI * 32) * 256 + wn * (NI * 32);
        constexpr uint32_t LDF = NI * 32 + 4; /* floats per staged row */
        auto write_slab = [&](int mi) __attribute__((always_inline)) {
            {
#pragma unroll
                for (int ni = 0; ni < NI; ni++)
#pragma unroll
                    for (int g = 0; g < 4; g++)
                        *(floatx4 *)(region + i32 * LDF + ni * 32 + 8 * g + 4 * h) =
                            floatx4{acc[ni][mi][4 * g], acc[ni][mi][4 * g + 1],
                                    acc[ni][mi][4 * g + 2], acc[ni][mi][4 * g + 3]};
            }
        };
        gemm_epilogue_lds<EPI, INT8, MI, NI, QW_EPI_RP_D>(a, write_slab, region, row0, col0, lane,
                                             pst ? pst + poff : nullptr, pld ? pld + poff : nullptr,
                                             npart, own);
    }
}

template <int EPI, int INT8, int WM, int WN, int MI, int NI>
__device__ __forceinline__ void qw_gemm_impl(const qw_gemm_args &a, unsigned char *lds,
                                             unsigned char *lds_b) {
    const uint32_t KT = a.k / GBK;
    const uint32_t nt = a.tiles_m * a.tiles_n;
    const bool split = a.split > 1;
    const uint32_t ndp = split ? a.dp_tiles : nt;
    floatx16 acc[NI][MI]; /* C^T blocks */
    uint32_t pid = blockIdx.x, tm, tn;
    if (pid < ndp) { /* whole tile; ids XCD-remapped over the whole-tile range */
        if ((ndp & 7u) == 0) pid = (pid & 7u) * (ndp >> 3) + (pid >> 3);
        gemm_tile_at(a, pid, tm, tn);
        gemm_mainloop<INT8, WM, WN, MI, NI>(a, lds, lds_b, tm, tn, 0, KT, acc);
        gemm_finish<EPI, INT8, WM, WN, MI, NI>(a, lds, lds_b, tm, tn, acc);
        return;
    }
    /* Piece of a split tile. Pieces are numbered k-range-major, so the
     * workgroups resident together multiply neighbouring tiles over the same
     * k-range and share their A and W panels in L2, as whole tiles do. */
    __shared__ uint32_t ticket;
    const uint32_t R = nt - ndp, S = a.split, np = R * S;
    uint32_t q = pid - ndp;
    if ((np & 7u) == 0) q = (q & 7u) * (np >> 3) + (q >> 3);
    const uint32_t piece = q / R, r = q % R;
    const uint32_t kb = piece * KT / S, ke = (piece + 1) * KT / S;
    gemm_tile_at(a, ndp + r, tm, tn);
    gemm_mainloop<INT8, WM, WN, MI, NI>(a, lds, lds_b, tm, tn, kb, ke, acc);
    float *slots = a.sk_part + (size_t)r * S * QW_SPLIT_PART;
    gemm_finish<EPI, INT8, WM, WN, MI, NI>(a, lds, lds_b, tm, tn, acc,
                                               slots + (size_t)piece * QW_SPLIT_PART);
    /* publish the partial (its coherent stores complete before the
     * workgroup's barrier), then count it. Agent-scope release/acquire
     * fences are not used: on this part they write back and invalidate the
     * whole L2, which the other tiles' panels live in. */
    __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0): the partial's stores are done */
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (threadIdx.x == 0)
        ticket = __hip_atomic_fetch_add(a.sk_flag + r, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (ticket != S - 1) return;
    /* last piece in: the others' partials are read with coherent loads */
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    gemm_finish<EPI, INT8, WM, WN, MI, NI>(a, lds, lds_b, tm, tn, acc, nullptr, slots, S,
                                               piece);
    if (threadIdx.x == 0)
        __hip_atomic_store(a.sk_flag + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* LDS of the direct-to-LDS pipeline: two stages, each also large enough
 * for half of the waves' epilogue slabs */
template <int WM, int WN, int MI, int NI>
struct GemmLds {
    static constexpr int SLABS = WM * WN / 2 * 32 * (NI * 32 + 4) * 4;
    static constexpr int STAGE = GemmShape<WM, WN, MI, NI>::STAGE;
    static constexpr int BYTES = STAGE > SLABS ? STAGE : SLABS;
};

#define QW_GEMM_ENTRY(name, EPI, INT8, WM, WN, MI, NI)                           \
    QW_KERNEL void __launch_bounds__(64 * WM * WN, 1) name(qw_gemm_args a) {                 \
        __shared__ __attribute__((aligned(16))) unsigned char lds[GemmLds<WM, WN, MI, NI>::BYTES]; \
        __shared__ __attribute__((aligned(16))) unsigned char lds_b[GemmLds<WM, WN, MI, NI>::BYTES]; \
        qw_gemm_impl<EPI, INT8, WM, WN, MI, NI>(a, lds, lds_b);                  \
    }

/* int8 weights widened in the K loop (linears of fewer than 512 rows, where
 * a separate widening pass would not amortise, and the allocation-free
 * entry point): 8 waves (two per SIMD) of 64 x 128 with
 * v_mfma_f32_32x32x16_bf16. bf16 weights run on the 4-wave kernels of
 * gemm_q.h. */
QW_GEMM_ENTRY(qw_gemm_i8_store_w8, QW_EPI_STORE, 1, 4, 2, 2, 4)
QW_GEMM_ENTRY(qw_gemm_i8_gelu_w8, QW_EPI_GELU, 1, 4, 2, 2, 4)
QW_GEMM_ENTRY(qw_gemm_i8_gate_w8, QW_EPI_GATE, 1, 4, 2, 2, 4)
QW_GEMM_ENTRY(qw_gemm_i8_qkn_w8, QW_EPI_QKNORM, 1, 4, 2, 2, 4)

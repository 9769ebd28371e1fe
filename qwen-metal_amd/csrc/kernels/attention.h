/* Block-causal prefix flash attention, D = 128, on CDNA4 matrix cores.
 *
 * One workgroup = 8 waves (256 query rows of one (batch, head), one
 * workgroup per CU, two waves per SIMD), or 4 waves (128 rows, two
 * workgroups per CU) for launches of fewer 256-row blocks than CUs; each
 * wave owns 32 queries. The loop is software pipelined: the QK MFMAs of tile t + 1 are
 * issued between the VALU instructions of tile t's softmax (the first
 * 32-key block under the tile max, the second under the exp / convert).
 *
 * Scores are computed transposed, S^T = K Q^T, with
 * v_mfma_f32_32x32x16_bf16: in that output layout each lane holds ONE query
 * (column lane % 32) and 16 keys per 32-key block, so the row max / row sum
 * of the online softmax need at most one cross-half exchange (lane ^ 32)
 * instead of a 32-lane reduction (the max only when it moves, the sum once
 * at the end), and the per-query rescale of the output is a lane scalar.
 * The output is accumulated transposed too, O^T = V^T P^T: the
 * probabilities stay in registers and feed the MFMA B operand directly.
 * Within each 16-key K-step the keys are permuted identically in the V^T
 * (A) and P^T (B) operands, which leaves the contraction unchanged.
 *
 * K and V tiles (64 keys x 128 d each) go from global memory straight into
 * LDS (buffer_load ... lds), double-buffered, one tile ahead; V keeps its
 * row-major layout and the V^T operand is read with the transposing LDS
 * read of CDNA4 (ds_read_b64_tr_b16), so no register staging, transpose
 * arithmetic or LDS write instruction touches the operands.
 *
 * Softmax runs in fp32 in the log2 domain (scale * log2 e folded into one
 * FMA before exp2; t2i text rows pre-scale q instead); P is rounded to bf16 for the P.V MFMA and the row sum
 * adds the same rounded values. The running max
 * is moved lazily (only when a row's tile max exceeds it by 2^8), which
 * keeps O and l consistent while skipping the rescale on most tiles.
 *
 * Masking: query row r of a batch entry sees keys [0, limit(r)), with
 * limit = kv_limit[r] when given (qwen_dit.h:141-145 prefix tables), else
 * the t2i closed form (qwen_dit.m:1373-1440): text rows causal (or the
 * whole text prefix), image rows every key. KV tiles past the block's
 * largest limit are never loaded. */
#pragma once
#include "common.h"

#define AKB 2                       /* 32-key blocks per tile */
#define AKT (32 * AKB)              /* keys per tile */
#define A_TILE (AKT * 256)          /* one K or V tile: AKT keys x 128 bf16 */

__device__ __forceinline__ uint32_t attn_limit(const qw_attn_args &a, uint32_t r) {
    if (r >= a.q_rows) return 0;
    if (a.kv_limit) return min(a.kv_limit[r], a.kv_rows);
    if (r < a.text_rows) return a.text_causal ? r + 1 : a.text_rows;
    return a.kv_rows;
}

/* Key of s[kbk][v] in a tile: kv0 + 32 kbk + 8 (v / 4) + 4 h + v % 4.
 * Masks keys at or past the row's limit L. */
__device__ __forceinline__ void attn_mask(floatx16 (&s)[AKB], uint32_t kv0, uint32_t L, uint32_t h) {
#pragma unroll
    for (int kbk = 0; kbk < AKB; kbk++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            uint32_t key = kv0 + 32 * kbk + 8 * (v >> 2) + 4 * h + (v & 3);
            if (key >= L) s[kbk][v] = -INFINITY;
        }
}

/* P = exp2(S c - m) rounded to bf16 (the B operand of P.V, one bf16x8 per
 * 16-key K-step) and the lane's part of the row sum, which adds the same
 * rounded values (v_dot2 against ones). */
__device__ __forceinline__ float attn_exp(const floatx16 (&s)[AKB], bf16x8 (&pf)[2 * AKB],
                                          float c, float m_use) {
    float rs = 0.0f;
    const qw_b2 ones = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int tk = 0; tk < 2 * AKB; tk++) {
        const int kbk = tk >> 1, v0 = 8 * (tk & 1);
#pragma unroll
        for (int u = 0; u < 8; u += 2) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kbk][v0 + u], c, -m_use));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kbk][v0 + u + 1], c, -m_use));
            const qw_b2 pp = __builtin_bit_cast(qw_b2, pack_bf(p0, p1));
            pf[tk][u] = pp[0];
            pf[tk][u + 1] = pp[1];
            rs = __builtin_amdgcn_fdot2_f32_bf16(pp, ones, rs, false);
        }
    }
    return rs;
}

__device__ __forceinline__ void attn_store_rows(const qw_attn_args &a, const floatx16 (&o)[4],
                                                float l_run, uint32_t b, uint32_t r,
                                                uint32_t head, uint32_t h) {
    if (r >= a.q_rows) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    u16 *orow = a.out + ((size_t)b * a.q_rows + r) * a.ldo + head * 128;
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t w0 = pack_bf(o[db][4 * g] * inv, o[db][4 * g + 1] * inv);
            uint32_t w1 = pack_bf(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
            *(u32x2 *)(orow + 32 * db + 8 * g + 4 * h) = u32x2{w0, w1};
        }
}

/* One 16-byte-per-lane direct load into LDS (buffer_load_dwordx4 ... lds):
 * M0 = the wave's LDS base, lane l writes base + 16 l. Issued from inline
 * assembly so the compiler does not treat it as a pending LDS store (it
 * would wait for every one in flight before each LDS read); the kernel
 * waits for them itself (vmcnt) before the barrier that publishes a tile. The
 * load reads M0 one wait state after its write at the earliest (gfx9 rule;
 * the compiler does not see inside the asm to insert it). */
__device__ __forceinline__ void attn_dma(u32x4 rsrc, uint32_t lds_base, uint32_t voff,
                                         uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff)
                 : "m0");
}

__device__ __forceinline__ void attn_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

typedef __attribute__((address_space(3))) bf16x4 attn_lds_b4;

/* 256 queries per workgroup: launches that fill the part */
#define ANW 8 /* waves per workgroup, 32 queries each */
#define AQB (32 * ANW) /* queries per workgroup */
#define QW_ATTN_NAME qw_attention_bf16
#include "attention_kernel.inc"
#undef QW_ATTN_NAME
#undef AQB
#undef ANW

/* 128 queries per workgroup, two per CU: launches of fewer 256-query
 * blocks than CUs (the 512^2 and 320-row configurations) */
#define ANW 4
#define AQB (32 * ANW)
#define QW_ATTN_NAME qw_attention_w4_bf16
#include "attention_kernel.inc"
#undef QW_ATTN_NAME
#undef AQB
#undef ANW

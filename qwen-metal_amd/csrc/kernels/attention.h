/* Block-causal prefix flash attention, D = 128, on CDNA4 matrix cores.
 *
 * One workgroup = 4 waves = 128 query rows of one (batch, head); each wave
 * owns 32 queries. Scores are computed transposed, S^T = K Q^T, with
 * v_mfma_f32_32x32x16_bf16: in that output layout each lane holds ONE query
 * (column lane % 32) and 16 keys per 32-key block, so the row max / row sum
 * of the online softmax need one cross-half exchange (lane ^ 32) instead of
 * a 32-lane reduction, and the per-query rescale of the output is a lane
 * scalar. The output is accumulated transposed too, O^T = V^T P^T: the
 * probabilities stay in registers and feed the MFMA B operand directly; the
 * keys of an MFMA K-step are permuted identically in the V^T (A) and P^T
 * (B) operands, which leaves the contraction unchanged.
 *
 * K tiles (64 keys x 128) and V^T tiles (128 x 64 keys) are staged through
 * LDS, double-buffered, with the next tile's global loads in flight during
 * the current tile's math; row padding keeps the MFMA operand reads
 * conflict-free. Softmax runs in fp32 in the log2 domain (scale * log2 e
 * folded into one FMA before exp2); P is rounded to bf16 for the P.V MFMA,
 * the row sum uses the fp32 P.
 *
 * Masking: query row r of a batch entry sees keys [0, limit(r)), with
 * limit = kv_limit[r] when given (qwen_dit.h:141-145 prefix tables), else
 * the t2i closed form (qwen_dit.m:1373-1440): text rows causal (or the
 * whole text prefix), image rows every key. KV tiles past the block's
 * largest limit are never loaded. */
#pragma once
#include "common.h"

#define AQB 128     /* queries per workgroup */
#define AKT 64      /* keys per tile */
#define KS_LD 136   /* K tile row stride (elements) */
#define VT_LD 68    /* V^T tile row stride (elements) */
#define A_K_BYTES (AKT * KS_LD * 2)
#define A_V_BYTES (128 * VT_LD * 2)
#define A_STAGE (A_K_BYTES + A_V_BYTES)

__device__ __forceinline__ uint32_t attn_limit(const qw_attn_args &a, uint32_t r) {
    if (r >= a.q_rows) return 0;
    if (a.kv_limit) return min(a.kv_limit[r], a.kv_rows);
    if (r < a.text_rows) return a.text_causal ? r + 1 : a.text_rows;
    return a.kv_rows;
}

QW_KERNEL void __launch_bounds__(256, 2) qw_attention_bf16(qw_attn_args a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * A_STAGE];
    __shared__ uint32_t lim_red[8];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t h = lane >> 5, j = lane & 31;
    const uint32_t head = blockIdx.y, b = blockIdx.z;
    const uint32_t q0 = blockIdx.x * AQB;
    const uint32_t r = q0 + wave * 32 + j; /* this lane's query row */

    const u16 *qb = a.q + (size_t)b * a.q_rows * a.ldq + head * 128;
    const u16 *kb = a.k + (size_t)b * a.kv_rows * a.ldk + head * 128;
    const u16 *vb = a.v + (size_t)b * a.kv_rows * a.ldv + head * 128;

    /* ---- limits: per lane, then block max / min ------------------------- */
    const uint32_t L = attn_limit(a, r);
    uint32_t lmax = L, lmin = L;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        lmax = max(lmax, (uint32_t)__shfl_xor((int)lmax, o, 64));
        lmin = min(lmin, (uint32_t)__shfl_xor((int)lmin, o, 64));
    }
    if (lane == 0) {
        lim_red[wave] = lmax;
        lim_red[4 + wave] = lmin;
    }
    __syncthreads();
    lmax = max(max(lim_red[0], lim_red[1]), max(lim_red[2], lim_red[3]));
    lmin = min(min(lim_red[4], lim_red[5]), min(lim_red[6], lim_red[7]));
    const uint32_t ntiles = (lmax + AKT - 1) / AKT;

    /* ---- Q^T fragments (B operand), resident for the whole loop --------- */
    bf16x8 qf[8];
    {
        const u16 *qrow = qb + (size_t)min(r, a.q_rows - 1) * a.ldq;
#pragma unroll
        for (int s = 0; s < 8; s++) qf[s] = *(const bf16x8 *)(qrow + 16 * s + 8 * h);
    }

    /* ---- tile loaders ---------------------------------------------------- */
    const uint32_t kc = tid & 15, kr = tid >> 4; /* K: chunk, key (+16 j) */
    const uint32_t vq = (tid >> 4) * 4;          /* V: 4 keys, chunk kc (8 d) */
    u32x4 rk[4], rv[4];
    auto load_tile = [&](uint32_t kv0) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            uint32_t key = min(kv0 + kr + 16 * t, a.kv_rows - 1);
            rk[t] = *(const u32x4 *)(kb + (size_t)key * a.ldk + kc * 8);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            uint32_t key = min(kv0 + vq + t, a.kv_rows - 1);
            rv[t] = *(const u32x4 *)(vb + (size_t)key * a.ldv + kc * 8);
        }
    };
    auto store_tile = [&](uint32_t buf) {
        unsigned char *ks = lds + buf * A_STAGE;
        unsigned char *vt = ks + A_K_BYTES;
#pragma unroll
        for (int t = 0; t < 4; t++)
            *(u32x4 *)(ks + ((kr + 16 * t) * KS_LD + kc * 8) * 2) = rk[t];
        /* transpose 4 keys x 8 d into 8 rows of V^T, 4 keys each */
#pragma unroll
        for (int d = 0; d < 8; d++) {
            const uint32_t w = d >> 1;
            const uint32_t sh = (d & 1) ? 16 : 0;
            uint32_t k01 = ((rv[0][w] >> sh) & 0xffffu) | (((rv[1][w] >> sh) & 0xffffu) << 16);
            uint32_t k23 = ((rv[2][w] >> sh) & 0xffffu) | (((rv[3][w] >> sh) & 0xffffu) << 16);
            *(u32x2 *)(vt + ((kc * 8 + d) * VT_LD + vq) * 2) = u32x2{k01, k23};
        }
    };

    floatx16 o[4];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int v = 0; v < 16; v++) o[db][v] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float c = a.scale_log2;

    if (ntiles) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();
    for (uint32_t t = 0; t < ntiles; t++) {
        const uint32_t cur = t & 1, kv0 = t * AKT;
        if (t + 1 < ntiles) load_tile(kv0 + AKT);
        const unsigned char *ks = lds + cur * A_STAGE;
        const unsigned char *vt = ks + A_K_BYTES;

        /* S^T for keys kv0 + [0, 32) and [32, 64) */
        floatx16 s[2];
#pragma unroll
        for (int kbk = 0; kbk < 2; kbk++) {
#pragma unroll
            for (int v = 0; v < 16; v++) s[kbk][v] = 0.0f;
#pragma unroll
            for (int st = 0; st < 8; st++) {
                bf16x8 kf = *(const bf16x8 *)(ks + ((kbk * 32 + j) * KS_LD + 16 * st + 8 * h) * 2);
                s[kbk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s[kbk], 0, 0, 0);
            }
        }
        /* key of s[kbk][v]: kv0 + 32 kbk + 8 (v / 4) + 4 h + v % 4 */
        if (kv0 + AKT > lmin) {
#pragma unroll
            for (int kbk = 0; kbk < 2; kbk++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    uint32_t key = kv0 + 32 * kbk + 8 * (v >> 2) + 4 * h + (v & 3);
                    if (key >= L) s[kbk][v] = -INFINITY;
                }
        }
        float mt = -INFINITY;
#pragma unroll
        for (int kbk = 0; kbk < 2; kbk++)
#pragma unroll
            for (int v = 0; v < 16; v++) mt = fmaxf(mt, s[kbk][v]);
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float m_new = fmaxf(m_run, mt * c);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float rs = 0.0f;
#pragma unroll
        for (int kbk = 0; kbk < 2; kbk++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kbk][v], c, -m_use));
                s[kbk][v] = p;
                rs += p;
            }
        rs += __shfl_xor(rs, 32, 64);
        l_run = l_run * alpha + rs;
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < 4; db++)
#pragma unroll
            for (int v = 0; v < 16; v++) o[db][v] *= alpha;

        /* O^T += V^T P^T over 4 K-steps of 16 keys */
#pragma unroll
        for (int tk = 0; tk < 4; tk++) {
            const int kbk = tk >> 1, v0 = 8 * (tk & 1);
            bf16x8 pf;
#pragma unroll
            for (int u = 0; u < 8; u++) pf[u] = (__bf16)s[kbk][v0 + u];
#pragma unroll
            for (int db = 0; db < 4; db++) {
                const unsigned char *row = vt + ((db * 32 + j) * VT_LD) * 2;
                u32x2 lo = *(const u32x2 *)(row + (16 * tk + 4 * h) * 2);
                u32x2 hi = *(const u32x2 *)(row + (16 * tk + 8 + 4 * h) * 2);
                u32x4 vv = {lo[0], lo[1], hi[0], hi[1]};
                bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[db], 0, 0, 0);
            }
        }
        if (t + 1 < ntiles) store_tile(cur ^ 1);
        __syncthreads();
    }

    /* ---- normalise and store: o[db][v] = O[r][32 db + 8 (v/4) + 4 h + v%4] */
    if (r < a.q_rows) {
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
}

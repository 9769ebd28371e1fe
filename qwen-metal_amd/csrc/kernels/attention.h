/* Block-causal prefix flash attention, D = 128, on CDNA4 matrix cores.
 *
 * One workgroup = 4 waves = 128 query rows of one (batch, head); each wave
 * owns 32 queries; two workgroups share a CU. The loop is software
 * pipelined: the QK MFMAs of tile t + 1 are issued before the softmax of
 * tile t, so that VALU work can issue under them.
 *
 * Scores are computed transposed, S^T = K Q^T, with
 * v_mfma_f32_32x32x16_bf16: in that output layout each lane holds ONE query
 * (column lane % 32) and 16 keys per 32-key block, so the row max / row sum
 * of the online softmax need one cross-half exchange (lane ^ 32) instead of
 * a 32-lane reduction, and the per-query rescale of the output is a lane
 * scalar. The output is accumulated transposed too, O^T = V^T P^T: the
 * probabilities stay in registers and feed the MFMA B operand directly.
 * Within each 16-key K-step the keys are permuted identically in the V^T
 * (A) and P^T (B) operands, which leaves the contraction unchanged.
 *
 * K tiles (64 keys x 128) and V^T tiles (128 x 64 keys) are staged through
 * LDS, double-buffered, with the next tile's global loads in flight during
 * the current tile's math. Softmax runs in fp32 in the log2 domain (scale *
 * log2 e folded into one FMA before exp2); P is rounded to bf16 for the
 * P.V MFMA and the row sum adds the same rounded values. The running max
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

#define AQB 128     /* queries per workgroup (4 waves x 32) */
#define AKT 64      /* keys per tile */
#define KS_LD 136   /* K tile row stride (elements) */
#define VT_LD 72    /* V^T tile row stride (elements) */
#define A_K_BYTES (AKT * KS_LD * 2)
#define A_V_BYTES (128 * VT_LD * 2)
#define A_STAGE (A_K_BYTES + A_V_BYTES)

__device__ __forceinline__ uint32_t attn_limit(const qw_attn_args &a, uint32_t r) {
    if (r >= a.q_rows) return 0;
    if (a.kv_limit) return min(a.kv_limit[r], a.kv_rows);
    if (r < a.text_rows) return a.text_causal ? r + 1 : a.text_rows;
    return a.kv_rows;
}

/* Key of s[kbk][v] in a 64-key tile: kv0 + 32 kbk + 8 (v / 4) + 4 h + v % 4.
 * Masks keys at or past the row's limit L. */
__device__ __forceinline__ void attn_mask(floatx16 (&s)[2], uint32_t kv0, uint32_t L, uint32_t h) {
#pragma unroll
    for (int kbk = 0; kbk < 2; kbk++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            uint32_t key = kv0 + 32 * kbk + 8 * (v >> 2) + 4 * h + (v & 3);
            if (key >= L) s[kbk][v] = -INFINITY;
        }
}

/* P = exp2(S c - m) rounded to bf16 (the B operand of P.V, one bf16x8 per
 * 16-key K-step) and the lane's part of the row sum, which adds the same
 * rounded values (v_dot2 against ones). */
__device__ __forceinline__ float attn_exp(const floatx16 (&s)[2], bf16x8 (&pf)[4], float c,
                                          float m_use) {
    float rs = 0.0f;
    const qw_b2 ones = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int tk = 0; tk < 4; tk++) {
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

QW_KERNEL void __launch_bounds__(256, 2) qw_attention_bf16(qw_attn_args a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * A_STAGE];
    __shared__ uint32_t lim_red[8];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t h = lane >> 5, j = lane & 31;
    /* Workgroup ids are dealt round-robin to the 8 XCDs; remap them so
     * each XCD owns a contiguous range of (batch, head) pairs and all query
     * blocks of a pair share that XCD's L2 copy of its K and V. */
    const uint32_t nq = (a.q_rows + AQB - 1) / AQB, nwg = nq * a.heads * a.batch;
    uint32_t pid = blockIdx.x;
    if ((nwg & 7u) == 0) pid = (pid & 7u) * (nwg >> 3) + (pid >> 3);
    const uint32_t qblk = pid % nq, head = (pid / nq) % a.heads, b = pid / (nq * a.heads);
    const uint32_t q0 = qblk * AQB;
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

    /* ---- tile loaders ----------------------------------------------------
     * K: 16 lanes per key row (16 B each), stored row-major (stride KS_LD).
     * V: lane (vc = tid / 16, vq = 4 (tid % 16)) loads 8 d (chunk vc) of the
     * 4 keys vq..vq+3 and stores them transposed, 4 keys per 8-byte write
     * into rows vc*8 + d of V^T. Inside every 16-key group the 4-key
     * quarters are stored in the order 0, 2, 1, 3, so that the 8 keys an
     * MFMA lane needs (quarters {0, 2} for k-half 0, {1, 3} for k-half 1,
     * the key order of the P^T operand) are 16 contiguous bytes. With a
     * 144-byte row both the writes (two rows 8 apart per pass) and the
     * 16-byte reads (16 rows per pass) hit distinct banks.
     * The K tile runs one tile ahead of the V tile (QK of tile t + 1 is
     * computed while the softmax of tile t runs), so each has its own pair
     * of stages: K of tile x in stage x % 2, V of tile x in stage x % 2. */
    const uint32_t kc = tid & 15, kr = tid >> 4; /* K: chunk, key (+16 t) */
    const uint32_t vc = tid >> 4, vq = (tid & 15) * 4;
    const uint32_t vcol = (vq & ~15u) | ((((vq >> 2) & 1) << 1 | ((vq >> 3) & 1)) << 2);
    u32x4 rk[4], rv[4];
    auto load_k = [&](uint32_t kv0) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            uint32_t key = min(kv0 + kr + 16 * t, a.kv_rows - 1);
            rk[t] = *(const u32x4 *)(kb + (size_t)key * a.ldk + kc * 8);
        }
    };
    auto load_v = [&](uint32_t kv0) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            uint32_t key = min(kv0 + vq + t, a.kv_rows - 1);
            rv[t] = *(const u32x4 *)(vb + (size_t)key * a.ldv + vc * 8);
        }
    };
    auto store_k = [&](uint32_t buf) {
        unsigned char *ks = lds + buf * A_STAGE;
#pragma unroll
        for (int t = 0; t < 4; t++)
            *(u32x4 *)(ks + ((kr + 16 * t) * KS_LD + kc * 8) * 2) = rk[t];
    };
    auto store_v = [&](uint32_t buf) {
        unsigned char *vt = lds + buf * A_STAGE + A_K_BYTES;
#pragma unroll
        for (int d = 0; d < 8; d++) {
            const uint32_t w = d >> 1;
            const uint32_t sh = (d & 1) ? 16 : 0;
            uint32_t k01 = ((rv[0][w] >> sh) & 0xffffu) | (((rv[1][w] >> sh) & 0xffffu) << 16);
            uint32_t k23 = ((rv[2][w] >> sh) & 0xffffu) | (((rv[3][w] >> sh) & 0xffffu) << 16);
            *(u32x2 *)(vt + ((vc * 8 + d) * VT_LD + vcol) * 2) = u32x2{k01, k23};
        }
    };
    /* S^T of one tile: keys kv0 + [0, 32) and [32, 64) */
    auto qk = [&](const unsigned char *ks, floatx16 (&s)[2]) {
#pragma unroll
        for (int kbk = 0; kbk < 2; kbk++) {
#pragma unroll
            for (int v = 0; v < 16; v++) s[kbk][v] = 0.0f;
#pragma unroll
            for (int st = 0; st < 8; st++) {
                const bf16x8 kf =
                    *(const bf16x8 *)(ks + ((kbk * 32 + j) * KS_LD + 16 * st + 8 * h) * 2);
                s[kbk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s[kbk], 0, 0, 0);
            }
        }
    };

    floatx16 o[4];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int v = 0; v < 16; v++) o[db][v] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float c = a.scale_log2;

    /* prologue: K(0), V(0), K(1) staged; S(0) computed */
    floatx16 s0[2], s1[2];
    if (ntiles) {
        load_k(0);
        load_v(0);
        store_k(0);
        store_v(0);
        load_k(AKT);
        store_k(1);
    }
    __syncthreads();
    if (ntiles) qk(lds, s0);

    /* One tile. Straight-line except the masking of boundary tiles and the
     * rare running-max move, so the QK MFMAs of tile t + 1 and the softmax
     * VALU work of tile t share one scheduling region, as do the P.V MFMAs
     * and the next tiles' LDS stores. Past the end, loads and QK run on
     * clamped or stale tiles whose results nobody reads. */
    auto iter = [&](floatx16 (&sc)[2], floatx16 (&sn)[2], uint32_t t) __attribute__((always_inline)) {
        const uint32_t kv0 = t * AKT;
#if !defined(QW_AEXP_NOLOAD) && !defined(QW_AEXP_NOK)
        load_k(kv0 + 2 * AKT); /* stored after this tile's math */
#endif
#if !defined(QW_AEXP_NOLOAD) && !defined(QW_AEXP_NOV)
        load_v(kv0 + AKT);
#endif
        if (kv0 + AKT > lmin) attn_mask(sc, kv0, L, h);

        qk(lds + ((t + 1) & 1) * A_STAGE, sn);
        float mt = -INFINITY;
#pragma unroll
        for (int kbk = 0; kbk < 2; kbk++)
#pragma unroll
            for (int v = 0; v < 16; v++) mt = fmaxf(mt, sc[kbk][v]);
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        /* Lazy running max: it moves only when a row's tile max exceeds it
         * by more than 2^8 (or on the first finite max), so p <= 256 and O,
         * l stay consistent; a move rescales and redoes this tile's P. */
        const float m_new = mt * c;
        const bool move = m_new > m_run + 8.0f;
        bf16x8 pf[4];
#ifdef QW_AEXP_NOSOFTMAX
        float rs = 1.0f;
#pragma unroll
        for (int tk = 0; tk < 4; tk++)
#pragma unroll
            for (int u = 0; u < 8; u++) pf[tk][u] = (__bf16)sc[tk >> 1][8 * (tk & 1) + u];
#else
        float rs = attn_exp(sc, pf, c, m_run == -INFINITY ? 0.0f : m_run);
#endif
        /* QK MFMAs of the next tile with the max/exp VALU and the K
         * fragment reads between them */
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0); /* fragment reads run 2 ahead */
#pragma unroll
        for (int i = 0; i < 16; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
        }
        if (__builtin_amdgcn_ballot_w64(move)) {
            const float m_to = move ? m_new : m_run;
            const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_to);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; db++)
#pragma unroll
                for (int v = 0; v < 16; v++) o[db][v] *= alpha;
            m_run = m_to;
            rs = attn_exp(sc, pf, c, m_run == -INFINITY ? 0.0f : m_run);
        }
        rs += __shfl_xor(rs, 32, 64);
        l_run += rs;

        /* O^T += V^T P^T over 4 K-steps of 16 keys */
        const unsigned char *vt = lds + (t & 1) * A_STAGE + A_K_BYTES;
#pragma unroll
        for (int tk = 0; tk < 4; tk++) {
#pragma unroll
            for (int db = 0; db < 4; db++) {
                const bf16x8 vf =
                    *(const bf16x8 *)(vt + ((db * 32 + j) * VT_LD + 16 * tk + 8 * h) * 2);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[tk], o[db], 0, 0, 0);
            }
        }
        /* K stage t % 2 (tile t, read by last iteration's QK) and V stage
         * (t + 1) % 2 (tile t - 1) are free: every wave passed the barrier
         * that ended the iteration which read them, and this iteration
         * reads only the other two */
#if !defined(QW_AEXP_NOLOAD) && !defined(QW_AEXP_NOK)
        store_k(t & 1);
#endif
#if !defined(QW_AEXP_NOLOAD) && !defined(QW_AEXP_NOV)
#ifdef QW_AEXP_NOVT
        {
            unsigned char *vt = lds + ((t + 1) & 1) * A_STAGE + A_K_BYTES;
#pragma unroll
            for (int q = 0; q < 4; q++) *(u32x4 *)(vt + (tid * 4 + q) * 16) = rv[q];
        }
#else
        store_v((t + 1) & 1);
#endif
#endif
        __syncthreads();
    };
    uint32_t t = 0;
    for (; t + 1 < ntiles; t += 2) {
        iter(s0, s1, t);
        iter(s1, s0, t + 1);
    }
    if (t < ntiles) iter(s0, s1, t);

    /* ---- normalise and store: o[db][v] = O[r][32 db + 8 (v/4) + 4 h + v%4] */
    attn_store_rows(a, o, l_run, b, r, head, h);
}

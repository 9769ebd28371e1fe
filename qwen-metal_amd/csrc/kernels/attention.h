/* Block-causal prefix flash attention, D = 128, on CDNA4 matrix cores.
 *
 * One workgroup = QW_ATTN_WAVES waves (8: 256 query rows of one (batch,
 * head), one workgroup per CU, two waves per SIMD); each wave owns 32
 * queries. The loop is software pipelined: the QK MFMAs of tile t + 1 are
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
#define ANW QW_ATTN_WAVES           /* waves per workgroup, 32 queries each */
#define AQB (32 * ANW)              /* queries per workgroup */
#define A_TILE (AKT * 256)          /* one K or V tile: AKT keys x 128 bf16 */
static_assert(AQB == QW_ATTN_QROWS, "queries per workgroup");

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

QW_KERNEL void __launch_bounds__(64 * ANW, 8 / ANW) qw_attention_bf16(qw_attn_args a) {
    /* K stages 0, 1 then V stages 0, 1; AKT keys x 256 B each */
    __shared__ __attribute__((aligned(16))) unsigned char lds[4 * A_TILE];
    __shared__ uint32_t lim_red[2 * ANW];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
        lim_red[ANW + wave] = lmin;
    }
    __syncthreads();
    lmax = 0;
    lmin = 0xffffffffu;
#pragma unroll
    for (int w = 0; w < ANW; w++) {
        lmax = max(lmax, lim_red[w]);
        lmin = min(lmin, lim_red[ANW + w]);
    }
    const uint32_t ntiles = (lmax + AKT - 1) / AKT;

    /* t2i text rows follow the reference's text-row kernel
     * (h3_shaders.metal:4397-4401): q is multiplied by the softmax scale
     * and re-rounded to bf16 before QK, and the scores are not scaled
     * again (their exp2 factor is log2 e alone). Prefix tables (ti2i) and
     * image rows keep bf16 q with the scale folded into the exp2 FMA. */
    const bool prescale = !a.kv_limit && r < a.text_rows;
    const float c = prescale ? 1.4426950408889634f : a.scale_log2;

    /* ---- Q^T fragments (B operand), resident for the whole loop --------- */
    bf16x8 qf[8];
    {
        const u16 *qrow = qb + (size_t)min(r, a.q_rows - 1) * a.ldq;
#pragma unroll
        for (int s = 0; s < 8; s++) qf[s] = *(const bf16x8 *)(qrow + 16 * s + 8 * h);
        if (prescale) { /* t2i text rows: q' = bf16(q * scale) */
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    qf[s][e] = (__bf16)((float)qf[s][e] * a.scale);
        }
    }
    floatx16 o[4];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int v = 0; v < 16; v++) o[db][v] = 0.0f;

    /* ---- K / V tiles: AKT keys x 128 d, row-major (256 B rows), straight
     * from global memory into LDS. 16-byte chunk c of key row k sits at
     * chunk c ^ (k % 16) in K tiles (the 16 rows of one QK fragment read
     * pass hit 16 distinct chunks) and at c ^ 4 (k % 4) in V tiles (the 4
     * rows x 64 B of one transposing read pass hit 16 distinct chunks).
     * A direct load covers 1 KB = 4 rows; lane l lands on row l / 16,
     * physical chunk l % 16, and fetches the logical chunk the swizzle puts
     * there. */
    constexpr int DPW = AKT / 4 / ANW; /* direct loads per wave per tile */
    static_assert(DPW * ANW * 4 == AKT, "K/V tile loads must split evenly over the waves");
    u32x4 rk, rv;
    {
        const uint64_t kbase = (uint64_t)kb, vbase = (uint64_t)vb;
        const uint32_t kbytes = (uint32_t)(((size_t)(a.kv_rows - 1) * a.ldk + 128) * 2);
        const uint32_t vbytes = (uint32_t)(((size_t)(a.kv_rows - 1) * a.ldv + 128) * 2);
        rk = u32x4{(uint32_t)kbase, (uint32_t)(kbase >> 32) & 0xffffu, kbytes, 0x00020000u};
        rv = u32x4{(uint32_t)vbase, (uint32_t)(vbase >> 32) & 0xffffu, vbytes, 0x00020000u};
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)lds;
    const uint32_t drow = lane >> 4, dphys = lane & 15;
    /* lane offsets of the wave's loads relative to the tile's first key row
     * (whose byte offset kv0 * ld * 2 goes in the scalar offset); rows past
     * the last key are clamped to it, which only the last tile needs */
    uint32_t kvo[DPW], vvo[DPW];
#pragma unroll
    for (int jj = 0; jj < DPW; jj++) {
        const uint32_t row = (wave * DPW + jj) * 4 + drow;
        kvo[jj] = (row * a.ldk + ((dphys ^ (row & 15)) * 8)) * 2;
        vvo[jj] = (row * a.ldv + ((dphys ^ (4 * (row & 3))) * 8)) * 2;
    }
    auto issue = [&](uint32_t kstage, uint32_t kv0k, uint32_t vstage, uint32_t kv0v)
        __attribute__((always_inline)) {
        if (kv0k + AKT <= a.kv_rows) {
#pragma unroll
            for (int jj = 0; jj < DPW; jj++) {
                const uint32_t blk = wave * DPW + jj; /* 1 KB block of the tile */
                attn_dma(rk, lds0 + kstage * A_TILE + blk * 1024, kvo[jj], kv0k * a.ldk * 2);
                attn_dma(rv, lds0 + (2 + vstage) * A_TILE + blk * 1024, vvo[jj],
                         kv0v * a.ldv * 2);
            }
            return;
        }
#pragma unroll
        for (int jj = 0; jj < DPW; jj++) {
            const uint32_t blk = wave * DPW + jj;
            const uint32_t row = blk * 4 + drow;
            const uint32_t kk = min(kv0k + row, a.kv_rows - 1);
            attn_dma(rk, lds0 + kstage * A_TILE + blk * 1024,
                     (kk * a.ldk + ((dphys ^ (row & 15)) * 8)) * 2, 0);
            const uint32_t kvv = min(kv0v + row, a.kv_rows - 1);
            attn_dma(rv, lds0 + (2 + vstage) * A_TILE + blk * 1024,
                     (kvv * a.ldv + ((dphys ^ (4 * (row & 3))) * 8)) * 2, 0);
        }
    };
    /* S^T of one tile: keys kv0 + 32 kbk + [0, 32), one MFMA per 16-d step;
     * steps [i0, i1) of the 8 AKB (kbk, st) pairs, st-major, so consecutive
     * MFMAs go to the AKB independent accumulators (measured 1% faster than
     * running each accumulator's 8 dependent MFMAs back to back) */
    auto qk = [&](uint32_t kstage, floatx16 (&s)[AKB], int i0, int i1) __attribute__((always_inline)) {
        const unsigned char *ks = lds + kstage * A_TILE;
#pragma unroll
        for (int i = i0; i < i1; i++) {
            const int kbk = i % AKB, st = i / AKB;
            if (st == 0) {
#pragma unroll
                for (int v = 0; v < 16; v++) s[kbk][v] = 0.0f;
            }
            const bf16x8 kf = *(const bf16x8 *)(ks + (kbk * 32 + j) * 256 +
                                                (((2 * st + h) ^ (j & 15)) << 4));
            s[kbk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s[kbk], 0, 0, 0);
        }
    };
    /* V^T operand by transposing reads (ds_read_b64_tr_b16): in each 16-lane
     * group, result lane i element e comes from source lane 4e + i / 4,
     * element i % 4. Source lane 4e + q reads key row rowbase + e, d =
     * d_base + 4q..+3, so result lane i holds keys rowbase + 0..3 of column
     * d_base + i: the A operand of O^T += V^T P^T, in the key order of P^T
     * (rows 16 tk + 4 h + 0..3, then 16 tk + 8 + 4 h + 0..3). */
    const uint32_t tq = lane & 3, te = (lane >> 2) & 3;
    const uint32_t tdb = 16 * ((lane >> 4) & 1) + 4 * tq; /* d offset inside a 32-d block */
    auto read_v = [&](uint32_t vstage, int tk, int db) __attribute__((always_inline)) {
        const unsigned char *vs = lds + (2 + vstage) * A_TILE;
        const uint32_t d = 32 * db + tdb, cc = d >> 3, half = (d >> 2) & 1;
        const uint32_t r0 = 16 * tk + 4 * h + te, r1 = r0 + 8;
        const bf16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (attn_lds_b4 *)(vs + r0 * 256 + ((cc ^ (4 * (r0 & 3))) << 4) + half * 8));
        const bf16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (attn_lds_b4 *)(vs + r1 * 256 + ((cc ^ (4 * (r1 & 3))) << 4) + half * 8));
        return bf16x8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
    };
    /* vpre: the V^T fragments of the first VPRE 16-key steps, read at the
     * top of the tile (V(t) landed at the previous barrier) so the first P.V
     * MFMAs do not wait on LDS (one step: two would spill beside the scores
     * the softmax keeps for its rare path) */
    constexpr int VPRE = 1;
    auto pv = [&](uint32_t vstage, const bf16x8 (&pf)[2 * AKB], const bf16x8 (&vpre)[VPRE > 0 ? VPRE : 1][4])
        __attribute__((always_inline)) {
#pragma unroll
        for (int tk = 0; tk < 2 * AKB; tk++) {
#pragma unroll
            for (int db = 0; db < 4; db++) {
                const bf16x8 vf = tk < VPRE ? vpre[tk < VPRE ? tk : 0][db] : read_v(vstage, tk, db);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[tk], o[db], 0, 0, 0);
            }
        }
    };

    float m_run = -INFINITY, l_run = 0.0f; /* l_run: this lane's half of the keys */
    /* Online-softmax step of a tile whose S is in `sc`, with the QK MFMAs of
     * the next tile (into `sn`) laid out between its VALU work: P =
     * bf16(exp2(S c - m)) and the row sum. The running max m moves lazily:
     * only when a row's tile max exceeds it by more than 8 (log2 units), or
     * on the first finite max, so p <= 2^8; a move rescales O and l and
     * recomputes P (a rare, wave-uniform branch). */
    /* VALU instructions placed after each QK MFMA (measured: 2 ahead of 1,
     * 3, 4, 5, 6, 8, 10 and of no placement hints, by 0.5-2%) */
    constexpr int QK_NV = 2;
    auto softmax_qk = [&](floatx16 (&sc)[AKB], bf16x8 (&pf)[2 * AKB], uint32_t kv0,
                          uint32_t kstage_next, floatx16 (&sn)[AKB]) __attribute__((always_inline)) {
        if (kv0 + AKT > lmin) attn_mask(sc, kv0, L, h);
        /* P with the running max as it stands; the QK MFMAs of the next tile
         * are laid out between the exp, convert and sum VALU instructions,
         * their K fragment reads two MFMAs ahead */
        float rs = attn_exp(sc, pf, c, m_run == -INFINITY ? 0.0f : m_run);
        qk(kstage_next, sn, 0, 8 * AKB);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
        for (int i = 0; i < 8 * AKB; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, QK_NV, 0);
            if (i + 2 < 8 * AKB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        /* The running max moves when the tile max exceeds it by more than 8
         * (log2 units), i.e. when some p would exceed 2^8; every p is at most
         * this half's sum of the rounded p, so a half whose sum stays below
         * 256 needs no move. Only otherwise (and while the max of a row
         * that sees any key is still -inf) is the tile max computed and the
         * rule applied, with P recomputed after a move: the same P, l and O
         * as applying the rule on every tile. A row that sees no key (past
         * q_rows) keeps m = -inf, P = 0 and l = 0 either way. */
        if (__builtin_amdgcn_ballot_w64(rs >= 256.0f || (m_run == -INFINITY && L != 0))) {
            float mt = -INFINITY;
#pragma unroll
            for (int kbk = 0; kbk < AKB; kbk++)
#pragma unroll
                for (int v = 0; v < 16; v++) mt = fmaxf(mt, sc[kbk][v]);
            const float m_new = fmaxf(mt, __shfl_xor(mt, 32, 64)) * c;
            const bool move = m_new > m_run + 8.0f;
            if (__builtin_amdgcn_ballot_w64(move)) {
                const float m_to = move ? m_new : m_run;
                const float alpha =
                    m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_to);
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < 4; db++)
#pragma unroll
                    for (int v = 0; v < 16; v++) o[db][v] *= alpha;
                m_run = m_to;
                rs = attn_exp(sc, pf, c, m_run == -INFINITY ? 0.0f : m_run);
            }
        }
        l_run += rs; /* this half's keys; the halves are added at the end */
    };

    /* prologue: K(0), V(0), K(1) staged; S(0) computed */
    floatx16 s0[AKB], s1[AKB];
    if (ntiles) {
        issue(0, 0, 0, 0);
        issue(1, AKT, 1, AKT); /* V(1) lands early; harmless */
    }
    __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0) */
    attn_barrier();
    if (ntiles) qk(0, s0, 0, 8 * AKB);
    /* One tile: issue K(t + 2) and V(t + 1) into the stages tile t - 1 used
     * (their readers passed the previous barrier), QK of tile t + 1, the
     * softmax and P.V of tile t, then wait for the issued tiles and
     * barrier. Past the end, loads are clamped and results unused. */
    auto iter = [&](floatx16 (&sc)[AKB], floatx16 (&sn)[AKB], uint32_t t, auto odd)
        __attribute__((always_inline)) {
        constexpr uint32_t st = decltype(odd)::value; /* t & 1, known at compile time */
        const uint32_t kv0 = t * AKT;
        issue(st, kv0 + 2 * AKT, st ^ 1, kv0 + AKT);
        bf16x8 vpre[VPRE > 0 ? VPRE : 1][4];
#pragma unroll
        for (int tk = 0; tk < VPRE; tk++)
#pragma unroll
            for (int db = 0; db < 4; db++) vpre[tk][db] = read_v(st, tk, db);
        bf16x8 pf[2 * AKB];
        softmax_qk(sc, pf, kv0, st ^ 1, sn);
        pv(st, pf, vpre);
        __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0): K(t + 2), V(t + 1) landed */
        attn_barrier();
    };
    uint32_t t = 0;
    for (; t + 1 < ntiles; t += 2) {
        iter(s0, s1, t, std::integral_constant<uint32_t, 0>());
        iter(s1, s0, t + 1, std::integral_constant<uint32_t, 1>());
    }
    if (t < ntiles) iter(s0, s1, t, std::integral_constant<uint32_t, 0>());

    /* ---- normalise and store: o[db][v] = O[r][32 db + 8 (v/4) + 4 h + v%4] */
    attn_store_rows(a, o, l_run + __shfl_xor(l_run, 32, 64), b, r, head, h);
}

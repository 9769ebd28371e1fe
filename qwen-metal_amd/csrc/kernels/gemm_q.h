/* The linears' GEMM on CDNA4 matrix cores: out[m, n] = epi(sum_k A[m, k]
 * W[n, k]), W bf16 or int8 (the "_w8" kernels: widened to bf16 in LDS once
 * per workgroup; per-row scale in the epilogue), fp32 accumulation, issued
 * as C^T = W A^T (W fragment as the A operand).
 *
 * Geometry: a 256 x 256 tile per workgroup of 4 waves (2 x 2), one wave per
 * SIMD, each wave a 128 x 128 block of 8 x 8 v_mfma_f32_16x16x32_bf16 tiles
 * whose 64 accumulators (256 fp32 per lane) sit in the accumulation
 * registers. Against 8 waves of 64 x 128 it reads a third fewer operand
 * bytes from LDS per MFMA (each wave's fragments serve 128 rows and 128
 * columns); each sub-step of 32 k is 64 independent MFMAs (1024
 * matrix-pipe cycles) under which its 16 fragment reads and the next
 * K-slice's direct loads are issued.
 *
 * Pipeline: K-slices of 64 in two LDS stages (A 256 rows x 128 B, then W),
 * the next slice's loads in flight while the current one is multiplied. A
 * and bf16 W go from global memory straight into LDS (buffer_load_dwordx4
 * ... lds, 1 KB = 8 rows per instruction). 16-byte chunks are XOR-swizzled
 * by (row / 2) % 8, which a fragment read (16 rows, one chunk) and the
 * loads' landing slots both respect. Each slice's second sub-step is held
 * back and multiplied after the slice barrier, under the next slice's
 * loads and first fragment reads, so the matrix pipe does not drain at the
 * barrier. (A ring of four 32-k stages, loads three slices ahead, measured
 * 10-14% slower: twice the barriers and half-line loads.)
 *
 * Tiles: one workgroup per CU walks the tiles in strides of the grid
 * (XCD-consistent), so a tile's output stores drain under the next tile's
 * loads; a partly filled last wave of tiles can instead be cut into
 * k-ranges whose fp32 partials meet in memory (split tiles). */
#pragma once
#include "gemm.h"

#define QG_A_BYTES (256 * 128) /* 256 rows x 64 bf16 */
#define QG_STAGE (2 * QG_A_BYTES)

struct QgCtx {
    u32x4 a_rs4, w_rs4;
    uint32_t a_dvoff[8], w_dvoff[8];
    uint32_t dst0;           /* this wave's 64-row share of a stage */
    uint32_t wdst0;          /* the same for the W tile (half tiles: A has 32 rows per wave) */
    uint32_t a_frag, w_frag; /* fragment row base (rows + lane % 16) in bytes */
    uint32_t ch[2];          /* swizzled 16-byte chunk of sub-step 0 / 1 */
};

/* acc += W-fragment x A-fragment, in place. The accumulator is an operand
 * tied to the result, so each of the wave's 64 accumulators keeps one set
 * of accumulation registers for the whole loop (with the compiler builtin
 * and a fixed interleave the register allocator rotated them through
 * ordinary registers: hundreds of copies per K-slice). Volatile: the
 * MFMAs, the direct loads and the fragment reads issue in source order. */
#define QG_MFMA(acc, w, x) \
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(w), "v"(x))
/* The first MFMA of an accumulator (srcC = 0) defines it: no zeroing
 * instruction precedes the MFMAs. An asm MFMA is invisible to the compiler's
 * hazard tracking, so a VALU write of an accumulator placed right before the
 * MFMA that reads it (fewer than the 2 wait states gfx9 requires) would feed
 * it the old value; with no such writes there is nothing to misplace. */
#define QG_MFMA0(acc, w, x) \
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(acc) : "v"(w), "v"(x))

/* A VALU write of an MFMA operand needs 2 wait states before the MFMA that
 * reads it, and the compiler does not see the asm MFMAs to insert them. This
 * fence takes the fragments as inputs, so whatever writes them (int8
 * widening, register copies) is placed before it, and supplies the 2. */
template <int N = 8>
__device__ __forceinline__ void qg_ready(const bf16x8 (&f)[8]) {
    static_assert(N == 4 || N == 7 || N == 8, "fragment count");
    if constexpr (N == 8)
        asm volatile("s_nop 1" ::"v"(f[0]), "v"(f[1]), "v"(f[2]), "v"(f[3]), "v"(f[4]), "v"(f[5]),
                     "v"(f[6]), "v"(f[7]));
    else if constexpr (N == 4)
        asm volatile("s_nop 1" ::"v"(f[0]), "v"(f[1]), "v"(f[2]), "v"(f[3]));
    else
        asm volatile("s_nop 1" ::"v"(f[0]), "v"(f[1]), "v"(f[2]), "v"(f[3]), "v"(f[4]), "v"(f[5]),
                     "v"(f[6]));
}

/* fragment j of a sub-step, in the order its MFMAs consume them (W block 0,
 * A blocks 0..MB-1, W blocks 1-7) */
template <int MB = 8, int AB = QG_A_BYTES>
__device__ __forceinline__ void qg_read(const QgCtx &c, const unsigned char *cur, uint32_t ch,
                                        bf16x8 (&af)[8], bf16x8 (&bw)[8], int j) {
    if (j == 0)
        bw[0] = *(const bf16x8 *)(cur + AB + c.w_frag + ch);
    else if (j <= MB)
        af[j - 1] = *(const bf16x8 *)(cur + c.a_frag + (j - 1) * 2048 + ch);
    else
        bw[j - MB] = *(const bf16x8 *)(cur + AB + c.w_frag + (j - MB) * 2048 + ch);
}

/* One 64-k slice: the stage `cur` is multiplied while slice k_next streams
 * into `nxt`. The slice's second sub-step is held back (its fragments in
 * pa, pw) and runs at the start of the next slice, after the barrier, while
 * that slice's direct loads and first fragments are issued: one direct load
 * and one fragment read every 4 MFMAs (measured 7-10% faster than the 16
 * direct loads issued back to back, than the loads spread over both
 * sub-steps, and than the read placed before the load); under the 64 MFMAs
 * of sub-step 0 the 16 fragments of sub-step 1 are read, one every 4 MFMAs
 * (256-row tiles; 224-row tiles: 56 MFMAs, 15 loads and reads, the last
 * ones right after their MFMAs). */
template <bool PREV, int MB = 8, int AB = QG_A_BYTES>
__device__ __forceinline__ void qg_slice(const QgCtx &c, floatx4 (&acc)[8][8], bf16x8 (&pa)[8],
                                         bf16x8 (&pw)[8], const unsigned char *__restrict__ cur,
                                         unsigned char *__restrict__ nxt, uint32_t k_next) {
    /* MB A blocks of 16 rows per wave (8: 256-row tiles, 7: 224-row
     * tiles): 8 MB MFMAs per sub-step; MB + 8 direct loads (A, then W) and
     * fragment reads, those past the one-per-4-MFMAs slots right after */
    constexpr int NM = 8 * MB, NL = MB + 8;
    const uint32_t nl = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)nxt;
    auto dma = [&](int j) __attribute__((always_inline)) {
        if (j < MB)
            gemm_dma16(c.a_rs4, nl + c.dst0 + j * 1024, c.a_dvoff[j], k_next * 2);
        else
            gemm_dma16(c.w_rs4, nl + AB + (MB == 8 ? c.dst0 : c.wdst0) + (j - MB) * 1024,
                       c.w_dvoff[j - MB], k_next * 2);
    };
    bf16x8 af[8], bw[8], af1[8], bw1[8];
    if (PREV) {
        qg_ready(pw);
        qg_ready<MB>(pa);
#pragma unroll
        for (int i = 0; i < NM; i++) {
            QG_MFMA(acc[i % MB][i / MB], pw[i / MB], pa[i % MB]);
            if ((i & 3) == 1) dma(i >> 2);
            if ((i & 3) == 3) qg_read<MB, AB>(c, cur, c.ch[0], af, bw, i >> 2);
        }
#pragma unroll
        for (int j = NM / 4; j < NL; j++) {
            dma(j);
            qg_read<MB, AB>(c, cur, c.ch[0], af, bw, j);
        }
    } else {
#pragma unroll
        for (int j = 0; j < NL; j++) dma(j);
#pragma unroll
        for (int j = 0; j < NL; j++) qg_read<MB, AB>(c, cur, c.ch[0], af, bw, j);
    }
#pragma unroll
    for (int i = 0; i < NM; i++) {
        if (PREV)
            QG_MFMA(acc[i % MB][i / MB], bw[i / MB], af[i % MB]);
        else
            QG_MFMA0(acc[i % MB][i / MB], bw[i / MB], af[i % MB]);
        if ((i & 3) == 3) qg_read<MB, AB>(c, cur, c.ch[1], af1, bw1, i >> 2);
    }
#pragma unroll
    for (int j = NM / 4; j < NL; j++) qg_read<MB, AB>(c, cur, c.ch[1], af1, bw1, j);
#pragma unroll
    for (int i = 0; i < MB; i++) pa[i] = af1[i];
#pragma unroll
    for (int i = 0; i < 8; i++) pw[i] = bw1[i];
}

/* Sums of tile (tm, tn) over k-steps [kb, ke) into acc; ends with the LDS
 * stages free (after a barrier). MB = 8: 256-row tiles; MB = 7: 224-row
 * tiles (each wave's 112 rows; the A stage's last 32 rows unused). */
template <int MB = 8>
__device__ __forceinline__ void qg_mainloop(const qw_gemm_args &a, unsigned char *lds,
                                            unsigned char *lds_b, uint32_t tm, uint32_t tn,
                                            uint32_t kb, uint32_t ke, floatx4 (&acc)[8][8]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = tm * (MB * 32), n0 = tn * 256;
    QgCtx c;
    const uint32_t lrow = lane >> 3, lp = lane & 7;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t r = wave * 64 + j * 8 + lrow;
        const uint32_t ra = wave * (MB * 8) + j * 8 + lrow; /* A row: 8 MB rows per wave */
        if (j < MB)
            c.a_dvoff[j] = (min(m0 + ra, a.m - 1) * a.lda + (lp ^ ((ra >> 1) & 7u)) * 8) * 2;
        c.w_dvoff[j] = (min(n0 + r, a.n - 1) * a.k + (lp ^ ((r >> 1) & 7u)) * 8) * 2;
    }
    c.a_rs4 = gemm_rs4(a.a, a.a_bytes);
    c.w_rs4 = gemm_rs4(a.w, a.w_bytes);
    c.dst0 = wave * (MB * 8) * 128;
    c.wdst0 = wave * 64 * 128;
    const uint32_t l16 = lane & 15, h = lane >> 4, swz = (l16 >> 1) & 7u;
    c.a_frag = (wm * (MB * 16) + l16) * 128;
    c.w_frag = (wn * 128 + l16) * 128;
    c.ch[0] = ((0 + h) ^ swz) << 4;
    c.ch[1] = ((4 + h) ^ swz) << 4;
    const uint32_t KT = ke;
    {
        const uint32_t nb =
            (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)lds;
#pragma unroll
        for (int j = 0; j < MB; j++)
            gemm_dma16(c.a_rs4, nb + c.dst0 + j * 1024, c.a_dvoff[j], kb * GBK * 2);
#pragma unroll
        for (int j = 0; j < 8; j++)
            gemm_dma16(c.w_rs4, nb + QG_A_BYTES + (MB == 8 ? c.dst0 : c.wdst0) + j * 1024,
                       c.w_dvoff[j], kb * GBK * 2);
    }
    QW_SLICE_END();
    bf16x8 pa[8], pw[8];
    qg_slice<false, MB>(c, acc, pa, pw, lds, lds_b, (kb + 1 < KT ? kb + 1 : kb) * GBK);
    QW_SLICE_END();
    uint32_t kt = kb + 1;
    for (; kt + 1 < KT; kt += 2) {
        qg_slice<true, MB>(c, acc, pa, pw, lds_b, lds, (kt + 1) * GBK);
        QW_SLICE_END();
        qg_slice<true, MB>(c, acc, pa, pw, lds, lds_b, (kt + 2 < KT ? kt + 2 : kt + 1) * GBK);
        QW_SLICE_END();
    }
    if (kt < KT) {
        qg_slice<true, MB>(c, acc, pa, pw, lds_b, lds, kt * GBK);
        QW_SLICE_END();
    }
    qg_ready(pw);
    qg_ready<MB>(pa);
#pragma unroll
    for (int i = 0; i < 8 * MB; i++) QG_MFMA(acc[i % MB][i / MB], pw[i / MB], pa[i % MB]);
    /* the epilogue reads the accumulators with ordinary instructions: let
     * the last MFMAs' results land first (the inline assembly hides them
     * from the compiler's hazard tracking) */
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}

/* Half tiles (MB = 4) with three LDS stages of 48 KB (A 16 KB, then W
 * 32 KB), loads two slices ahead: for launches of at most half as many
 * tiles as CUs, whose slices are bound by the load latency rather than the
 * MFMAs (one slice ahead, a 128 x 256 slice takes most of a 256 x 256
 * slice's time). Slice j is computed from stage j % 3 while slice j + 2
 * streams into stage (j + 2) % 3, the stage slice j - 1 was computed from;
 * each slice ends waiting for all but the newest slice's loads. Slices past
 * ke - 1 reload ke - 1 so that every slice issues the same loads. Ends
 * with the LDS free (all loads landed, after a barrier). */
#define QG3_AB (4 * 32 * 128)         /* A bytes per stage: 128 rows x 64 bf16 */
#define QG3_STAGE (QG3_AB + 256 * 128) /* + W: 256 rows x 64 bf16 */
#define QG3_WAIT_NEWEST() asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)\n\ts_barrier" ::: "memory")
__device__ __forceinline__ void qg_mainloop3(const qw_gemm_args &a, unsigned char *lds,
                                             uint32_t th, uint32_t tn, uint32_t kb, uint32_t ke,
                                             floatx4 (&acc)[8][8]) {
    constexpr int MB = 4, NL = MB + 8; /* 12 loads per slice and thread: QG3_WAIT_NEWEST */
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = th * 128, n0 = tn * 256;
    QgCtx c;
    const uint32_t lrow = lane >> 3, lp = lane & 7;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t r = wave * 64 + j * 8 + lrow;
        const uint32_t ra = wave * (MB * 8) + j * 8 + lrow;
        if (j < MB)
            c.a_dvoff[j] = (min(m0 + ra, a.m - 1) * a.lda + (lp ^ ((ra >> 1) & 7u)) * 8) * 2;
        c.w_dvoff[j] = (min(n0 + r, a.n - 1) * a.k + (lp ^ ((r >> 1) & 7u)) * 8) * 2;
    }
    c.a_rs4 = gemm_rs4(a.a, a.a_bytes);
    c.w_rs4 = gemm_rs4(a.w, a.w_bytes);
    c.dst0 = wave * (MB * 8) * 128;
    c.wdst0 = wave * 64 * 128;
    const uint32_t l16 = lane & 15, h = lane >> 4, swz = (l16 >> 1) & 7u;
    c.a_frag = (wm * (MB * 16) + l16) * 128;
    c.w_frag = (wn * 128 + l16) * 128;
    c.ch[0] = ((0 + h) ^ swz) << 4;
    c.ch[1] = ((4 + h) ^ swz) << 4;
    unsigned char *s0 = lds, *s1 = lds + QG3_STAGE, *s2 = lds + 2 * QG3_STAGE;
    const uint32_t last = ke - 1;
    auto issue = [&](unsigned char *st, uint32_t k) __attribute__((always_inline)) {
        const uint32_t nb =
            (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)st;
#pragma unroll
        for (int j = 0; j < MB; j++)
            gemm_dma16(c.a_rs4, nb + c.dst0 + j * 1024, c.a_dvoff[j], k * GBK * 2);
#pragma unroll
        for (int j = 0; j < 8; j++)
            gemm_dma16(c.w_rs4, nb + QG3_AB + c.wdst0 + j * 1024, c.w_dvoff[j], k * GBK * 2);
    };
    issue(s0, kb);
    issue(s1, min(kb + 1, last));
    QG3_WAIT_NEWEST(); /* slice kb landed */
    bf16x8 pa[8], pw[8];
    qg_slice<false, MB, QG3_AB>(c, acc, pa, pw, s0, s2, min(kb + 2, last) * GBK);
    QG3_WAIT_NEWEST(); /* slice kb + 1 landed */
    uint32_t kt = kb + 1;
    for (; kt + 2 < ke; kt += 3) {
        qg_slice<true, MB, QG3_AB>(c, acc, pa, pw, s1, s0, min(kt + 2, last) * GBK);
        QG3_WAIT_NEWEST();
        qg_slice<true, MB, QG3_AB>(c, acc, pa, pw, s2, s1, min(kt + 3, last) * GBK);
        QG3_WAIT_NEWEST();
        qg_slice<true, MB, QG3_AB>(c, acc, pa, pw, s0, s2, min(kt + 4, last) * GBK);
        QG3_WAIT_NEWEST();
    }
    /* the last 0-2 slices, in the rotation's order */
    if (kt < ke) {
        qg_slice<true, MB, QG3_AB>(c, acc, pa, pw, s1, s0, min(kt + 2, last) * GBK);
        QG3_WAIT_NEWEST();
    }
    if (kt + 1 < ke) {
        qg_slice<true, MB, QG3_AB>(c, acc, pa, pw, s2, s1, min(kt + 3, last) * GBK);
        QG3_WAIT_NEWEST();
    }
    qg_ready(pw);
    qg_ready<MB>(pa);
#pragma unroll
    for (int i = 0; i < 8 * MB; i++) QG_MFMA(acc[i % MB][i / MB], pw[i / MB], pa[i % MB]);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    QW_SLICE_END(); /* the reloads past ke - 1 land before the epilogue uses the LDS */
}

/* int8 W widened once per workgroup (the "_w8" kernels): the bf16 kernel's
 * pipeline and LDS layout, with the W stage filled by the workgroup itself
 * instead of a direct load. Each thread owns 4 row pieces of the 256-row x
 * 64-k int8 W tile (rows wave * 64 + 16 i + lane / 4, 16 bytes at k offset
 * 16 (lane % 4)), loaded into registers (global -> VGPR, 16 KB per slice
 * per workgroup: half the bf16 tile's bytes), widened to bf16 (exact) and
 * written into the W stage with the bf16 tile's swizzle, so the fragment
 * reads and MFMAs are the bf16 kernel's. Every weight element is widened
 * once per workgroup (an earlier form widened each 8-byte fragment in
 * registers in every wave that read it, twice per element: 8-10% slower
 * than this on the step's shapes), and no widened copy goes through HBM.
 *
 * Timing, slice s (stage cur holds A(s), W(s); nxt receives slice s + 1):
 * the held-back sub-step's MFMAs cover the 8 direct A loads of s + 1, the
 * 16 fragment reads of sub-step 0, and then, one VALU step per MFMA from
 * MFMA QW8_S0 on, the widening of W(s + 1) (its raw int8 loaded during
 * slice s - 1) into nxt and the raw loads of W(s + 2) into the freed
 * registers (QW8_S0 must not be below 30: every direct load of the slice
 * is issued before the first piece's wait). The slice ends waiting
 * for the A loads only (vmcnt(4): the 4 raw loads issued after them stay
 * in flight across the barrier, a whole slice ahead of their use). The
 * raw loads are inline assembly, like the direct loads, so their waits are
 * explicit: before piece p is widened, the 11 memory operations issued
 * after its load may still be outstanding (the 3 - p later raw loads of the
 * previous slice, this slice's 8 direct loads, this slice's p earlier
 * reloads). */
#define QW8_SLICE_END() asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory")

__device__ __forceinline__ void qw8_load(u32x4 &r, u32x4 rsrc, uint32_t voff, uint32_t soff) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(r) : "v"(voff), "s"(rsrc),
                 "s"(soff));
}
/* the raw piece has landed once at most N memory operations remain
 * outstanding; the piece is an operand, so its readers are placed after */
template <int N>
__device__ __forceinline__ void qw8_wait(u32x4 &r) {
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(r) : "n"(N));
}

struct Qw8 {
    u32x4 raw[4];
    uint32_t voff[4];      /* raw piece i: byte offset of its row piece at k = 0 */
    uint32_t wdst[4][2];   /* LDS byte offset (in a stage) of its two bf16 chunks */
    float fa, fb;          /* widening temporaries */
    uint32_t o[8];         /* the piece being widened, as packed bf16 pairs */
};

/* whole-piece widening (prologue) */
__device__ __forceinline__ void qw8_widen(Qw8 &w, int i, unsigned char *stage) {
    u32x4 lo, hi;
    i8x16_to_bf16(w.raw[i], lo, hi);
    *(u32x4 *)(stage + w.wdst[i][0]) = lo;
    *(u32x4 *)(stage + w.wdst[i][1]) = hi;
}

/* byte B of x, sign-extended, to fp32 (exact) */
template <int B>
__device__ __forceinline__ float qw8_cvt(uint32_t x) {
    float f;
    if constexpr (B == 0)
        asm volatile("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD "
                     "src0_sel:BYTE_0" : "=v"(f) : "v"(x));
    else if constexpr (B == 1)
        asm volatile("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD "
                     "src0_sel:BYTE_1" : "=v"(f) : "v"(x));
    else if constexpr (B == 2)
        asm volatile("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD "
                     "src0_sel:BYTE_2" : "=v"(f) : "v"(x));
    else
        asm volatile("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD "
                     "src0_sel:BYTE_3" : "=v"(f) : "v"(x));
    return f;
}
__device__ __forceinline__ uint32_t qw8_pack(float lo, float hi) {
    uint32_t o;
    asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(o) : "v"(lo), "v"(hi));
    return o;
}

/* Step t (0..23) of widening raw piece p into stage `nxt`: per dword of the
 * piece, two byte conversions, a pack, two conversions, a pack. The steps
 * are inline assembly so each stays in the MFMA slot it is written in (the
 * compiler would otherwise bunch a piece's 24 VALU instructions between two
 * MFMAs and leave the matrix pipe idle). Step 0 waits for the raw piece;
 * after step 23 the two bf16 chunks are stored and the piece's registers
 * reloaded with the raw W of slice k_raw. */
template <int P, int T>
__device__ __forceinline__ void qw8_step(Qw8 &w, const QgCtx &c, unsigned char *nxt,
                                         uint32_t k_raw) {
    constexpr int D = T / 6, U = T % 6;
    if constexpr (T == 0) qw8_wait<11>(w.raw[P]);
    const uint32_t x = w.raw[P][D];
    if constexpr (U == 0) w.fa = qw8_cvt<0>(x);
    if constexpr (U == 1) w.fb = qw8_cvt<1>(x);
    if constexpr (U == 2) w.o[2 * D] = qw8_pack(w.fa, w.fb);
    if constexpr (U == 3) w.fa = qw8_cvt<2>(x);
    if constexpr (U == 4) w.fb = qw8_cvt<3>(x);
    if constexpr (U == 5) w.o[2 * D + 1] = qw8_pack(w.fa, w.fb);
    if constexpr (T == 23) {
        qw8_load(w.raw[P], c.w_rs4, w.voff[P], k_raw);
        *(u32x4 *)(nxt + w.wdst[P][0]) = u32x4{w.o[0], w.o[1], w.o[2], w.o[3]};
        *(u32x4 *)(nxt + w.wdst[P][1]) = u32x4{w.o[4], w.o[5], w.o[6], w.o[7]};
    }
}
/* global step g (0..95) of a slice's widening: piece g / 24, step g % 24 */
template <int G>
__device__ __forceinline__ void qw8_g(Qw8 &w, const QgCtx &c, unsigned char *nxt,
                                      uint32_t k_raw) {
    if constexpr (G >= 0 && G < 96) qw8_step<G / 24, G % 24>(w, c, nxt, k_raw);
}
/* The 96 steps spread evenly over the MFMA slots [S0, 128) of a slice
 * (slots 0-63: the held-back sub-step, 64-127: sub-step 0); the first slice
 * of a tile has no held-back sub-step and spreads them over 64-127. */
#ifndef QW8_S0
#define QW8_S0 48 /* 48 and 32 within noise of each other, both ahead of 64 */
#endif
static_assert(QW8_S0 >= 30, "the first widening step waits on all 8 direct loads");
constexpr int qw8_start(int slot, int s0) {
    return slot <= s0 ? 0 : slot >= 128 ? 96 : (slot - s0) * 96 / (128 - s0);
}
template <int SLOT, int S0>
__device__ __forceinline__ void qw8_slot(Qw8 &w, const QgCtx &c, unsigned char *nxt,
                                         uint32_t k_raw) {
    constexpr int g0 = qw8_start(SLOT, S0), g1 = qw8_start(SLOT + 1, S0);
    static_assert(g1 - g0 <= 3, "widening steps per MFMA slot");
    if constexpr (g1 > g0) qw8_g<g0>(w, c, nxt, k_raw);
    if constexpr (g1 > g0 + 1) qw8_g<g0 + 1>(w, c, nxt, k_raw);
    if constexpr (g1 > g0 + 2) qw8_g<g0 + 2>(w, c, nxt, k_raw);
}

template <int I, bool PREV>
__device__ __forceinline__ void qw8_loop1_at(const QgCtx &c, Qw8 &w, floatx4 (&acc)[8][8],
                                             bf16x8 (&pa)[8], bf16x8 (&pw)[8], bf16x8 (&af)[8],
                                             bf16x8 (&bw)[8], const unsigned char *cur,
                                             unsigned char *nxt, uint32_t nl, uint32_t k_next,
                                             uint32_t k_raw) {
    QG_MFMA(acc[I & 7][I >> 3], pw[I >> 3], pa[I & 7]);
    if constexpr ((I & 3) == 1 && (I >> 2) < 8)
        gemm_dma16(c.a_rs4, nl + c.dst0 + (I >> 2) * 1024, c.a_dvoff[I >> 2], k_next * 2);
    if constexpr ((I & 3) == 3) qg_read(c, cur, c.ch[0], af, bw, I >> 2);
    qw8_slot<I, QW8_S0>(w, c, nxt, k_raw);
    if constexpr (I + 1 < 64)
        qw8_loop1_at<I + 1, PREV>(c, w, acc, pa, pw, af, bw, cur, nxt, nl, k_next, k_raw);
}

template <int I, bool PREV>
__device__ __forceinline__ void qw8_loop2_at(const QgCtx &c, Qw8 &w, floatx4 (&acc)[8][8],
                                             bf16x8 (&af)[8], bf16x8 (&bw)[8], bf16x8 (&af1)[8],
                                             bf16x8 (&bw1)[8], const unsigned char *cur,
                                             unsigned char *nxt, uint32_t k_raw) {
    if constexpr (PREV)
        QG_MFMA(acc[I & 7][I >> 3], bw[I >> 3], af[I & 7]);
    else
        QG_MFMA0(acc[I & 7][I >> 3], bw[I >> 3], af[I & 7]);
    if constexpr ((I & 3) == 3) qg_read(c, cur, c.ch[1], af1, bw1, I >> 2);
    qw8_slot<64 + I, PREV ? QW8_S0 : 64>(w, c, nxt, k_raw);
    if constexpr (I + 1 < 64)
        qw8_loop2_at<I + 1, PREV>(c, w, acc, af, bw, af1, bw1, cur, nxt, k_raw);
}

template <bool PREV>
__device__ __forceinline__ void qw8_slice(const QgCtx &c, Qw8 &w, floatx4 (&acc)[8][8],
                                          bf16x8 (&pa)[8], bf16x8 (&pw)[8],
                                          const unsigned char *__restrict__ cur,
                                          unsigned char *__restrict__ nxt, uint32_t k_next,
                                          uint32_t k_raw) {
    const uint32_t nl = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)nxt;
    bf16x8 af[8], bw[8], af1[8], bw1[8];
    if constexpr (PREV) {
        qg_ready(pw);
        qg_ready(pa);
        qw8_loop1_at<0, true>(c, w, acc, pa, pw, af, bw, cur, nxt, nl, k_next, k_raw);
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++)
            gemm_dma16(c.a_rs4, nl + c.dst0 + j * 1024, c.a_dvoff[j], k_next * 2);
#pragma unroll
        for (int j = 0; j < 16; j++) qg_read(c, cur, c.ch[0], af, bw, j);
    }
    qw8_loop2_at<0, PREV>(c, w, acc, af, bw, af1, bw1, cur, nxt, k_raw);
#pragma unroll
    for (int i = 0; i < 8; i++) pa[i] = af1[i];
#pragma unroll
    for (int i = 0; i < 8; i++) pw[i] = bw1[i];
}

/* Sums of tile (tm, tn) over k-steps [kb, ke), int8 W widened per
 * workgroup; ends with the LDS stages free and no load in flight. */
__device__ __forceinline__ void qw8_mainloop(const qw_gemm_args &a, unsigned char *lds,
                                             unsigned char *lds_b, uint32_t tm, uint32_t tn,
                                             uint32_t kb, uint32_t ke, floatx4 (&acc)[8][8]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = tm * 256, n0 = tn * 256;
    QgCtx c;
    Qw8 w;
    const uint32_t lrow = lane >> 3, lp = lane & 7;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t r = wave * 64 + j * 8 + lrow;
        c.a_dvoff[j] = (min(m0 + r, a.m - 1) * a.lda + (lp ^ ((r >> 1) & 7u)) * 8) * 2;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t r = wave * 64 + i * 16 + (lane >> 2), q = lane & 3;
        w.voff[i] = min(n0 + r, a.n - 1) * a.k + q * 16;
#pragma unroll
        for (int h = 0; h < 2; h++)
            w.wdst[i][h] = QG_A_BYTES + r * 128 + (((2 * q + h) ^ ((r >> 1) & 7u)) << 4);
    }
    c.a_rs4 = gemm_rs4(a.a, a.a_bytes);
    c.w_rs4 = gemm_rs4(a.w, a.w_bytes);
    c.dst0 = wave * 64 * 128;
    const uint32_t l16 = lane & 15, h = lane >> 4, swz = (l16 >> 1) & 7u;
    c.a_frag = (wm * 128 + l16) * 128;
    c.w_frag = (wn * 128 + l16) * 128;
    c.ch[0] = ((0 + h) ^ swz) << 4;
    c.ch[1] = ((4 + h) ^ swz) << 4;
    const uint32_t KT = ke;
    auto kraw = [&](uint32_t s) __attribute__((always_inline)) {
        return (s < KT ? s : KT - 1) * GBK;
    };
    {
        /* prologue: W(kb) raw, A(kb) direct, W(kb) widened into stage 0,
         * then W(kb + 1) raw in flight */
        const uint32_t nb =
            (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)lds;
#pragma unroll
        for (int i = 0; i < 4; i++) qw8_load(w.raw[i], c.w_rs4, w.voff[i], kb * GBK);
#pragma unroll
        for (int j = 0; j < 8; j++)
            gemm_dma16(c.a_rs4, nb + c.dst0 + j * 1024, c.a_dvoff[j], kb * GBK * 2);
        asm volatile("s_waitcnt vmcnt(8)" : "+v"(w.raw[0]), "+v"(w.raw[1]), "+v"(w.raw[2]),
                     "+v"(w.raw[3]));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            qw8_widen(w, i, lds);
            qw8_load(w.raw[i], c.w_rs4, w.voff[i], kraw(kb + 1));
        }
    }
    QW8_SLICE_END();
    bf16x8 pa[8], pw[8];
    qw8_slice<false>(c, w, acc, pa, pw, lds, lds_b, (kb + 1 < KT ? kb + 1 : kb) * GBK,
                     kraw(kb + 2));
    QW8_SLICE_END();
    uint32_t kt = kb + 1;
    for (; kt + 1 < KT; kt += 2) {
        qw8_slice<true>(c, w, acc, pa, pw, lds_b, lds, (kt + 1) * GBK, kraw(kt + 2));
        QW8_SLICE_END();
        qw8_slice<true>(c, w, acc, pa, pw, lds, lds_b, (kt + 2 < KT ? kt + 2 : kt + 1) * GBK,
                        kraw(kt + 3));
        QW8_SLICE_END();
    }
    if (kt < KT) {
        qw8_slice<true>(c, w, acc, pa, pw, lds_b, lds, kt * GBK, kraw(kt + 2));
        QW8_SLICE_END();
    }
    /* the last raw loads (of slices never used) land before their
     * registers can be given to anything else */
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(w.raw[0]), "+v"(w.raw[1]), "+v"(w.raw[2]),
                 "+v"(w.raw[3]));
    qg_ready(pw);
    qg_ready(pa);
#pragma unroll
    for (int i = 0; i < 64; i++) QG_MFMA(acc[i & 7][i >> 3], pw[i >> 3], pa[i & 7]);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}

/* Half tiles (128 x 256, bf16 W): a tile walk whose last wave of tiles
 * would leave at least half the CUs idle runs those tiles as twice as many
 * half tiles instead. Same 2 x 2 waves, each 64 x 128 (4 x 8 MFMA tiles);
 * the A stage holds 128 rows (4 direct loads per wave), the W stage is the
 * full tile's. Per 32-k sub-step: 32 MFMAs, 12 fragments (W block 0, A
 * blocks 0-3, W blocks 1-7), and under the held-back sub-step the 12 direct
 * loads of the next slice, one load and one read every 2 MFMAs. */
template <bool PREV>
__device__ __forceinline__ void qh_slice(const QgCtx &c, floatx4 (&acc)[8][8], bf16x8 (&pa)[8],
                                         bf16x8 (&pw)[8], const unsigned char *__restrict__ cur,
                                         unsigned char *__restrict__ nxt, uint32_t k_next) {
    const uint32_t nl = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)nxt;
    auto dma = [&](int j) __attribute__((always_inline)) {
        if (j < 4)
            gemm_dma16(c.a_rs4, nl + c.dst0 + j * 1024, c.a_dvoff[j], k_next * 2);
        else
            gemm_dma16(c.w_rs4, nl + QG_A_BYTES + c.wdst0 + (j - 4) * 1024, c.w_dvoff[j - 4],
                       k_next * 2);
    };
    auto rd = [&](int ks, int j, bf16x8(&A)[8], bf16x8(&W)[8]) __attribute__((always_inline)) {
        if (j == 0)
            W[0] = *(const bf16x8 *)(cur + QG_A_BYTES + c.w_frag + c.ch[ks]);
        else if (j <= 4)
            A[j - 1] = *(const bf16x8 *)(cur + c.a_frag + (j - 1) * 2048 + c.ch[ks]);
        else
            W[j - 4] = *(const bf16x8 *)(cur + QG_A_BYTES + c.w_frag + (j - 4) * 2048 + c.ch[ks]);
    };
    bf16x8 af[8], bw[8], af1[8], bw1[8];
    if (PREV) {
        qg_ready(pw);
        qg_ready(pa);
#pragma unroll
        for (int i = 0; i < 32; i++) {
            QG_MFMA(acc[i & 3][i >> 2], pw[i >> 2], pa[i & 3]);
            if ((i & 1) == 0 && (i >> 1) < 12) dma(i >> 1);
            if ((i & 1) == 1 && (i >> 1) < 12) rd(0, i >> 1, af, bw);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 12; j++) dma(j);
#pragma unroll
        for (int j = 0; j < 12; j++) rd(0, j, af, bw);
    }
#pragma unroll
    for (int i = 0; i < 32; i++) {
        if (PREV)
            QG_MFMA(acc[i & 3][i >> 2], bw[i >> 2], af[i & 3]);
        else
            QG_MFMA0(acc[i & 3][i >> 2], bw[i >> 2], af[i & 3]);
        if ((i & 1) == 1 && (i >> 1) < 12) rd(1, i >> 1, af1, bw1);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) pa[i] = af1[i];
#pragma unroll
    for (int i = 0; i < 8; i++) pw[i] = bw1[i];
}

/* Sums of the half tile at rows [m0, m0 + 128), columns [n0, n0 + 256) over
 * all of K into acc[0..3][*]; ends with the LDS stages free. */
__device__ __forceinline__ void qh_mainloop(const qw_gemm_args &a, unsigned char *lds,
                                            unsigned char *lds_b, uint32_t m0, uint32_t n0,
                                            floatx4 (&acc)[8][8]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1;
    QgCtx c;
    const uint32_t lrow = lane >> 3, lp = lane & 7;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t r = wave * 32 + j * 8 + lrow;
        c.a_dvoff[j] = (min(m0 + r, a.m - 1) * a.lda + (lp ^ ((r >> 1) & 7u)) * 8) * 2;
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t r = wave * 64 + j * 8 + lrow;
        c.w_dvoff[j] = (min(n0 + r, a.n - 1) * a.k + (lp ^ ((r >> 1) & 7u)) * 8) * 2;
    }
    c.a_rs4 = gemm_rs4(a.a, a.a_bytes);
    c.w_rs4 = gemm_rs4(a.w, a.w_bytes);
    c.dst0 = wave * 32 * 128;
    c.wdst0 = wave * 64 * 128;
    const uint32_t l16 = lane & 15, h = lane >> 4, swz = (l16 >> 1) & 7u;
    c.a_frag = (wm * 64 + l16) * 128;
    c.w_frag = (wn * 128 + l16) * 128;
    c.ch[0] = ((0 + h) ^ swz) << 4;
    c.ch[1] = ((4 + h) ^ swz) << 4;
    const uint32_t KT = a.k / GBK;
    {
        const uint32_t nb =
            (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)lds;
#pragma unroll
        for (int j = 0; j < 4; j++) gemm_dma16(c.a_rs4, nb + c.dst0 + j * 1024, c.a_dvoff[j], 0);
#pragma unroll
        for (int j = 0; j < 8; j++)
            gemm_dma16(c.w_rs4, nb + QG_A_BYTES + c.wdst0 + j * 1024, c.w_dvoff[j], 0);
    }
    QW_SLICE_END();
    bf16x8 pa[8], pw[8];
    qh_slice<false>(c, acc, pa, pw, lds, lds_b, (1 < KT ? 1 : 0) * GBK);
    QW_SLICE_END();
    uint32_t kt = 1;
    for (; kt + 1 < KT; kt += 2) {
        qh_slice<true>(c, acc, pa, pw, lds_b, lds, (kt + 1) * GBK);
        QW_SLICE_END();
        qh_slice<true>(c, acc, pa, pw, lds, lds_b, (kt + 2 < KT ? kt + 2 : kt + 1) * GBK);
        QW_SLICE_END();
    }
    if (kt < KT) {
        qh_slice<true>(c, acc, pa, pw, lds_b, lds, kt * GBK);
        QW_SLICE_END();
    }
    qg_ready(pw);
    qg_ready(pa);
#pragma unroll
    for (int i = 0; i < 32; i++) QG_MFMA(acc[i & 3][i >> 2], pw[i >> 2], pa[i & 3]);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}

/* INT8: 0 bf16 W, 1 int8 W widened once per workgroup */
template <int INT8>
__device__ __forceinline__ void qg_mainloop_any(const qw_gemm_args &a, unsigned char *lds,
                                                unsigned char *lds_b, uint32_t tm, uint32_t tn,
                                                uint32_t kb, uint32_t ke, floatx4 (&acc)[8][8]) {
    if constexpr (INT8)
        qw8_mainloop(a, lds, lds_b, tm, tn, kb, ke, acc);
    else
        qg_mainloop(a, lds, lds_b, tm, tn, kb, ke, acc);
}

/* The epilogue of the tile (MB = 8), 224-row tile (MB = 7) or half tile
 * (MB = 4) whose rows start at m0 and columns at n0: each wave's MB x 8
 * accumulator blocks. */
template <int EPI, int INT8, int MB>
__device__ __forceinline__ void qg_finish_at(const qw_gemm_args &a, unsigned char *lds,
                                             unsigned char *lds_b, uint32_t m0, uint32_t n0,
                                             floatx4 (&acc)[8][8], float *pst = nullptr,
                                             const float *pld = nullptr, uint32_t npart = 0,
                                             uint32_t own = 0) {
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t row0 = m0 + wm * (MB * 16), col0 = n0 + wn * 128;
    constexpr uint32_t LDF = 128 + 4, REG = 32 * LDF * 4;
    /* waves 0, 1 stage through `lds`, 2, 3 through `lds_b` (free after the
     * loop's last barrier), one 32-row slab (16.5 KB) at a time */
    float *region = (float *)((wave < 2 ? lds : lds_b) + (wave & 1) * REG);
    const uint32_t poff = wm * 128 * 256 + wn * 128;
    /* slab mi: rows SB 16 mi + 16 q + lane % 16 (tile mb = SB mi + q), columns
     * 32 ni + 16 p + 4 (lane / 16) + 0..3 (tile nb = 2 ni + p); SB = 2 blocks
     * of 16 rows per slab, 1 for an odd block count (224-row tiles). Columns
     * 64-127 are stored with the two 16-byte halves of each 32-byte group
     * exchanged (column c at c ^ 4). */
    constexpr int SB = (MB & 1) ? 1 : 2;
    const uint32_t wc_lo = 4 * (lane >> 4), wc_hi = wc_lo ^ 4; /* column within 16, plain / exchanged */
    auto write_slab = [&](int mi) __attribute__((always_inline)) {
#pragma unroll
        for (int ni = 0; ni < 4; ni++)
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int q = 0; q < SB; q++)
                    *(floatx4 *)(region + (16 * q + (lane & 15)) * LDF + ni * 32 + 16 * p +
                                 (ni >= 2 ? wc_hi : wc_lo)) = acc[SB * mi + q][2 * ni + p];
    };
    /* the lane's 32 read-back bytes (columns 8 cc..8 cc + 7) as two
     * ds_read_b128: lanes 8-15 of a row (columns 64-127, stored exchanged)
     * read the upper physical half first, so one pass of 16 lanes covers all
     * 64 banks and both reads return the columns in order */
    const uint32_t cc = lane & 15, swap = (cc >> 3) & 1;
    auto read_row = [&](uint32_t lr, float (&v)[8]) __attribute__((always_inline)) {
        const floatx4 v0 = *(const floatx4 *)(region + lr * LDF + cc * 8 + 4 * swap);
        const floatx4 v1 = *(const floatx4 *)(region + lr * LDF + cc * 8 + 4 * (swap ^ 1));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[j] = v0[j];
            v[4 + j] = v1[j];
        }
    };
    gemm_epilogue_lds<EPI, INT8, MB / SB, 16 * SB, 4 * SB>(a, write_slab, read_row, row0, col0, lane,
                                            pst ? pst + poff : nullptr,
                                            pld ? pld + poff : nullptr, npart, own);
}

template <int EPI, int INT8>
__device__ __forceinline__ void qg_finish(const qw_gemm_args &a, unsigned char *lds,
                                          unsigned char *lds_b, uint32_t tm, uint32_t tn,
                                          floatx4 (&acc)[8][8], float *pst = nullptr,
                                          const float *pld = nullptr, uint32_t npart = 0,
                                          uint32_t own = 0) {
    qg_finish_at<EPI, INT8, 8>(a, lds, lds_b, tm * 256, tn * 256, acc, pst, pld, npart, own);
}

template <int EPI, int INT8>
__device__ __forceinline__ void qg_impl(const qw_gemm_args &a, unsigned char *lds,
                                        unsigned char *lds_b) {
    const uint32_t KT = a.k / GBK;
    const uint32_t nt = a.tiles_m * a.tiles_n;
    const bool split = a.split > 1;
    const uint32_t ndp = split ? a.dp_tiles : nt;
    floatx4 acc[8][8];
    uint32_t pid = blockIdx.x, tm, tn;
    /* no split tiles: the walk (its grid may exceed the tile count when the
     * tiles run as half tiles); split: workgroups below ndp take a whole
     * tile, the rest one piece */
    if (!split || pid < ndp) {
        if (!split) {
            /* one workgroup per CU walks the tiles in strides of the grid;
             * id and id + grid sit on the same XCD (grid % 8 == 0). Tiles
             * [half_from, nt) run as half tiles, ids half_from + [0, 2 R):
             * the two halves of a tile go to one XCD. */
            const uint32_t H = INT8 ? 0u : a.half_count;
            const uint32_t F = H ? a.half_from : ndp;
            for (uint32_t id = pid; id < F + H; id += gridDim.x) {
                if (id < F) {
                    uint32_t q = id;
                    if ((F & 7u) == 0) q = (q & 7u) * (F >> 3) + (q >> 3);
                    gemm_tile_at(a, q, tm, tn);
                    qg_mainloop_any<INT8>(a, lds, lds_b, tm, tn, 0, KT, acc);
                    qg_finish<EPI, INT8>(a, lds, lds_b, tm, tn, acc);
                } else if (!INT8) {
                    uint32_t hq = id - F;
                    if ((H & 15u) == 0) hq = (hq & 7u) * (H >> 3) + (hq >> 3);
                    gemm_tile_at(a, F + (hq >> 1), tm, tn);
                    const uint32_t m0 = tm * 256 + (hq & 1) * 128;
                    if (a.half3)
                        qg_mainloop3(a, lds, m0 / 128, tn, 0, KT, acc);
                    else
                        qh_mainloop(a, lds, lds_b, m0, tn * 256, acc);
                    qg_finish_at<EPI, INT8, 4>(a, lds, lds_b, m0, tn * 256, acc);
                }
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            }
            return;
        }
        if ((ndp & 7u) == 0) pid = (pid & 7u) * (ndp >> 3) + (pid >> 3);
        gemm_tile_at(a, pid, tm, tn);
        qg_mainloop_any<INT8>(a, lds, lds_b, tm, tn, 0, KT, acc);
        qg_finish<EPI, INT8>(a, lds, lds_b, tm, tn, acc);
        return;
    }
    /* piece of a split tile (k-range-major numbering, as gemm.h); with
     * half_count set (bf16 W, a launch of at most half as many tiles as
     * CUs) the split tiles run as half tiles, r = 2 tile + half */
    uint32_t &ticket = *(uint32_t *)(lds_b + QG_STAGE); /* reserved by QG_ENTRY */
    const bool hs = !INT8 && a.half_count;
    const uint32_t R = (nt - ndp) << (hs ? 1 : 0), S = a.split, np = R * S;
    uint32_t q = pid - ndp;
    if ((np & 7u) == 0) q = (q & 7u) * (np >> 3) + (q >> 3);
    const uint32_t piece = q / R, r = q % R;
    const uint32_t kb = piece * KT / S, ke = (piece + 1) * KT / S;
    gemm_tile_at(a, ndp + (hs ? r >> 1 : r), tm, tn);
    const uint32_t th = tm * 2 + (r & 1); /* half tile row (128 rows) */
    float *slots = a.sk_part + (size_t)r * S * QW_SPLIT_PART;
    if constexpr (!INT8) {
        if (hs) {
            qg_mainloop<4>(a, lds, lds_b, th, tn, kb, ke, acc);
            qg_finish_at<EPI, INT8, 4>(a, lds, lds_b, th * 128, tn * 256, acc,
                                       slots + (size_t)piece * QW_SPLIT_PART);
        }
    }
    if (!hs) {
        qg_mainloop_any<INT8>(a, lds, lds_b, tm, tn, kb, ke, acc);
        qg_finish<EPI, INT8>(a, lds, lds_b, tm, tn, acc, slots + (size_t)piece * QW_SPLIT_PART);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0): the partial's stores are done */
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (threadIdx.x == 0)
        ticket = __hip_atomic_fetch_add(a.sk_flag + r, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (ticket != S - 1) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if constexpr (!INT8) {
        if (hs)
            qg_finish_at<EPI, INT8, 4>(a, lds, lds_b, th * 128, tn * 256, acc, nullptr, slots, S,
                                       piece);
    }
    if (!hs) qg_finish<EPI, INT8>(a, lds, lds_b, tm, tn, acc, nullptr, slots, S, piece);
    if (threadIdx.x == 0)
        __hip_atomic_store(a.sk_flag + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* 224-row tiles (bf16 W, no split tiles): one workgroup per CU walks the
 * tiles, as the 256-row kernels do. Chosen where the tile count leaves a
 * partly filled last wave that 224-row tiles avoid (the out projection at
 * M = 8704: 468 tiles of 224 x 256 in 2 waves of 0.875 of a 256-row tile's
 * work, against 408 tiles in 2 waves). */
template <int EPI>
__device__ __forceinline__ void qg_impl_t224(const qw_gemm_args &a, unsigned char *lds,
                                             unsigned char *lds_b) {
    const uint32_t KT = a.k / GBK;
    const uint32_t nt = a.tiles_m * a.tiles_n;
    floatx4 acc[8][8];
    uint32_t tm, tn;
    for (uint32_t id = blockIdx.x; id < nt; id += gridDim.x) {
        uint32_t q = id;
        if ((nt & 7u) == 0) q = (q & 7u) * (nt >> 3) + (q >> 3);
        gemm_tile_at(a, q, tm, tn);
        qg_mainloop<7>(a, lds, lds_b, tm, tn, 0, KT, acc);
        qg_finish_at<EPI, 0, 7>(a, lds, lds_b, tm * 224, tn * 256, acc);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
}

/* Small launches (at most cus / 2 tiles, bf16 W) as half tiles on the
 * three-stage loop, one half tile -- or one k-range piece of one, when
 * a.split > 1 -- per workgroup: grid = 2 tiles x split. Pieces meet as in
 * qg_impl (k-range-major numbering, the last one in adds them in piece
 * order and runs the epilogue). */
template <int EPI>
__device__ __forceinline__ void qg_impl_h3(const qw_gemm_args &a, unsigned char *lds) {
    const uint32_t KT = a.k / GBK;
    const uint32_t R = 2 * a.tiles_m * a.tiles_n, S = a.split > 1 ? a.split : 1, np = R * S;
    uint32_t q = blockIdx.x;
    if (q >= np) return;
    if ((np & 7u) == 0) q = (q & 7u) * (np >> 3) + (q >> 3);
    const uint32_t piece = q / R, r = q % R;
    const uint32_t kb = piece * KT / S, ke = (piece + 1) * KT / S;
    uint32_t tm, tn;
    gemm_tile_at(a, r >> 1, tm, tn);
    const uint32_t th = tm * 2 + (r & 1);
    floatx4 acc[8][8];
    qg_mainloop3(a, lds, th, tn, kb, ke, acc);
    unsigned char *lds_b = lds + QG_STAGE;
    if (S == 1) {
        qg_finish_at<EPI, 0, 4>(a, lds, lds_b, th * 128, tn * 256, acc);
        return;
    }
    uint32_t &ticket = *(uint32_t *)(lds + 3 * QG3_STAGE); /* reserved by QG_ENTRY_H3 */
    float *slots = a.sk_part + (size_t)r * S * QW_SPLIT_PART;
    qg_finish_at<EPI, 0, 4>(a, lds, lds_b, th * 128, tn * 256, acc,
                            slots + (size_t)piece * QW_SPLIT_PART);
    __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0): the partial's stores are done */
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (threadIdx.x == 0)
        ticket = __hip_atomic_fetch_add(a.sk_flag + r, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (ticket != S - 1) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    qg_finish_at<EPI, 0, 4>(a, lds, lds_b, th * 128, tn * 256, acc, nullptr, slots, S, piece);
    if (threadIdx.x == 0)
        __hip_atomic_store(a.sk_flag + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* One LDS array fixes the layout: the first stage at offset 0, the second
 * at 64 KB, the split-tile counter after them; the bf16 kernels' array also
 * holds the three 48 KB stages of the walk's half tiles (the counter, used
 * only by split tiles, falls inside the third). */
#define QG_ENTRY(name, EPI, INT8)                                                              \
    QW_KERNEL void __launch_bounds__(256, 1) name(qw_gemm_args a) {                            \
        __shared__ __attribute__((aligned(16)))                                                \
        unsigned char smem[(INT8 ? 2 * QG_STAGE : 3 * QG3_STAGE) + 16];                        \
        qg_impl<EPI, INT8>(a, smem, smem + QG_STAGE);                                          \
    }

QG_ENTRY(qw_gemm_bf16_store_q, QW_EPI_STORE, 0)
QG_ENTRY(qw_gemm_bf16_gelu_q, QW_EPI_GELU, 0)
QG_ENTRY(qw_gemm_bf16_gate_q, QW_EPI_GATE, 0)
QG_ENTRY(qw_gemm_bf16_qkn_q, QW_EPI_QKNORM, 0)
/* int8 weights (per-row scale in the epilogue), widened once per workgroup
 * into the bf16 W stage */
QG_ENTRY(qw_gemm_w8_store_q, QW_EPI_STORE, 1)
QG_ENTRY(qw_gemm_w8_gelu_q, QW_EPI_GELU, 1)
QG_ENTRY(qw_gemm_w8_gate_q, QW_EPI_GATE, 1)
QG_ENTRY(qw_gemm_w8_qkn_q, QW_EPI_QKNORM, 1)
/* bf16 W, 224-row tiles */
#define QG_ENTRY_T224(name, EPI)                                                               \
    QW_KERNEL void __launch_bounds__(256, 1) name(qw_gemm_args a) {                            \
        __shared__ __attribute__((aligned(16))) unsigned char smem[2 * QG_STAGE + 16];          \
        qg_impl_t224<EPI>(a, smem, smem + QG_STAGE);                                           \
    }
QG_ENTRY_T224(qw_gemm_bf16_store_t224, QW_EPI_STORE)
QG_ENTRY_T224(qw_gemm_bf16_gelu_t224, QW_EPI_GELU)
QG_ENTRY_T224(qw_gemm_bf16_gate_t224, QW_EPI_GATE)
QG_ENTRY_T224(qw_gemm_bf16_qkn_t224, QW_EPI_QKNORM)
/* bf16 W, small launches: half tiles on three stages */
#define QG_ENTRY_H3(name, EPI)                                                                 \
    QW_KERNEL void __launch_bounds__(256, 1) name(qw_gemm_args a) {                            \
        __shared__ __attribute__((aligned(16))) unsigned char smem[3 * QG3_STAGE + 16];         \
        qg_impl_h3<EPI>(a, smem);                                                              \
    }
QG_ENTRY_H3(qw_gemm_bf16_store_h3, QW_EPI_STORE)
QG_ENTRY_H3(qw_gemm_bf16_gelu_h3, QW_EPI_GELU)
QG_ENTRY_H3(qw_gemm_bf16_gate_h3, QW_EPI_GATE)
QG_ENTRY_H3(qw_gemm_bf16_qkn_h3, QW_EPI_QKNORM)

/* Register-staged GEMM, two workgroups per CU:
 *   out[m, n] = epilogue( sum_k A[m, k] * W[n, k] )
 * with the operands, accumulation and epilogue of the 256 x 256 kernels
 * (gemm.h). What differs is how latency is hidden:
 *
 *  - a workgroup is 4 waves (2 x 2) computing a 128 x 256 tile, each wave a
 *    64 x 128 block (2 x 4 MFMA tiles, 128 accumulators), small enough in
 *    registers (<= 256 per lane) and LDS (48 KB) that two workgroups share
 *    a CU. They run out of step, so one workgroup's epilogue, barrier waits
 *    and exposed LDS latency are covered by the other's MFMAs;
 *  - K advances in slices of 32. Slice s + 2 is loaded into registers
 *    while slice s is multiplied from LDS, and slice s + 1 (loaded one step
 *    earlier) is written, int8 W widened to bf16, into the other LDS stage
 *    between the MFMAs: two register sets, two LDS stages, one barrier per
 *    slice. Every load is an ordinary register load, so the compiler's own
 *    vmcnt tracking places the waits (LDS-DMA loads would make it wait for
 *    every load in flight before each LDS read).
 *
 * LDS rows are 64 B (32 bf16 of K); 16-byte chunk c of row r is stored at
 * chunk c ^ ((r / 4) % 4), so that the 16 lanes of one ds_read_b128 pass
 * (16 consecutive rows, one logical chunk) hit 16 distinct (row % 4,
 * chunk) bank groups of the 256-byte bank window. */
#pragma once
#include "gemm.h"

#define RBK 32

__device__ __forceinline__ uint32_t r_swz(uint32_t row, uint32_t chunk) {
    return row * 64u + ((chunk ^ ((row >> 2) & 3u)) << 4);
}

template <int INT8>
struct RingShape {
    static constexpr int WM = 2, WN = 2, MI = 2, NI = 4;
    static constexpr int NT = 256;
    static constexpr int BM = WM * MI * 32; /* 128 */
    static constexpr int BN = WN * NI * 32; /* 256 */
    static constexpr int A_BYTES = BM * 64;
    static constexpr int STAGE = A_BYTES + BN * 64; /* 24 KB */
    static constexpr int A_RL = BM * 4 / NT;        /* 16-byte A loads per thread: 2 */
    /* W loads per thread: int8 rows are 32 B (2 per row), bf16 rows 64 B */
    static constexpr int W_RL = INT8 ? BN * 2 / NT : BN * 4 / NT; /* 2 | 4 */
};

template <int INT8>
struct RingRegs {
    u32x4 a[RingShape<INT8>::A_RL];
    u32x4 w[RingShape<INT8>::W_RL];
};

template <int INT8>
struct RingCtx {
    __amdgpu_buffer_rsrc_t a_rsrc, w_rsrc;
    uint32_t a_off[RingShape<INT8>::A_RL]; /* byte offsets of this thread's loads */
    uint32_t w_off[RingShape<INT8>::W_RL];
    uint32_t a_put[RingShape<INT8>::A_RL]; /* LDS offsets inside a stage */
    uint32_t w_put[RingShape<INT8>::W_RL]; /* bf16: the chunk; int8: first of two */
    uint32_t w_put2[RingShape<INT8>::W_RL];
    uint32_t a_frag, w_frag; /* fragment row offsets (row * 64) */
    uint32_t fsw, h;         /* fragment swizzle term, k-half */
};

template <int INT8>
__device__ __forceinline__ void ring_load(const RingCtx<INT8> &c, RingRegs<INT8> &r, uint32_t k0) {
    typedef RingShape<INT8> S;
#pragma unroll
    for (int j = 0; j < S::A_RL; j++)
        r.a[j] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(c.a_rsrc, c.a_off[j] + k0 * 2, 0, 0));
#pragma unroll
    for (int j = 0; j < S::W_RL; j++)
        r.w[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               c.w_rsrc, c.w_off[j] + k0 * (INT8 ? 1 : 2), 0, 0));
}

template <int INT8>
__device__ __forceinline__ void ring_put(const RingCtx<INT8> &c, const RingRegs<INT8> &r,
                                         unsigned char *stage) {
    typedef RingShape<INT8> S;
#pragma unroll
    for (int j = 0; j < S::A_RL; j++) *(u32x4 *)(stage + c.a_put[j]) = r.a[j];
    unsigned char *Ws = stage + S::A_BYTES;
#pragma unroll
    for (int j = 0; j < S::W_RL; j++) {
        if (INT8) {
            u32x4 lo, hi;
            i8x16_to_bf16(r.w[j], lo, hi);
            *(u32x4 *)(Ws + c.w_put[j]) = lo;
            *(u32x4 *)(Ws + c.w_put2[j]) = hi;
        } else {
            *(u32x4 *)(Ws + c.w_put[j]) = r.w[j];
        }
    }
}

/* Workgroup barrier once this thread's LDS writes have completed. */
__device__ __forceinline__ void ring_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

/* One step: multiply stage `cur`; load slice k_load into `ld`; write `put`
 * (the slice after `cur`) into stage `nxt`; barrier. */
template <int INT8>
__device__ __forceinline__ void ring_step(const RingCtx<INT8> &c,
                                          floatx16 (&acc)[RingShape<INT8>::NI][RingShape<INT8>::MI],
                                          const unsigned char *cur, unsigned char *nxt,
                                          RingRegs<INT8> &ld, const RingRegs<INT8> &put,
                                          uint32_t k_load) {
    typedef RingShape<INT8> S;
    constexpr int MI = S::MI, NI = S::NI;
    constexpr int NMF = MI * NI, NRD = MI + NI;
    constexpr int NV = S::A_RL + S::W_RL;
    constexpr int NW = S::A_RL + (INT8 ? 2 : 1) * S::W_RL;
    const unsigned char *As = cur + c.a_frag, *Ws = cur + S::A_BYTES + c.w_frag;
#define QR_FR(base, i, ks) (*(const bf16x8 *)((base) + (i) * 2048 + ((((2 * (ks) + c.h) ^ c.fsw)) << 4)))
    bf16x8 af[2][MI], bw[2][NI];
#pragma unroll
    for (int i = 0; i < MI; i++) af[0][i] = QR_FR(As, i, 0);
#pragma unroll
    for (int i = 0; i < NI; i++) bw[0][i] = QR_FR(Ws, i, 0);
    ring_load<INT8>(c, ld, k_load);
#pragma unroll
    for (int i = 0; i < MI; i++) af[1][i] = QR_FR(As, i, 1);
#pragma unroll
    for (int i = 0; i < NI; i++) bw[1][i] = QR_FR(Ws, i, 1);
#undef QR_FR
#pragma unroll
    for (int ni = 0; ni < NI; ni++)
#pragma unroll
        for (int mi = 0; mi < MI; mi++)
            acc[ni][mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw[0][ni], af[0][mi], acc[ni][mi], 0, 0, 0);
    /* first half: fragments of sub-step 0, then the slice loads and the
     * fragments of sub-step 1 between the first MFMAs */
    __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);
#pragma unroll
    for (int i = 0; i < NMF; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i < NV) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        if (i < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    /* the next slice's registers are used only from here on, half a step
     * later than the scheduler would otherwise put them */
    __builtin_amdgcn_sched_barrier(0);
    ring_put<INT8>(c, put, nxt);
#pragma unroll
    for (int ni = 0; ni < NI; ni++)
#pragma unroll
        for (int mi = 0; mi < MI; mi++)
            acc[ni][mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw[1][ni], af[1][mi], acc[ni][mi], 0, 0, 0);
    /* second half: the LDS writes of the next slice between the MFMAs */
#pragma unroll
    for (int i = 0; i < NMF; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i < NW) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
    }
    ring_barrier();
}

template <int EPI, int INT8>
__device__ __forceinline__ void qw_gemm_ring_impl(const qw_gemm_args &a, unsigned char *lds) {
    typedef RingShape<INT8> S;
    constexpr int MI = S::MI, NI = S::NI;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave / S::WN, wn = wave % S::WN;
    const uint32_t h = lane >> 5, i32 = lane & 31;
    uint32_t tm, tn;
    gemm_tile(a, tm, tn);
    const uint32_t m0 = tm * S::BM, n0 = tn * S::BN;

    RingCtx<INT8> c;
    c.a_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)a.a, (short)0, (int)a.a_bytes, 0x00020000);
    c.w_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)a.w, (short)0, (int)a.w_bytes, 0x00020000);
    /* A: 4 threads per 64-byte row; rows clamped at the bottom edge */
#pragma unroll
    for (int j = 0; j < S::A_RL; j++) {
        const uint32_t q = tid + S::NT * j, r = q >> 2, ch = q & 3;
        c.a_off[j] = (min(m0 + r, a.m - 1) * a.lda + ch * 8) * 2;
        c.a_put[j] = r_swz(r, ch);
    }
#pragma unroll
    for (int j = 0; j < S::W_RL; j++) {
        if (INT8) {
            /* int8 W: 2 threads per 32-byte row, each widening 16 k into
             * two bf16 chunks */
            const uint32_t q = tid + S::NT * j, r = q >> 1, c16 = q & 1;
            c.w_off[j] = min(n0 + r, a.n - 1) * a.k + c16 * 16;
            c.w_put[j] = r_swz(r, 2 * c16);
            c.w_put2[j] = r_swz(r, 2 * c16 + 1);
        } else {
            const uint32_t q = tid + S::NT * j, r = q >> 2, ch = q & 3;
            c.w_off[j] = (min(n0 + r, a.n - 1) * a.k + ch * 8) * 2;
            c.w_put[j] = c.w_put2[j] = r_swz(r, ch);
        }
    }
    c.a_frag = (wm * MI * 32 + i32) * 64;
    c.w_frag = (wn * NI * 32 + i32) * 64;
    c.fsw = (i32 >> 2) & 3u;
    c.h = h;

    floatx16 acc[NI][MI];
#pragma unroll
    for (int ni = 0; ni < NI; ni++)
#pragma unroll
        for (int mi = 0; mi < MI; mi++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[ni][mi][v] = 0.0f;

    /* slice s is multiplied from stage s % 2 and loaded into register set
     * s % 2; past the end the last slice is re-loaded (and written only to
     * a stage nobody reads) */
    const uint32_t KT = a.k / RBK, last = (KT - 1) * RBK;
    unsigned char *st0 = lds, *st1 = lds + S::STAGE;
    RingRegs<INT8> r0, r1;
    ring_load<INT8>(c, r0, 0);
    ring_load<INT8>(c, r1, min(RBK, last));
    ring_put<INT8>(c, r0, st0);
    ring_barrier();
    /* both steps unconditional in the loop body: a path that skipped the
     * second would leave set 0's loads in flight at the loop head */
    uint32_t kt = 0;
    for (; kt + 1 < KT; kt += 2) {
        ring_step<INT8>(c, acc, st0, st1, r0, r1, min((kt + 2) * RBK, last));
        ring_step<INT8>(c, acc, st1, st0, r1, r0, min((kt + 3) * RBK, last));
    }
    if (kt < KT) ring_step<INT8>(c, acc, st0, st1, r0, r1, last);
    gemm_epilogue<EPI, INT8, MI, NI>(a, acc, m0 + wm * (MI * 32), n0 + wn * (NI * 32), h, i32);
}

#define QW_GEMM_RING_ENTRY(name, EPI, INT8)                                              \
    QW_KERNEL void __launch_bounds__(256, 2) name(qw_gemm_args a) {                     \
        __shared__ __attribute__((aligned(16))) unsigned char lds[2 * RingShape<INT8>::STAGE]; \
        qw_gemm_ring_impl<EPI, INT8>(a, lds);                                            \
    }

QW_GEMM_RING_ENTRY(qw_gemm_bf16_store_r, QW_EPI_STORE, 0)
QW_GEMM_RING_ENTRY(qw_gemm_bf16_gelu_r, QW_EPI_GELU, 0)
QW_GEMM_RING_ENTRY(qw_gemm_bf16_gate_r, QW_EPI_GATE, 0)
QW_GEMM_RING_ENTRY(qw_gemm_i8_store_r, QW_EPI_STORE, 1)
QW_GEMM_RING_ENTRY(qw_gemm_i8_gelu_r, QW_EPI_GELU, 1)
QW_GEMM_RING_ENTRY(qw_gemm_i8_gate_r, QW_EPI_GATE, 1)

/* Kernel argument blocks shared by the host runtime (h3_gpu_hip.cpp) and
 * the gfx950 code object (qwen_kernels.hip). Every kernel takes exactly one
 * of these by value, so hipModuleLaunchKernel passes a single parameter. */
#ifndef QW_KERNEL_ARGS_H
#define QW_KERNEL_ARGS_H

#include <stdint.h>

#define QW_HEAD_DIM 128

/* GEMM epilogues: y = acc * wscale[n] + bias[n] rounded to bf16, then */
enum {
    QW_EPI_STORE = 0, /* store y */
    QW_EPI_GELU = 1,  /* store bf16(gelu_tanh(y)) */
    QW_EPI_GATE = 2,  /* out = bf16(out + y * gate[row_map[r]][n]) in place */
    QW_EPI_QKNORM = 3 /* store y; columns below qk_cols (q then k heads of 128)
                       * first get the per-head RMS norm and the RoPE rotation
                       * of qw_qk_norm_rope_bf16, with its rounding points */
};

typedef struct {
    const void *a;        /* bf16 [m, k], row stride lda */
    const void *w;        /* bf16 or int8 [n, k], row stride k */
    const float *wscale;  /* per-row scale [n]: int8 weights, or bf16 weights
                           * widened from int8; NULL for plain bf16 */
    const uint16_t *bias; /* bf16 [n] or NULL */
    uint16_t *out;        /* bf16 [m, n], row stride ldc */
    const uint16_t *gate; /* QW_EPI_GATE: modulation base (slot offset applied) */
    const uint32_t *row_map;
    uint32_t m, n, k;
    uint32_t lda, ldc;
    uint32_t gate_row_stride; /* elements between modulation rows */
    uint32_t tiles_m, tiles_n;
    uint32_t a_bytes, w_bytes, out_bytes; /* buffer-resource extents (< 2^31) */
    /* Split tiles (split > 1): the first dp_tiles tiles (whole waves of
     * workgroups) run one per workgroup; each remaining tile r is cut into
     * `split` k-ranges, one workgroup each, numbered k-range-major. Every
     * piece stores its fp32 sums in sk_part[r * split + piece]; the last to
     * count itself in sk_flag[r] (0 between launches) adds them in piece
     * order and runs the epilogue. split <= 1: one workgroup per tile. */
    uint32_t dp_tiles, split;
    float *sk_part;
    uint32_t *sk_flag;
    /* QW_EPI_QKNORM: norm weights (k from column qk_cols / 2 on), RoPE
     * tables [rope_rows, 64] (table row = row % rope_rows), epsilon */
    const uint16_t *norm_q, *norm_k;
    const float *rope_cos, *rope_sin;
    uint32_t rope_rows, qk_cols;
    float eps;
    /* Tile walk (split <= 1, bf16 W): tiles [half_from, tiles) run as
     * half_count = 2 (tiles - half_from) half tiles of 128 x 256; 0: none.
     * Split tiles (split > 1, bf16 W): half_count != 0 runs them as half
     * tiles, each in `split` pieces. */
    uint32_t half_from, half_count;
    /* the walk's half tiles on three LDS stages (bf16 W kernels) */
    uint32_t half3;
} qw_gemm_args;

typedef struct {
    uint16_t *out;
    const uint16_t *in;
    const uint16_t *modulation; /* [mod_rows, slots * width] */
    const uint32_t *row_map;
    uint32_t rows, width, slots, scale_slot;
    int32_t shift_slot; /* < 0: none */
    float eps;
} qw_ln_mod_args;

typedef struct {
    uint16_t *out;
    const uint16_t *in;
    const uint16_t *weight; /* effective weight = weight + 1 */
    uint32_t rows, width;
    float eps;
} qw_rms_one_args;

typedef struct {
    uint16_t *qk;           /* [rows, ld]: q at col 0, k at col k_offset */
    const uint16_t *norm_q; /* [128] */
    const uint16_t *norm_k; /* [128] */
    const float *rope_cos;  /* [rope_rows, 64] */
    const float *rope_sin;
    uint32_t rows, heads, ld, k_offset;
    uint32_t rope_rows; /* table row = row % rope_rows (batched sequences) */
    int32_t do_norm, do_rope;
    float eps;
} qw_qk_norm_rope_args;

typedef struct {
    uint16_t *out;
    const uint16_t *residual;
    const uint16_t *branch;
    const uint16_t *modulation;
    const uint32_t *row_map;
    uint32_t rows, width, slots, gate_slot;
} qw_gate_args;

enum { QW_ACT_GELU_TANH = 0, QW_ACT_SILU = 1, QW_ACT_TANH = 2 };

typedef struct {
    uint16_t *out;
    const uint16_t *in;
    uint64_t count;
    int32_t act;
} qw_act_args;

typedef struct {
    uint16_t *out;     /* [rows, width] */
    const uint16_t *fc1; /* [rows, 2 * width] = [gate | up] */
    uint32_t rows, width;
} qw_swiglu_args;

typedef struct {
    uint16_t *out;
    const float *in;
    uint64_t count;
} qw_cast_args;

/* Guided Euler step of the denoise loop (qwen_pipeline.m:421-429,
 * qwen_host.c:372-378): v = neg ? n + cfg (p - n) : p, x += dt v, in fp32
 * with the host's rounding points (no contraction). */
typedef struct {
    float *x;
    const uint16_t *pos; /* bf16 prediction, image rows */
    const uint16_t *neg; /* bf16 unconditional prediction or NULL */
    uint64_t count;
    float dt, cfg;
} qw_euler_args;

typedef struct {
    uint16_t *slots_out; /* [mod_rows, S * hidden] */
    const uint16_t *raw;
    uint32_t mod_rows, hidden;
    int32_t shift_variant;
} qw_reorder_args;

typedef struct {
    uint16_t *out;
    uint64_t count;
    uint64_t seed, stream;
    float std, offset;
} qw_fill_args;

typedef struct {
    int8_t *q;
    float *scales;
    const uint16_t *w;
    uint32_t rows, cols;
} qw_quant_args;

typedef struct {
    uint16_t *out;
    const int8_t *in;
    uint64_t count; /* multiple of 16 */
} qw_widen_args;

typedef struct {
    float *out;
    const int8_t *q;
    const float *scales;
    uint32_t rows, cols;
} qw_dequant_args;

typedef struct {
    void *dst;
    const void *src;
    uint64_t rows, row_bytes, dst_stride, src_stride; /* bytes */
} qw_copy2d_args;

typedef struct {
    uint32_t *p;
    uint64_t count;
} qw_zero_args;

/* Flash attention over a joint sequence: out[b*q_rows + r] attends keys
 * [b*kv_rows, b*kv_rows + limit(r)) of the same batch entry. */
typedef struct {
    uint16_t *out;
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    const uint32_t *kv_limit; /* optional per-query-row limits [q_rows] */
    uint32_t q_rows, kv_rows, heads, batch;
    uint32_t ldq, ldk, ldv, ldo; /* row strides in elements */
    uint32_t text_rows;          /* closed-form limits when kv_limit == NULL */
    int32_t text_causal;
    float scale;      /* softmax scale */
    float scale_log2; /* softmax scale * log2(e) */
} qw_attn_args;

/* LoRA fusion: out[rows, cols] = RNE(fp32(base) + sum of the terms) */
#define QW_LORA_MAX_RANK 256
#define QW_LORA_MAX_TERMS 24
typedef struct {
    const uint16_t *a; /* bf16 [rank, cols] */
    const uint16_t *b; /* bf16 [rows, rank]: fused rows [row0, row0 + rows) */
    uint32_t row0, rows, rank;
    float scale;
} qw_lora_term;
typedef struct {
    uint16_t *out;
    const uint16_t *base;
    uint32_t rows, cols, nterms;
    qw_lora_term terms[QW_LORA_MAX_TERMS];
} qw_lora_args;

#endif

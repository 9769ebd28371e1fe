/* qdit_oracle — CPU restatement of the qwen-metal DiT denoising forward.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it. The product library (libqwen_dit_hip.so) never links or calls it.
 *
 * Every function states the reference file:line whose semantics it follows
 * (paths relative to the wangyancz/qwen-metal tree). All tensors are
 * row-major; bf16 values travel as uint16_t bit patterns. Each op computes
 * in fp32 and rounds to bf16 (round-to-nearest-even) at its output, the
 * rounding point of the reference kernels.
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   bf16 RNE/trunc .............. closed form + exhaustive tie cases
 *   rng (PCG32 + Box-Muller) .... oracle/_ref (reference qwen_host.c built)
 *   schedule / shift ............ tests/golden/host_ref.json (4 cases) +
 *                                 pipeline_fixture/schedule_*.f32 + _ref
 *   rope tables ................. dit_fixture a/b/c rope, pipeline_fixture
 *                                 rope_{4,8}, host_ref.json samples, _ref
 *   rope tables, ti2i blocks .... hand-computed positions of a 3-block
 *                                 layout; one block = the single-grid table
 *                                 with its frame moved by the text rows
 *   timestep features ........... closed form (cos/sin of known angles)
 *   layer_norm_mod .............. dit_fixture a/b joint_in -> attn_in
 *   gate (+ layer_norm_mod) ..... dit_fixture attn_out/mlp_in/mlp_out/
 *                                 block_out identities
 *   norm_out LN ................. dit_fixture block_out -> norm_out
 *                                 (per-column ratio consistency)
 *   linear / linear_i8 .......... brute-force double dot on tiny shapes,
 *                                 identity/one-hot weights
 *   attention ................... brute-force double softmax, single key
 *                                 -> V, uniform scores -> mean V, limits
 *                                 reducing to causal / full
 *   head_rms_norm, qk_rope ...... closed form: norm -> unit RMS, rotation
 *                                 preserves pair norm, zero angle = identity
 *   gelu / silu / swiglu ........ textbook values at known points
 *   int8 quantizer .............. closed form (max row -> +-127, ties even)
 *   modulation reorder .......... dit_fixture modulation layout (slots)
 *   embed / conditioning / block / final / forward / ti2i forward
 *                                 structured weights reduce each stage to
 *                                 a float64 closed form (q = k = 0 gives
 *                                 uniform attention, identity and scaled
 *                                 identity linears, distinct slot values),
 *                                 zero gates give the identity, masking
 *                                 invariants, forward = the reference's
 *                                 composition bit for bit
 *                                 (tests/test_oracle_composition.py; each
 *                                 check fails under a swapped slot, a
 *                                 misplaced shift or activation, a wrong
 *                                 row_map, mask or feature row)
 */
#ifndef QDIT_ORACLE_H
#define QDIT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 ------------------------------------------------------------ */
uint16_t qo_f32_to_bf16(float value);       /* RNE, h3_shaders.metal:16-20 */
uint16_t qo_f32_to_bf16_trunc(float value); /* truncation, qwen_dit.m:229-233 */
float qo_bf16_to_f32(uint16_t bits);        /* h3_shaders.metal:11-13 */
void qo_bf16_to_f32_array(const uint16_t *in, float *out, size_t n);
void qo_f32_to_bf16_array(const float *in, uint16_t *out, size_t n);

/* ---- host math: qwen_host.c / qwen_pipeline.m ------------------------- */
typedef struct {
    uint64_t state;
    uint64_t increment;
    float spare;
    int has_spare;
} qo_rng;
void qo_rng_seed(qo_rng *rng, uint64_t seed);       /* qwen_host.c:452-458 */
uint32_t qo_rng_u32(qo_rng *rng);                   /* qwen_host.c:440-446 */
float qo_rng_normal(qo_rng *rng);                   /* qwen_host.c:460-471 */
void qo_rng_fill_normal(qo_rng *rng, float *v, size_t n);
double qo_calculate_shift(int image_seq_len);       /* qwen_host.c:18-26 */
/* qwen_host.c:335-370: exponential dynamic shift, terminal 0.02, sigma[steps]=0 */
int qo_schedule_build(int steps, int image_seq_len, float *sigma);
/* qwen_pipeline.m:130-205 with an explicit exp(mu) and optional terminal
 * stretch (terminal <= 0 disables it). */
int qo_schedule_exp_mu(int steps, double exp_mu, double terminal, float *sigma);
/* qwen_host.c:372-378 */
void qo_euler_step(float *sample, const float *velocity, size_t n,
                   float sigma, float sigma_next);
/* qwen_host.c:388-430: one entry of the released per-axis tables */
void qo_rope_table_entry(int axis_dim, int table_row, int pair,
                         float *cos_out, float *sin_out);
/* qwen_pipeline.m:212-273: joint [text_rows + gh*gw, 64] tables */
void qo_rope_tables(uint32_t text_rows, uint32_t gh, uint32_t gw,
                    float *cos_out, float *sin_out);
/* ti2i multi-block tables (qwen_pipeline.m:611-680); returns the rows. */
size_t qo_rope_tables_blocks(const uint32_t *block_h, const uint32_t *block_w,
                             const uint32_t *text_before, uint32_t n_blocks,
                             float *cos_out, float *sin_out);
/* qwen_dit.m:1085-1096 */
void qo_timestep_features(const float *sigmas, size_t count, float *features);

/* Synthetic N(0,1)-like generator used for weights and activations on both
 * the GPU and the oracle: counter-based, integer arithmetic, bit-identical
 * on CPU and GPU. value(i) = std * (sum of 12 16-bit uniforms - 6) from
 * splitmix64(seed, stream, i); stored as bf16 RNE (or +1 offset). */
float qo_synth_normal(uint64_t seed, uint64_t stream, uint64_t index);
void qo_fill_normal_bf16(uint16_t *out, size_t n, uint64_t seed,
                         uint64_t stream, float std, float offset);

/* ---- kernels (h3_shaders.metal / MPSGraph semantics) ------------------ */
/* C = A * B^T in fp32, A [m,k] lda, B [n,k] ldb, C [m,n] ldc. OpenMP. */
void qo_gemm_nt_f32(const float *a, size_t lda, const float *b, size_t ldb,
                    float *c, size_t ldc, size_t m, size_t n, size_t k);
/* y[rows, n] (row stride ldy) = bf16(x[rows,k] . w[n,k]^T + bias)
 * h3_gpu.m:2618-2695 / h3_shaders.metal:788-816 */
void qo_linear(uint16_t *y, size_t ldy, const uint16_t *x, size_t ldx,
               const uint16_t *w, const uint16_t *bias, size_t rows,
               size_t k, size_t n);
/* int8 weight-only: y = bf16((x . q^T) * scale[n] + bias) */
void qo_linear_i8(uint16_t *y, size_t ldy, const uint16_t *x, size_t ldx,
                  const int8_t *q, const float *scales, const uint16_t *bias,
                  size_t rows, size_t k, size_t n);
/* h3_shaders.metal:1320-1390 with clip 1.0 (h3_gpu.m:3305-3312) */
void qo_quantize_int8_rows(int8_t *q, float *scales, const uint16_t *w,
                           size_t rows, size_t cols);
/* dequantised weight q * scale in fp32 */
void qo_dequant_int8_rows(float *w, const int8_t *q, const float *scales,
                          size_t rows, size_t cols);
/* h3_shaders.metal:4767-4815 (+ optional shift slot; shift_slot < 0 = none) */
void qo_layer_norm_mod(uint16_t *out, const uint16_t *in,
                       const uint16_t *modulation, const uint32_t *row_map,
                       size_t rows, size_t width, uint32_t slots,
                       uint32_t scale_slot, int shift_slot, float eps);
/* torch_rounding = 1 reproduces the bf16 rounding points of the diffusers
 * module that wrote tests/dit_fixture (LN output and 1 + scale each rounded
 * before the product); 0 is the reference kernel's single rounding. */
void qo_layer_norm_mod_r(uint16_t *out, const uint16_t *in,
                         const uint16_t *modulation, const uint32_t *row_map,
                         size_t rows, size_t width, uint32_t slots,
                         uint32_t scale_slot, int shift_slot, float eps,
                         int torch_rounding);
/* h3_shaders.metal:4817-4850 */
void qo_rms_norm_one(uint16_t *out, const uint16_t *in, const uint16_t *w,
                     size_t rows, size_t width, float eps);
/* h3_shaders.metal:4309-4329, in place on [rows, heads, 128], row stride ld */
void qo_head_rms_norm(uint16_t *t, size_t ld, const uint16_t *w, size_t rows,
                      size_t heads, size_t head_dim, float eps);
/* h3_shaders.metal:4864-4896, in place, row stride ld, tables [rows, hd/2] */
void qo_qk_rope(uint16_t *t, size_t ld, const float *cos_t, const float *sin_t,
                size_t rows, size_t heads, size_t head_dim);
/* h3_shaders.metal:3583-3599 */
void qo_gate(uint16_t *out, const uint16_t *residual, const uint16_t *branch,
             const uint16_t *modulation, const uint32_t *row_map, size_t rows,
             size_t width, uint32_t slots, uint32_t gate_slot);
/* torch_rounding = 1 rounds branch * gate to bf16 before the add (the
 * diffusers fixture's rounding point). */
void qo_gate_r(uint16_t *out, const uint16_t *residual, const uint16_t *branch,
               const uint16_t *modulation, const uint32_t *row_map,
               size_t rows, size_t width, uint32_t slots, uint32_t gate_slot,
               int torch_rounding);
/* h3_shaders.metal:3385-3408 (approximate = 1) */
void qo_gelu_tanh(uint16_t *out, const uint16_t *in, size_t n);
/* h3_shaders.metal:3284-3291 */
void qo_silu(uint16_t *out, const uint16_t *in, size_t n);
/* h3_shaders.metal:5078-5095, fc1 [rows, 2*width] = [gate | up] */
void qo_swiglu(uint16_t *out, const uint16_t *fc1, size_t rows, size_t width);
/* Prefix-visible attention, fp32 softmax (tests/test_prefix_kernel.c:72-97).
 * q [q_rows, heads*hd] row stride ldq; k, v [kv_rows, heads*hd] strides ldk,
 * ldv; out [q_rows, heads*hd] stride ldo; limits[q_rows] visible key count. */
void qo_attention(uint16_t *out, size_t ldo, const uint16_t *q, size_t ldq,
                  const uint16_t *k, size_t ldk, const uint16_t *v, size_t ldv,
                  const uint32_t *limits, size_t q_rows, size_t kv_rows,
                  size_t heads, size_t head_dim, float scale);
/* The same with the t2i text-row rule (h3_shaders.metal:4397-4401): rows
 * below prescale_rows contract bf16(q * scale) with K, unscaled after. */
void qo_attention_ex(uint16_t *out, size_t ldo, const uint16_t *q, size_t ldq,
                     const uint16_t *k, size_t ldk, const uint16_t *v, size_t ldv,
                     const uint32_t *limits, size_t q_rows, size_t kv_rows,
                     size_t heads, size_t head_dim, float scale,
                     size_t prescale_rows);
/* qwen_dit.m:1651-1665 (t2i form): text rows causal (or full text prefix),
 * image rows see every key. */
void qo_t2i_limits(uint32_t *limits, uint32_t rows, uint32_t text_rows,
                   int text_causal);
/* qwen_dit.m:1159-1186: raw modulation [mod_rows, S*H] in the checkpoint's
 * column order -> slot layout. Reference (4 slots): [s1|g1|s2|g2] ->
 * [s1, s2, tanh g1, tanh g2]. Shift variant (6 slots): [sh1|s1|g1|sh2|s2|g2]
 * -> [s1, s2, tanh g1, tanh g2, sh1, sh2]. tanh in fp32, truncating store. */
void qo_modulation_reorder(uint16_t *slots_out, const uint16_t *raw,
                           size_t mod_rows, size_t hidden, int shift_variant);

/* ---- model ------------------------------------------------------------ */
enum { QO_MLP_SWIGLU = 0, QO_MLP_GELU_TANH = 1 };

typedef struct {
    uint32_t hidden, heads, mlp_width, text_dim, z_dim, layers;
    int mlp_act;      /* QO_MLP_* */
    int adaln_shift;  /* 0: scale+gate (4 slots), 1: shift+scale+gate (6) */
    int has_bias;
    int text_causal;
    int int8_weights;
} qo_config;

typedef struct {
    uint16_t *w;      /* bf16 [n, k] */
    int8_t *q;        /* int8 [n, k] when quantized */
    float *scales;    /* [n] */
    uint16_t *bias;   /* bf16 [n] or NULL */
    uint32_t n, k;
    int int8;
} qo_lin;

typedef struct {
    qo_lin qkv, out, fc1, fc2;
    uint16_t *norm_q, *norm_k; /* bf16 [128] */
} qo_layer;

typedef struct {
    qo_config cfg;
    qo_layer *layer;
    qo_lin img_in, txt_in1, txt_in2, time_l1, time_l2, mod, norm_out, proj_out;
    uint16_t *txt_norm; /* bf16 [text_dim] */
} qo_model;

/* Seeded random model: the same streams the GPU library generates. */
int qo_model_init_random(qo_model *m, const qo_config *cfg, uint64_t seed,
                         uint32_t layers_to_build);
void qo_model_free(qo_model *m);
void qo_apply_linear(const qo_lin *l, uint16_t *y, size_t ldy,
                     const uint16_t *x, size_t ldx, size_t rows);

/* qwen_dit.m:1031-1083 -> joint [text_rows + image_rows, hidden] */
void qo_embed(const qo_model *m, const uint16_t *text_in, uint32_t text_rows,
              const uint16_t *latents, uint32_t image_rows, uint16_t *joint);
/* qwen_dit.m:1098-1192: temb [mod_rows,H], modulation slots
 * [mod_rows, slots*H], norm_out [mod_rows, H or 2H] */
void qo_conditioning(const qo_model *m, const float *features,
                     uint32_t mod_rows, uint16_t *temb, uint16_t *modulation,
                     uint16_t *norm_out_mod);
/* qwen_dit.m:1220-1476, hidden in place. limits NULL -> t2i limits. */
void qo_block(const qo_model *m, int layer, uint16_t *hidden,
              const uint16_t *modulation, const float *rope_cos,
              const float *rope_sin, const uint32_t *row_map, uint32_t rows,
              uint32_t text_rows, const uint32_t *limits,
              uint16_t *debug_attn);
/* qo_block evaluated for the output rows listed in sample[n_sample] only
 * (all rows still feed K and V): out [n_sample, H] in sample order. t2i
 * limits; the same arithmetic as qo_block for those rows. */
void qo_block_rows(const qo_model *m, int layer, const uint16_t *hidden,
                   const uint16_t *modulation, const float *rope_cos,
                   const float *rope_sin, const uint32_t *row_map,
                   uint32_t rows, uint32_t text_rows, const uint32_t *sample,
                   uint32_t n_sample, uint16_t *out);
/* qwen_dit.m:1478-1496 */
void qo_final(const qo_model *m, const uint16_t *hidden,
              const uint16_t *norm_out_mod, const uint32_t *row_map,
              uint32_t rows, uint16_t *output);
/* qwen_dit.m:1498-1568, one branch; output [rows, z_dim]. Runs layers
 * [0, layers) (layers <= built layers). */
int qo_forward(const qo_model *m, const uint16_t *text_in, uint32_t text_rows,
               const uint16_t *latents, uint32_t image_rows, float sigma,
               const float *rope_cos, const float *rope_sin, uint32_t layers,
               uint16_t *output);

/* A ti2i joint-sequence run (qwen_dit.h:21-29): text rows from text_in or
 * image rows from latents, starting at src_offset of that source. */
typedef struct {
    uint32_t rows;
    int is_image;
    uint32_t src_offset;
} qo_segment;
/* qwen_dit.m:1651-1665: text rows see their run up to themselves (run
 * start + r + 1), image rows their whole run (run end); limits[rows]. */
void qo_prefix_limits(const qo_segment *segs, uint32_t seg_count, uint32_t *limits);
/* The ti2i forward's full pass (qwen_dit.m:1667-1860): every text_in row
 * and every latents row projected (qwen_dit.m:1572-1648), runs scattered
 * into the joint order, rows before the last run modulated from t = 0 and
 * the last (target image) run from sigma, block-causal prefix limits, all
 * blocks, the final head over every row. output [rows, z_dim]. Returns 0
 * when the last run is not an image run or a run reads past its source. */
int qo_forward_ti2i(const qo_model *m, const uint16_t *text_in, uint32_t text_total,
                    const uint16_t *latents, uint32_t image_total, const qo_segment *segs,
                    uint32_t seg_count, float sigma, const float *rope_cos,
                    const float *rope_sin, uint32_t layers, uint16_t *output);

/* Threads used by the OpenMP regions (for the baseline report). */
int qo_num_threads(void);
/* 0 (default): fp32 softmax probabilities; 1: probabilities rounded to
 * bf16 before P.V, as the reference's flash kernel does. */
void qo_set_attention_p_mode(int mode);
/* K-slice width of the fp32 contractions (default 512): only the
 * summation order changes. */
void qo_set_gemm_kc(size_t kc);

#ifdef __cplusplus
}
#endif
#endif

/* qwen_dit — the Qwen-Image DiT denoising forward on MI355X (gfx950).
 *
 * Drop-in for the reference's qwen_dit.h (t2i path): same entry points,
 * argument meaning, tensor layouts and error convention (int 1/0 + error
 * string). Activations are bf16 [rows, hidden] (text rows first, then
 * image rows), RoPE tables fp32 [rows, 64], latents bf16 [image_rows, z].
 *
 * Modulation slot layout ([mod_rows, slots * hidden], reference
 * qwen_dit.h:9-17):
 *   slot 0: mod1.scale   slot 1: mod2.scale
 *   slot 2: tanh(mod1.gate)   slot 3: tanh(mod2.gate)
 *   shift variant only: slot 4: mod1.shift   slot 5: mod2.shift
 * norm_out_scale: [mod_rows, hidden] (scale), shift variant [mod_rows,
 * 2 * hidden] (scale | shift).
 *
 * The block is parametric so one kernel family serves the reference model
 * (hidden 4096, 32 heads, SwiGLU 12288, scale+gate, no bias, causal text)
 * and the Flux-like benchmark geometry (hidden 3072, 24 heads, GELU-tanh
 * 12288, shift+scale+gate, bias, text attends the whole text prefix). */
#ifndef QWEN_DIT_H
#define QWEN_DIT_H

#include <stddef.h>
#include <stdint.h>

#include "h3_gpu.h"
#include "qwen_host.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qw_dit qw_dit;

/* reference qwen_dit.h:25-29 */
typedef struct {
    uint32_t rows;
    int is_image;
    uint32_t src_offset;
} qw_dit_segment;

enum { QW_MLP_SWIGLU = 0, QW_MLP_GELU_TANH = 1 };

typedef struct {
    uint32_t hidden;    /* multiple of 256 */
    uint32_t heads;     /* hidden = heads * 128 */
    uint32_t mlp_width; /* multiple of 64 */
    uint32_t text_dim;  /* text_in width (text-encoder hidden) */
    uint32_t z_dim;     /* latent channels per token (64) */
    uint32_t layers;
    int mlp_act;        /* QW_MLP_* */
    int adaln_shift;    /* 0: scale+gate (4 slots), 1: shift+scale+gate (6) */
    int has_bias;       /* biases on every linear */
    int text_causal;    /* text rows causal among text (1) or full text (0) */
    int int8_weights;   /* block linears int8 weight-only, fp32 row scales */
} qw_dit_config;

/* Reference Qwen-Image-2.1 geometry (qwen_host.h:208-229). */
void qw_dit_config_reference(qw_dit_config *cfg);
/* Benchmark geometry: hidden 3072, 24 heads, GELU-tanh 12288, shift,
 * bias, full text prefix, 32 layers. */
void qw_dit_config_baseline(qw_dit_config *cfg);

/* reference qwen_dit.h:31-32 (qwen_dit.m:235-371): the reference geometry
 * (qw_dit_config_reference with `layers` blocks) from the safetensors
 * shards in <model_dir>/transformer, tensors by their diffusers names
 * (img_in, txt_in.*, time_text_embed.timestep_embedder.linear_{1,2},
 * modulation.1, norm_out.linear, proj_out, transformer_blocks.N.attn.to_{q,k,v},
 * .to_out.0, .norm_{q,k}, .img_mlp.{gate_layer,proj,out}), bf16 with exact
 * shapes. q, k, v rows are fused into one [3H, H] weight and gate, proj into
 * [2F, H]. Returns NULL with the reason (missing tensor, dtype, shape, I/O). */
qw_dit *qw_dit_create(h3_gpu *gpu, const char *model_dir, int layers,
                      char *error, size_t error_size);
/* The same loader for any geometry of that architecture (cfg->mlp_act =
 * SwiGLU, no shift, no biases): shapes follow cfg, and cfg->int8_weights
 * quantises the block linears on device after loading. No counterpart in
 * the reference. */
qw_dit *qw_dit_load(h3_gpu *gpu, const char *model_dir,
                    const qw_dit_config *cfg, char *error, size_t error_size);
/* Seeded random weights, N(0, 0.02) bf16 from the counter-based generator
 * (weight stream ids below); norm_q/norm_k = 1 + N(0, 0.02); block
 * linears quantised on device when cfg->int8_weights. */
qw_dit *qw_dit_create_random(h3_gpu *gpu, const qw_dit_config *cfg,
                             uint64_t seed, char *error, size_t error_size);
void qw_dit_free(qw_dit *dit);
const qw_dit_config *qw_dit_get_config(const qw_dit *dit);

/* Weight streams of qw_dit_create_random (generator stream ids). */
enum {
    QW_W_IMG_IN = 1, QW_W_IMG_IN_B, QW_W_TXT_NORM, QW_W_TXT_IN1, QW_W_TXT_IN1_B,
    QW_W_TXT_IN2, QW_W_TXT_IN2_B, QW_W_TIME_L1, QW_W_TIME_L1_B, QW_W_TIME_L2,
    QW_W_TIME_L2_B, QW_W_MOD, QW_W_MOD_B, QW_W_NORM_OUT, QW_W_NORM_OUT_B,
    QW_W_PROJ_OUT, QW_W_PROJ_OUT_B
};
enum {
    QW_L_QKV = 1, QW_L_QKV_B, QW_L_OUT, QW_L_OUT_B, QW_L_FC1, QW_L_FC1_B,
    QW_L_FC2, QW_L_FC2_B, QW_L_NORM_Q, QW_L_NORM_K
};
#define QW_LAYER_STREAM(layer, field) (256ull * (uint64_t)((layer) + 1) + (field))

/* reference qwen_dit.h:84-86: the live weight tensor of one block field,
 * 0 = to_q, 1 = to_k, 2 = to_v, 3 = to_out, 4 = fc1, 5 = fc2. q, k and v
 * are non-owning [H, H] row views of the fused [3H, H] weight, owned by the
 * model (valid until the next LoRA change or qw_dit_free). int8 weights
 * return the int8 tensor; qw_dit_block_scales gives its fp32 row scales
 * (for fields 0-2 the [H] slice of the fused scales). */
const h3_gpu_tensor *qw_dit_block_tensor(const qw_dit *dit, int block,
                                         int field);
const h3_gpu_tensor *qw_dit_block_scales(const qw_dit *dit, int block,
                                         int field);

/* reference qwen_dit.h:81-84 */
int qw_dit_embed(qw_dit *dit, const h3_gpu_tensor *text_in,
                 uint32_t text_rows, const h3_gpu_tensor *latents,
                 uint32_t image_rows, h3_gpu_tensor *joint, char *error,
                 size_t error_size);

/* reference qwen_dit.h:89-90 */
void qw_dit_timestep_features(const float *row_sigmas, size_t count,
                              float *features);

/* reference qwen_dit.h:94-98. The slot reorder runs on device: no host
 * round trip, no submit inside. */
int qw_dit_conditioning(qw_dit *dit, const h3_gpu_tensor *features,
                        uint32_t mod_rows, h3_gpu_tensor *temb,
                        h3_gpu_tensor *modulation,
                        h3_gpu_tensor *norm_out_scale, char *error,
                        size_t error_size);

/* reference qwen_dit.h:117-124. kv_limit (u32 [rows]) replaces the t2i
 * topology with per-row prefix limits; segs are accepted and unused (one
 * prefix kernel serves every run layout). k_out/v_out receive the roped
 * K / V rows [rows, hidden] when given. debug_attn receives the merged
 * attention before the output projection. */
int qw_dit_block(qw_dit *dit, int layer, h3_gpu_tensor *hidden,
                 const h3_gpu_tensor *modulation,
                 const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin,
                 const h3_gpu_tensor *row_map, uint32_t rows,
                 uint32_t text_rows, const h3_gpu_tensor *kv_limit,
                 const qw_dit_segment *segs, uint32_t seg_count,
                 h3_gpu_tensor *k_out, h3_gpu_tensor *v_out,
                 h3_gpu_tensor *debug_attn, char *error, size_t error_size);

/* reference qwen_dit.h:133-139 (qwen_dit.m:1572-1648): text runs from the
 * rows of text_in at src_offset, image runs from the rows of latents at
 * src_offset, in segs order into joint. Each run is embedded straight into
 * its joint rows (the embedding is row-wise). */
int qw_dit_embed_segments(qw_dit *dit, const h3_gpu_tensor *text_in,
                          const h3_gpu_tensor *latents,
                          const qw_dit_segment *segs, uint32_t seg_count,
                          h3_gpu_tensor *joint, char *error,
                          size_t error_size);

/* reference qwen_dit.h:166-181 (qwen_dit.m:1667-1967): ti2i forward over a
 * segmented joint sequence whose last run is the target image. Rows before
 * it modulate from t = 0, the target from sigma; attention is block-causal
 * as a prefix table (qw_dit_prefix_limits). cache_slot (0 or 1) keeps the
 * K/V of every row of every layer from a full pass; a later call with the
 * same run layout recomputes only the target rows, against those cached
 * K/V, and writes only the target rows of output. Output [rows, z_dim]. */
int qw_dit_forward_ti2i(qw_dit *dit, const h3_gpu_tensor *text_in,
                        const h3_gpu_tensor *latents,
                        const qw_dit_segment *segs, uint32_t seg_count,
                        uint32_t cache_slot, const h3_gpu_tensor *rope_cos,
                        const h3_gpu_tensor *rope_sin, float sigma,
                        h3_gpu_tensor *output, char *error,
                        size_t error_size);

/* reference qwen_dit.h:42-82: LoRA adapters (single safetensors files,
 * rank-r pairs transformer_blocks.N.<module>.lora_A / .lora_B.default.weight
 * for the modules attn.to_q, .to_k, .to_v, .to_out.0, img_mlp.gate_layer,
 * .proj, .out; A bf16 [r, in], B bf16 [out, r]). Adapters stack:
 * W' = RNE_bf16(fp32(W) + sum_a scale_a B_a A_a), rebuilt on the device
 * from the kept base weights on every change (one rounding, order
 * independent); missing targets are skipped; no lora_alpha (scale is the
 * caller's strength). Any change drops the ti2i caches. A failed rebuild
 * resets the stack to none. Adapters fuse into bf16 block weights of the
 * reference architecture: an int8 or GELU/bias model refuses them. */
#define QW_DIT_MAX_LORA 8
/* new path: appended, or an existing path's scale updated; fails without
 * a state change on an unreadable file, no matching tensor or a full stack */
int qw_dit_apply_lora(qw_dit *dit, const char *path, float scale,
                      char *error, size_t error_size);
/* NULL or "" removes all; an unknown path is a no-op */
int qw_dit_remove_lora(qw_dit *dit, const char *path, char *error,
                       size_t error_size);
/* replaces the single active adapter; a broken file leaves it active */
int qw_dit_switch_lora(qw_dit *dit, const char *path, float scale,
                       char *error, size_t error_size);
int qw_dit_clear_lora(qw_dit *dit, char *error, size_t error_size);
int qw_dit_lora_count(const qw_dit *dit);
const char *qw_dit_lora_path_at(const qw_dit *dit, int index);
float qw_dit_lora_scale_at(const qw_dit *dit, int index);

/* reference qwen_dit.h:35-40: drop both ti2i caches (they hold one
 * request's conditioning; call at the end of every ti2i generation). */
void qw_dit_ti2i_cache_clear(qw_dit *dit);

/* reference qwen_dit.h:141-145 */
void qw_dit_prefix_limits(const qw_dit_segment *segs, uint32_t seg_count,
                          uint32_t *limits);

/* reference qwen_dit.h:149-152 */
int qw_dit_final(qw_dit *dit, h3_gpu_tensor *hidden,
                 const h3_gpu_tensor *norm_out_scale,
                 const h3_gpu_tensor *row_map, uint32_t rows,
                 h3_gpu_tensor *output, char *error, size_t error_size);

/* reference qwen_dit.h:159-165 */
int qw_dit_forward(qw_dit *dit, const h3_gpu_tensor *text_in,
                   uint32_t text_rows, const h3_gpu_tensor *latents,
                   uint32_t image_rows, float sigma,
                   const h3_gpu_tensor *rope_cos,
                   const h3_gpu_tensor *rope_sin, h3_gpu_tensor *output,
                   char *error, size_t error_size);

/* Batched forward (CFG cond/uncond as one launch sequence): batch entries
 * stacked along rows. text_in [batch * text_rows, text_dim], latents
 * [batch * image_rows, z_dim], output [batch * rows, z_dim]; rope tables
 * [rows, 64] shared by every entry; one sigma for all. Enqueues only (no
 * submit): the caller submits. */
int qw_dit_forward_batch(qw_dit *dit, const h3_gpu_tensor *text_in,
                         uint32_t text_rows, const h3_gpu_tensor *latents,
                         uint32_t image_rows, uint32_t batch, float sigma,
                         const h3_gpu_tensor *rope_cos,
                         const h3_gpu_tensor *rope_sin,
                         h3_gpu_tensor *output, char *error,
                         size_t error_size);

/* qw_dit_forward_batch with the timestep features read from a device
 * table: f32 [2, 256] at feature_offset = qw_dit_timestep_features of
 * {sigma, 0}. No host transfer, so a denoise loop can enqueue every step
 * without synchronising. No counterpart in the reference. */
int qw_dit_forward_batch_features(qw_dit *dit, const h3_gpu_tensor *text_in,
                                  uint32_t text_rows, const h3_gpu_tensor *latents,
                                  uint32_t image_rows, uint32_t batch,
                                  const h3_gpu_tensor *features, size_t feature_offset,
                                  const h3_gpu_tensor *rope_cos,
                                  const h3_gpu_tensor *rope_sin, h3_gpu_tensor *output,
                                  char *error, size_t error_size);

/* Per-stage device time of the last qw_dit_forward_batch when
 * QWEN_BLOCK_PROFILE is on (ms summed over layers): input (LN + QKV +
 * norm/rope), attention, to_out+gate, LN2, mlp+gate; plus embed /
 * conditioning and final. Returns the number of stages written. */
int qw_dit_block_profile(const qw_dit *dit, double *ms, int max_stages);

/* No counterpart in the reference (a measurement aid): while on, every
 * block records one qw_gpu_span (qwen_gpu_ext.h) per stage on the
 * forward's stream, with no synchronisation, tagged QW_SPAN_*: the first
 * LN-mod, the QKV linear (with its q/k norm + RoPE, and its int8 widening
 * pass where it has one), attention, the out linear + gate, the second
 * LN-mod, the up linear (+ GELU or SwiGLU), the down linear + gate. The
 * caller reads them with qw_gpu_span_collect (at most 4096 between
 * collects: 18 forwards of 32 layers). */
enum { QW_SPAN_LN1 = 0, QW_SPAN_QKV, QW_SPAN_ATTN, QW_SPAN_OUT, QW_SPAN_LN2, QW_SPAN_UP,
       QW_SPAN_DOWN, QW_SPAN_COUNT };
int qw_dit_set_spans(qw_dit *dit, int on);

/* Diagnostic trace of the t2i forward (qw_dit_forward*), for per-block
 * parity checks; no reference counterpart (the reference dumps stages
 * through its QWEN_* diagnostic switches instead). While set, each
 * forward copies, on its stream: the joint hidden state after the embed
 * into rows [0, M) of `hidden` and after block l into rows
 * [(l + 1) M, (l + 2) M) (M = batch * rows, [M, hidden] bf16 each, so
 * `hidden` holds (layers + 1) M hidden); and the slot-ordered modulation
 * [2, slots * hidden] into `modulation` (may be NULL). A forward whose
 * trace tensors are too small fails with an error. NULL, NULL stops
 * tracing. The caller keeps ownership of both tensors. */
int qw_dit_set_trace(qw_dit *dit, h3_gpu_tensor *hidden, h3_gpu_tensor *modulation);

#ifdef __cplusplus
}
#endif
#endif

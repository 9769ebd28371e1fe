/* qwen_dit.c — C11 host of the DiT denoising forward over the HIP runtime.
 *
 * Follows the reference's qwen_dit.m (t2i path) call for call, with the
 * MI355X layout changes:
 *   - q|k|v come from ONE fused [rows, 3H] projection, per-head RMSNorm and
 *     RoPE run fused in place on it, and attention reads q/k/v straight out
 *     of it (no row-slice copies, qwen_dit.m:1373-1440);
 *   - GELU is the up-projection's epilogue, the residual gate
 *     (h += tanh(g) * branch) the down/out projections' epilogue, so the
 *     branch tensor never round-trips HBM;
 *   - the conditioning reorder runs on device (no submit + host round trip,
 *     qwen_dit.m:1140-1186);
 *   - CFG batch entries are stacked along rows: every linear sees
 *     M = batch * rows, attention has a batch grid dimension.
 * Rounding points are the reference kernels' (bf16 RNE at each reference
 * op boundary). */
#define _DEFAULT_SOURCE /* strdup */
#include "../../include/qwen_dit.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <strings.h>

#include "../../include/qwen_gpu_ext.h"
#include "../../include/h3_weights.h"

typedef struct {
    h3_gpu_tensor *w;      /* bf16 or int8 [n, k] */
    h3_gpu_tensor *scales; /* f32 [n] for int8 */
    h3_gpu_tensor *bias;   /* bf16 [n] or NULL */
    uint32_t n, k;
} qw_lin;

typedef struct {
    qw_lin qkv, out, fc1, fc2;
    h3_gpu_tensor *norm_q, *norm_k;
} qw_layer;

enum { P_EMBED, P_COND, P_INPUT, P_ATTN, P_OUT, P_LN, P_MLP, P_FINAL, P_COUNT };

struct qw_dit {
    h3_gpu *gpu;
    qw_dit_config cfg;
    qw_layer *layer;
    qw_lin img_in, txt_in1, txt_in2, time_l1, time_l2, mod, norm_out, proj_out;
    h3_gpu_tensor *txt_norm;
    /* activation workspaces, sized for ws_rows rows */
    uint32_t ws_rows;
    h3_gpu_tensor *ws_mod, *ws_qkv, *ws_attn, *ws_wide, *ws_act;
    uint32_t ws_text_rows;
    h3_gpu_tensor *ws_tnorm, *ws_twide;
    /* conditioning (2 modulation rows) */
    h3_gpu_tensor *feat, *feat_bf16, *c_wide, *c_silu, *temb, *mod_raw,
        *modulation, *norm_out_mod;
    /* forward-owned joint sequence and row map */
    uint32_t joint_rows;
    h3_gpu_tensor *joint;
    h3_gpu_tensor *row_map;
    uint32_t rm_rows, rm_text, rm_batch;
    int profile;
    double prof_ms[P_COUNT];
    int spans; /* qw_dit_set_spans: stage spans on the stream (QW_SPAN_*) */
    /* qw_dit_set_trace: per-block hidden states and the modulation */
    h3_gpu_tensor *trace_hidden, *trace_mod;
    /* LoRA adapters, in stack order; while any is active, base[4 l + j]
     * keeps layer l's base weight j (qkv, out, fc1, fc2) and the layer
     * holds the fused copy */
    struct qw_lora {
        char *path;
        float scale;
        uint32_t rank;
        h3_st_header header;
    } lora[QW_DIT_MAX_LORA];
    int n_lora;
    h3_gpu_tensor **lora_base;
    /* non-owning q / k / v row views of each layer's fused qkv weight (and
     * of its int8 row scales), made on first request and remade when the
     * live weight changes (LoRA fusion swaps it) */
    struct qw_qkv_views {
        const h3_gpu_tensor *src_w, *src_s;
        h3_gpu_tensor *w[3], *s[3];
    } *qkv_views;
    /* ti2i cross-step caches (slot 0: guided branch, 1: CFG negative) */
    struct qw_ti2i_cache {
        uint32_t rows, target_rows, seg_count;
        qw_dit_segment *segs;
        h3_gpu_tensor **k, **v;  /* per layer [rows, H]: every row's K / V */
        h3_gpu_tensor *th, *row0; /* target hidden [target_rows, H]; zeros */
        int filled;
    } ti2i[2];
};

static int set_error(char *error, size_t n, const char *fmt, ...) {
    if (error && n) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(error, n, fmt, ap);
        va_end(ap);
    }
    return 0;
}

static int env_on(const char *name) {
    const char *v = getenv(name);
    if (!v || !*v) return 0;
    return strcmp(v, "0") && strcasecmp(v, "off") && strcasecmp(v, "false");
}

static uint32_t slots_of(const qw_dit_config *c) { return c->adaln_shift ? 6u : 4u; }

void qw_dit_config_reference(qw_dit_config *c) {
    memset(c, 0, sizeof(*c));
    c->hidden = 4096;
    c->heads = 32;
    c->mlp_width = 12288;
    c->text_dim = 4096;
    c->z_dim = 64;
    c->layers = 32;
    c->mlp_act = QW_MLP_SWIGLU;
    c->adaln_shift = 0;
    c->has_bias = 0;
    c->text_causal = 1;
    c->int8_weights = 0;
}

void qw_dit_config_baseline(qw_dit_config *c) {
    memset(c, 0, sizeof(*c));
    c->hidden = 3072;
    c->heads = 24;
    c->mlp_width = 12288;
    c->text_dim = 4096;
    c->z_dim = 64;
    c->layers = 32;
    c->mlp_act = QW_MLP_GELU_TANH;
    c->adaln_shift = 1;
    c->has_bias = 1;
    c->text_causal = 0;
    c->int8_weights = 0;
}

const qw_dit_config *qw_dit_get_config(const qw_dit *d) { return d ? &d->cfg : NULL; }

/* ---------------------------------------------------------------------- */
/* weights                                                                */

static void lin_free(qw_lin *l) {
    h3_gpu_tensor_free(l->w);
    h3_gpu_tensor_free(l->scales);
    h3_gpu_tensor_free(l->bias);
    memset(l, 0, sizeof(*l));
}

/* W ~ bf16(0.02 z) from (seed, stream); int8 => quantised on device via the
 * temporary bf16 tensor tmp (large enough for n * k). */
static int lin_init(qw_dit *d, qw_lin *l, uint32_t n, uint32_t k, uint64_t seed,
                    uint64_t stream, uint64_t bstream, int int8, h3_gpu_tensor *tmp) {
    h3_gpu *g = d->gpu;
    l->n = n;
    l->k = k;
    size_t count = (size_t)n * k;
    if (int8) {
        h3_gpu_tensor *view = h3_gpu_tensor_view(tmp, 0, count);
        l->w = h3_gpu_tensor_new_i8(g, count);
        l->scales = h3_gpu_tensor_new_f32(g, n);
        int ok = view && l->w && l->scales &&
                 qw_gpu_fill_normal_bf16(g, view, 0, count, seed, stream, 0.02f, 0.0f) &&
                 h3_gpu_quantize_weight_int8(g, l->w, l->scales, view, n, k);
        h3_gpu_tensor_free(view);
        if (!ok) return 0;
    } else {
        l->w = h3_gpu_tensor_new_bf16(g, count);
        if (!l->w || !qw_gpu_fill_normal_bf16(g, l->w, 0, count, seed, stream, 0.02f, 0.0f))
            return 0;
    }
    if (d->cfg.has_bias) {
        l->bias = h3_gpu_tensor_new_bf16(g, n);
        if (!l->bias || !qw_gpu_fill_normal_bf16(g, l->bias, 0, n, seed, bstream, 0.02f, 0.0f))
            return 0;
    }
    return 1;
}

static int check_config(const qw_dit_config *c, char *error, size_t n) {
    if (!c) return set_error(error, n, "missing config");
    if (!c->heads || c->hidden != c->heads * 128)
        return set_error(error, n, "hidden %u must equal heads * 128", c->hidden);
    if (c->hidden % 256 || c->hidden > 8192)
        return set_error(error, n, "hidden %u must be a multiple of 256, <= 8192", c->hidden);
    if (!c->mlp_width || c->mlp_width % 64)
        return set_error(error, n, "mlp_width %u must be a multiple of 64", c->mlp_width);
    if (!c->text_dim || c->text_dim % 64 || c->text_dim > 8192)
        return set_error(error, n, "text_dim %u must be a multiple of 64, <= 8192", c->text_dim);
    if (!c->z_dim || c->z_dim % 64)
        return set_error(error, n, "z_dim %u must be a multiple of 64", c->z_dim);
    if (!c->layers || c->layers > 256) return set_error(error, n, "layers %u out of range", c->layers);
    if (c->mlp_act != QW_MLP_SWIGLU && c->mlp_act != QW_MLP_GELU_TANH)
        return set_error(error, n, "unknown mlp_act %d", c->mlp_act);
    return 1;
}

/* conditioning buffers (2 modulation rows) */
static int cond_buffers(qw_dit *d) {
    h3_gpu *gpu = d->gpu;
    const uint32_t H = d->cfg.hidden;
    const uint32_t nmod = slots_of(&d->cfg) * H, nout = (d->cfg.adaln_shift ? 2 : 1) * H;
    d->feat = h3_gpu_tensor_new_f32(gpu, 2 * 256);
    d->feat_bf16 = h3_gpu_tensor_new_bf16(gpu, 2 * 256);
    d->c_wide = h3_gpu_tensor_new_bf16(gpu, 2 * (size_t)H);
    d->c_silu = h3_gpu_tensor_new_bf16(gpu, 2 * (size_t)H);
    d->temb = h3_gpu_tensor_new_bf16(gpu, 2 * (size_t)H);
    d->mod_raw = h3_gpu_tensor_new_bf16(gpu, 2 * (size_t)nmod);
    d->modulation = h3_gpu_tensor_new_bf16(gpu, 2 * (size_t)nmod);
    d->norm_out_mod = h3_gpu_tensor_new_bf16(gpu, 2 * (size_t)nout);
    return d->feat && d->feat_bf16 && d->c_wide && d->c_silu && d->temb && d->mod_raw &&
           d->modulation && d->norm_out_mod;
}

qw_dit *qw_dit_create_random(h3_gpu *gpu, const qw_dit_config *cfg, uint64_t seed,
                             char *error, size_t error_size) {
    if (!gpu) {
        set_error(error, error_size, "no gpu");
        return NULL;
    }
    if (!check_config(cfg, error, error_size)) return NULL;
    qw_dit *d = calloc(1, sizeof(*d));
    if (!d) {
        set_error(error, error_size, "out of memory");
        return NULL;
    }
    d->gpu = gpu;
    d->cfg = *cfg;
    d->profile = env_on("QWEN_BLOCK_PROFILE");
    const uint32_t H = cfg->hidden, F = cfg->mlp_width;
    const uint32_t f1 = cfg->mlp_act == QW_MLP_SWIGLU ? 2 * F : F;
    const uint32_t nmod = slots_of(cfg) * H, nout = (cfg->adaln_shift ? 2 : 1) * H;
    size_t tmp_n = (size_t)f1 * H;
    if ((size_t)F * H > tmp_n) tmp_n = (size_t)F * H;
    if ((size_t)3 * H * H > tmp_n) tmp_n = (size_t)3 * H * H;
    h3_gpu_tensor *tmp = cfg->int8_weights ? h3_gpu_tensor_new_bf16(gpu, tmp_n) : NULL;
    d->layer = calloc(cfg->layers, sizeof(qw_layer));
    int ok = d->layer && (!cfg->int8_weights || tmp);
    /* global projections stay bf16, as the reference keeps them */
    ok = ok && lin_init(d, &d->img_in, H, cfg->z_dim, seed, QW_W_IMG_IN, QW_W_IMG_IN_B, 0, NULL);
    d->txt_norm = ok ? h3_gpu_tensor_new_bf16(gpu, cfg->text_dim) : NULL;
    ok = ok && d->txt_norm &&
         qw_gpu_fill_normal_bf16(gpu, d->txt_norm, 0, cfg->text_dim, seed, QW_W_TXT_NORM, 0.02f,
                                 0.0f);
    ok = ok && lin_init(d, &d->txt_in1, H, cfg->text_dim, seed, QW_W_TXT_IN1, QW_W_TXT_IN1_B, 0, NULL);
    ok = ok && lin_init(d, &d->txt_in2, H, H, seed, QW_W_TXT_IN2, QW_W_TXT_IN2_B, 0, NULL);
    ok = ok && lin_init(d, &d->time_l1, H, 256, seed, QW_W_TIME_L1, QW_W_TIME_L1_B, 0, NULL);
    ok = ok && lin_init(d, &d->time_l2, H, H, seed, QW_W_TIME_L2, QW_W_TIME_L2_B, 0, NULL);
    ok = ok && lin_init(d, &d->mod, nmod, H, seed, QW_W_MOD, QW_W_MOD_B, 0, NULL);
    ok = ok && lin_init(d, &d->norm_out, nout, H, seed, QW_W_NORM_OUT, QW_W_NORM_OUT_B, 0, NULL);
    ok = ok && lin_init(d, &d->proj_out, cfg->z_dim, H, seed, QW_W_PROJ_OUT, QW_W_PROJ_OUT_B, 0, NULL);
    for (uint32_t l = 0; ok && l < cfg->layers; l++) {
        qw_layer *L = &d->layer[l];
        int q8 = cfg->int8_weights;
        ok = lin_init(d, &L->qkv, 3 * H, H, seed, QW_LAYER_STREAM(l, QW_L_QKV),
                      QW_LAYER_STREAM(l, QW_L_QKV_B), q8, tmp) &&
             lin_init(d, &L->out, H, H, seed, QW_LAYER_STREAM(l, QW_L_OUT),
                      QW_LAYER_STREAM(l, QW_L_OUT_B), q8, tmp) &&
             lin_init(d, &L->fc1, f1, H, seed, QW_LAYER_STREAM(l, QW_L_FC1),
                      QW_LAYER_STREAM(l, QW_L_FC1_B), q8, tmp) &&
             lin_init(d, &L->fc2, H, F, seed, QW_LAYER_STREAM(l, QW_L_FC2),
                      QW_LAYER_STREAM(l, QW_L_FC2_B), q8, tmp);
        L->norm_q = ok ? h3_gpu_tensor_new_bf16(gpu, 128) : NULL;
        L->norm_k = ok ? h3_gpu_tensor_new_bf16(gpu, 128) : NULL;
        ok = ok && L->norm_q && L->norm_k &&
             qw_gpu_fill_normal_bf16(gpu, L->norm_q, 0, 128, seed, QW_LAYER_STREAM(l, QW_L_NORM_Q),
                                     0.02f, 1.0f) &&
             qw_gpu_fill_normal_bf16(gpu, L->norm_k, 0, 128, seed, QW_LAYER_STREAM(l, QW_L_NORM_K),
                                     0.02f, 1.0f);
    }
    ok = ok && cond_buffers(d) && h3_gpu_submit(gpu);
    h3_gpu_tensor_free(tmp);
    if (!ok) {
        set_error(error, error_size, "qw_dit_create_random failed: %s", h3_gpu_error(gpu));
        qw_dit_free(d);
        return NULL;
    }
    return d;
}

/* ---------------------------------------------------------------------- */
/* checkpoint loading (qwen_dit.m:235-371)                                */

/* A linear whose weight is the row-wise concatenation of named [rows_i, k]
 * bf16 tensors; int8 => read into the temporary bf16 tensor and quantised
 * on device (the same path as the seeded weights). */
static int lin_load(qw_dit *d, h3_weight_store *st, qw_lin *l, uint32_t k, const char *const *names,
                    const uint32_t *rows, int parts, int int8, h3_gpu_tensor *tmp, char *error,
                    size_t error_size) {
    h3_gpu *g = d->gpu;
    uint32_t n = 0;
    for (int i = 0; i < parts; i++) n += rows[i];
    l->n = n;
    l->k = k;
    const size_t count = (size_t)n * k;
    h3_gpu_tensor *dst = int8 ? h3_gpu_tensor_view(tmp, 0, count) : h3_gpu_tensor_new_bf16(g, count);
    if (!dst) return set_error(error, error_size, "%s: allocation failed", names[0]);
    int ok = 1;
    size_t off = 0;
    for (int i = 0; ok && i < parts; i++) {
        const uint64_t shape[2] = {rows[i], k};
        ok = h3_weight_read_bf16_into(st, names[i], 2, shape, dst, off, error, error_size);
        off += (size_t)rows[i] * k;
    }
    if (ok && int8) {
        l->w = h3_gpu_tensor_new_i8(g, count);
        l->scales = h3_gpu_tensor_new_f32(g, n);
        ok = l->w && l->scales && h3_gpu_quantize_weight_int8(g, l->w, l->scales, dst, n, k);
        if (!ok) set_error(error, error_size, "%s: int8 quantisation failed: %s", names[0],
                           h3_gpu_error(g));
        h3_gpu_tensor_free(dst);
    } else if (ok) {
        l->w = dst;
    } else {
        h3_gpu_tensor_free(dst);
    }
    return ok;
}

static int lin_load1(qw_dit *d, h3_weight_store *st, qw_lin *l, const char *name, uint32_t n,
                     uint32_t k, char *error, size_t error_size) {
    const char *names[1] = {name};
    const uint32_t rows[1] = {n};
    return lin_load(d, st, l, k, names, rows, 1, 0, NULL, error, error_size);
}

static h3_gpu_tensor *vec_load(h3_weight_store *st, h3_gpu *g, const char *name, uint32_t n,
                               char *error, size_t error_size) {
    const uint64_t shape[1] = {n};
    return h3_weight_load_bf16(st, g, name, 1, shape, error, error_size);
}

qw_dit *qw_dit_load(h3_gpu *gpu, const char *model_dir, const qw_dit_config *cfg, char *error,
                    size_t error_size) {
    if (!gpu || !model_dir) {
        set_error(error, error_size, "qw_dit_load: missing gpu or model directory");
        return NULL;
    }
    if (!check_config(cfg, error, error_size)) return NULL;
    if (cfg->mlp_act != QW_MLP_SWIGLU || cfg->adaln_shift || cfg->has_bias) {
        set_error(error, error_size,
                  "qw_dit_load: checkpoints use the reference architecture (SwiGLU MLP, "
                  "scale/gate modulation, no biases)");
        return NULL;
    }
    char dir[4096];
    snprintf(dir, sizeof(dir), "%s/transformer", model_dir);
    h3_weight_store *st = h3_weight_store_open(dir, error, error_size);
    if (!st) return NULL;
    qw_dit *d = calloc(1, sizeof(*d));
    if (!d) {
        h3_weight_store_free(st);
        set_error(error, error_size, "out of memory");
        return NULL;
    }
    d->gpu = gpu;
    d->cfg = *cfg;
    d->profile = env_on("QWEN_BLOCK_PROFILE");
    const uint32_t H = cfg->hidden, F = cfg->mlp_width, T = cfg->text_dim, Z = cfg->z_dim;
    const int q8 = cfg->int8_weights;
    h3_gpu_tensor *tmp = q8 ? h3_gpu_tensor_new_bf16(gpu, (size_t)2 * F * H > (size_t)3 * H * H
                                                              ? (size_t)2 * F * H
                                                              : (size_t)3 * H * H)
                            : NULL;
    d->layer = calloc(cfg->layers, sizeof(qw_layer));
    int ok = d->layer && (!q8 || tmp);
    if (!ok) set_error(error, error_size, "out of memory");
    ok = ok && lin_load1(d, st, &d->img_in, "img_in.weight", H, Z, error, error_size);
    ok = ok && (d->txt_norm = vec_load(st, gpu, "txt_in.text_norm.weight", T, error, error_size));
    ok = ok && lin_load1(d, st, &d->txt_in1, "txt_in.in_layer.weight", H, T, error, error_size);
    ok = ok && lin_load1(d, st, &d->txt_in2, "txt_in.out_layer.weight", H, H, error, error_size);
    ok = ok && lin_load1(d, st, &d->time_l1, "time_text_embed.timestep_embedder.linear_1.weight",
                         H, 256, error, error_size);
    ok = ok && lin_load1(d, st, &d->time_l2, "time_text_embed.timestep_embedder.linear_2.weight",
                         H, H, error, error_size);
    ok = ok && lin_load1(d, st, &d->mod, "modulation.1.weight", 4 * H, H, error, error_size);
    ok = ok && lin_load1(d, st, &d->norm_out, "norm_out.linear.weight", H, H, error, error_size);
    ok = ok && lin_load1(d, st, &d->proj_out, "proj_out.weight", Z, H, error, error_size);
    for (uint32_t l = 0; ok && l < cfg->layers; l++) {
        qw_layer *L = &d->layer[l];
        char q[160], k[160], v[160], o[160], nq[160], nk[160], gt[160], pj[160], ot[160];
        snprintf(q, sizeof(q), "transformer_blocks.%u.attn.to_q.weight", l);
        snprintf(k, sizeof(k), "transformer_blocks.%u.attn.to_k.weight", l);
        snprintf(v, sizeof(v), "transformer_blocks.%u.attn.to_v.weight", l);
        snprintf(o, sizeof(o), "transformer_blocks.%u.attn.to_out.0.weight", l);
        snprintf(nq, sizeof(nq), "transformer_blocks.%u.attn.norm_q.weight", l);
        snprintf(nk, sizeof(nk), "transformer_blocks.%u.attn.norm_k.weight", l);
        snprintf(gt, sizeof(gt), "transformer_blocks.%u.img_mlp.gate_layer.weight", l);
        snprintf(pj, sizeof(pj), "transformer_blocks.%u.img_mlp.proj.weight", l);
        snprintf(ot, sizeof(ot), "transformer_blocks.%u.img_mlp.out.weight", l);
        /* fused [q; k; v] and [gate; proj] rows, as the kernels take them */
        const char *qkv[3] = {q, k, v}, *fc1[2] = {gt, pj}, *out[1] = {o}, *fc2[1] = {ot};
        const uint32_t rq[3] = {H, H, H}, rf[2] = {F, F}, rh[1] = {H};
        ok = lin_load(d, st, &L->qkv, H, qkv, rq, 3, q8, tmp, error, error_size) &&
             lin_load(d, st, &L->out, H, out, rh, 1, q8, tmp, error, error_size) &&
             lin_load(d, st, &L->fc1, H, fc1, rf, 2, q8, tmp, error, error_size) &&
             lin_load(d, st, &L->fc2, F, fc2, rh, 1, q8, tmp, error, error_size) &&
             (L->norm_q = vec_load(st, gpu, nq, 128, error, error_size)) &&
             (L->norm_k = vec_load(st, gpu, nk, 128, error, error_size));
    }
    if (ok && !cond_buffers(d)) ok = set_error(error, error_size, "out of memory");
    if (ok && !h3_gpu_submit(gpu))
        ok = set_error(error, error_size, "qw_dit_load: %s", h3_gpu_error(gpu));
    h3_gpu_tensor_free(tmp);
    h3_weight_store_free(st);
    if (!ok) {
        qw_dit_free(d);
        return NULL;
    }
    return d;
}

qw_dit *qw_dit_create(h3_gpu *gpu, const char *model_dir, int layers, char *error,
                      size_t error_size) {
    qw_dit_config cfg;
    qw_dit_config_reference(&cfg);
    if (layers <= 0 || layers > 256) {
        set_error(error, error_size, "qw_dit_create: layers %d out of range", layers);
        return NULL;
    }
    cfg.layers = (uint32_t)layers;
    return qw_dit_load(gpu, model_dir, &cfg, error, error_size);
}

/* ---------------------------------------------------------------------- */
/* LoRA (qwen_dit.m:535-1010)                                              */

/* The adapter targets of block weight j: module name, first fused row,
 * rows (keys: transformer_blocks.N.<module>.lora_{A,B}.default.weight). */
typedef struct {
    const char *module;
    uint32_t row0, rows;
} lora_target;

static int lora_targets(const qw_dit *d, int j, lora_target *t, uint32_t *cols) {
    const uint32_t H = d->cfg.hidden, F = d->cfg.mlp_width;
    switch (j) {
    case 0:
        t[0] = (lora_target){"attn.to_q", 0, H};
        t[1] = (lora_target){"attn.to_k", H, H};
        t[2] = (lora_target){"attn.to_v", 2 * H, H};
        *cols = H;
        return 3;
    case 1:
        t[0] = (lora_target){"attn.to_out.0", 0, H};
        *cols = H;
        return 1;
    case 2:
        t[0] = (lora_target){"img_mlp.gate_layer", 0, F};
        t[1] = (lora_target){"img_mlp.proj", F, F};
        *cols = H;
        return 2;
    default:
        t[0] = (lora_target){"img_mlp.out", 0, H};
        *cols = F;
        return 1;
    }
}

static qw_lin *layer_lin(qw_layer *L, int j) {
    return j == 0 ? &L->qkv : j == 1 ? &L->out : j == 2 ? &L->fc1 : &L->fc2;
}

/* every adapter dropped, base weights back in the layers, fused copies and
 * ti2i caches (made with the old weights) freed */
static void qkv_views_free(qw_dit *d);

static void lora_reset(qw_dit *d) {
    qkv_views_free(d);
    if (d->lora_base) {
        for (uint32_t l = 0; l < d->cfg.layers; l++)
            for (int j = 0; j < 4; j++) {
                qw_lin *w = layer_lin(&d->layer[l], j);
                h3_gpu_tensor *base = d->lora_base[4 * l + j];
                if (base && w->w != base) {
                    h3_gpu_tensor_free(w->w);
                    w->w = base;
                }
            }
        free(d->lora_base);
        d->lora_base = NULL;
    }
    for (int i = 0; i < d->n_lora; i++) {
        free(d->lora[i].path);
        h3_st_free_header(&d->lora[i].header);
    }
    d->n_lora = 0;
    qw_dit_ti2i_cache_clear(d);
}

/* A bf16 [rows, cols] matrix of an adapter: 1 read into a new device
 * tensor, 0 absent (partial adapters are allowed), -1 broken */
static int lora_matrix(qw_dit *d, const h3_st_header *h, const char *key, uint32_t rows,
                       uint32_t cols, h3_gpu_tensor **out, char *error, size_t error_size) {
    *out = NULL;
    const h3_st_tensor *t = h3_st_find(h, key);
    if (!t) return 0;
    if (t->dtype != H3_DTYPE_BF16 || t->ndim != 2 || t->shape[0] != rows || t->shape[1] != cols) {
        set_error(error, error_size, "lora tensor %s: expected bf16 [%u x %u]", key, rows, cols);
        return -1;
    }
    const size_t n = (size_t)rows * cols;
    uint16_t *host = malloc(sizeof(uint16_t) * (n ? n : 1));
    *out = h3_gpu_tensor_new_bf16(d->gpu, n);
    int ok = host && *out && h3_st_read_data(h, t, host, sizeof(uint16_t) * n, error, error_size) &&
             h3_gpu_tensor_write_bf16(*out, host, n);
    free(host);
    if (!ok) {
        h3_gpu_tensor_free(*out);
        *out = NULL;
        if (error && !*error) set_error(error, error_size, "lora tensor %s: read failed", key);
        return -1;
    }
    return 1;
}

/* Every fused weight rebuilt from the kept base in one pass (so the order
 * of apply / remove / scale changes does not matter and nothing rounds
 * twice). On failure the adapter state is reset to none. */
static int lora_rebuild(qw_dit *d, char *error, size_t error_size) {
    qkv_views_free(d);
    h3_gpu *g = d->gpu;
    int ok = 1;
    if (!d->lora_base) {
        d->lora_base = calloc((size_t)4 * d->cfg.layers, sizeof(h3_gpu_tensor *));
        ok = d->lora_base != NULL;
        for (uint32_t l = 0; ok && l < d->cfg.layers; l++)
            for (int j = 0; ok && j < 4; j++) {
                qw_lin *w = layer_lin(&d->layer[l], j);
                h3_gpu_tensor *fused = h3_gpu_tensor_new_bf16(g, (size_t)w->n * w->k);
                ok = fused != NULL;
                if (ok) {
                    d->lora_base[4 * l + j] = w->w;
                    w->w = fused;
                }
            }
        if (!ok) set_error(error, error_size, "lora: out of memory for the fused weights");
    }
    for (uint32_t l = 0; ok && l < d->cfg.layers; l++)
        for (int j = 0; ok && j < 4; j++) {
            lora_target tg[3];
            uint32_t cols;
            const int nt = lora_targets(d, j, tg, &cols);
            qw_lora_term_desc terms[QW_GPU_LORA_MAX_TERMS];
            h3_gpu_tensor *held[2 * QW_GPU_LORA_MAX_TERMS];
            uint32_t n = 0, nh = 0;
            for (int a = 0; ok && a < d->n_lora; a++)
                for (int t = 0; ok && t < nt; t++) {
                    char ka[192], kb[192];
                    snprintf(ka, sizeof(ka), "transformer_blocks.%u.%s.lora_A.default.weight", l,
                             tg[t].module);
                    snprintf(kb, sizeof(kb), "transformer_blocks.%u.%s.lora_B.default.weight", l,
                             tg[t].module);
                    h3_gpu_tensor *A, *B;
                    const int ra = lora_matrix(d, &d->lora[a].header, ka, d->lora[a].rank, cols,
                                               &A, error, error_size);
                    if (ra <= 0) {
                        ok = ra == 0;
                        continue;
                    }
                    held[nh++] = A;
                    const int rb = lora_matrix(d, &d->lora[a].header, kb, tg[t].rows,
                                               d->lora[a].rank, &B, error, error_size);
                    if (rb <= 0) {
                        ok = rb == 0;
                        continue;
                    }
                    held[nh++] = B;
                    terms[n++] = (qw_lora_term_desc){A, B, tg[t].row0, tg[t].rows, d->lora[a].rank,
                                                     d->lora[a].scale};
                }
            qw_lin *w = layer_lin(&d->layer[l], j);
            ok = ok && qw_gpu_lora_fuse_bf16(g, w->w, d->lora_base[4 * l + j], w->n, w->k, terms, n);
            if (!ok && error && !*error) set_error(error, error_size, "lora: %s", h3_gpu_error(g));
            for (uint32_t i = 0; i < nh; i++) h3_gpu_tensor_free(held[i]); /* waits for the fuse */
        }
    qw_dit_ti2i_cache_clear(d); /* cached K/V came from the previous weights */
    if (!ok) lora_reset(d);
    return ok;
}

/* header readable, a rank (first bf16 2-D lora_A: its rows), and at least
 * one key that matches a block target */
static int lora_open(const qw_dit *d, const char *path, h3_st_header *h, uint32_t *rank,
                     char *error, size_t error_size) {
    if (!h3_st_read_header(path, h, error, error_size)) return 0;
    *rank = 0;
    for (size_t i = 0; i < h->tensor_count && !*rank; i++)
        if (h->tensors[i].dtype == H3_DTYPE_BF16 && h->tensors[i].ndim == 2 &&
            strstr(h->tensors[i].name, ".lora_A.default.weight"))
            *rank = (uint32_t)h->tensors[i].shape[0];
    if (!*rank || *rank > QW_GPU_LORA_MAX_RANK) {
        h3_st_free_header(h);
        return set_error(error, error_size, "lora file carries no bf16 lora_A matrices of rank "
                         "1..%d: %s", QW_GPU_LORA_MAX_RANK, path);
    }
    for (uint32_t l = 0; l < d->cfg.layers; l++)
        for (int j = 0; j < 4; j++) {
            lora_target tg[3];
            uint32_t cols;
            const int nt = lora_targets(d, j, tg, &cols);
            for (int t = 0; t < nt; t++) {
                char key[192];
                snprintf(key, sizeof(key), "transformer_blocks.%u.%s.lora_A.default.weight", l,
                         tg[t].module);
                if (h3_st_find(h, key)) return 1;
            }
        }
    h3_st_free_header(h);
    return set_error(error, error_size, "lora matched no checkpoint tensors: %s", path);
}

static int lora_supported(const qw_dit *d, char *error, size_t error_size) {
    if (d->cfg.int8_weights)
        return set_error(error, error_size, "lora: the block weights are int8; adapters fuse into "
                         "bf16 weights");
    if (d->cfg.mlp_act != QW_MLP_SWIGLU || d->cfg.has_bias)
        return set_error(error, error_size, "lora: adapters target the reference architecture "
                         "(SwiGLU MLP, no biases)");
    return 1;
}

int qw_dit_apply_lora(qw_dit *d, const char *path, float scale, char *error, size_t error_size) {
    if (error && error_size) error[0] = '\0';
    if (!d) return set_error(error, error_size, "no dit");
    if (!path || !*path) return set_error(error, error_size, "lora path is required");
    if (!lora_supported(d, error, error_size)) return 0;
    for (int i = 0; i < d->n_lora; i++)
        if (strcmp(d->lora[i].path, path) == 0) { /* known adapter: new scale */
            d->lora[i].scale = scale;
            return lora_rebuild(d, error, error_size);
        }
    if (d->n_lora >= QW_DIT_MAX_LORA)
        return set_error(error, error_size, "lora stack is full (%d adapters)", QW_DIT_MAX_LORA);
    h3_st_header h;
    uint32_t rank;
    if (!lora_open(d, path, &h, &rank, error, error_size)) return 0;
    char *copy = strdup(path);
    if (!copy) {
        h3_st_free_header(&h);
        return set_error(error, error_size, "out of memory");
    }
    d->lora[d->n_lora] = (struct qw_lora){copy, scale, rank, h};
    d->n_lora++;
    return lora_rebuild(d, error, error_size);
}

int qw_dit_switch_lora(qw_dit *d, const char *path, float scale, char *error,
                       size_t error_size) {
    if (error && error_size) error[0] = '\0';
    if (!d || !path || !*path) return set_error(error, error_size, "lora path is required");
    if (d->n_lora != 1)
        return set_error(error, error_size, "switch requires exactly one active adapter");
    if (strcmp(d->lora[0].path, path) == 0) return qw_dit_apply_lora(d, path, scale, error, error_size);
    h3_st_header h;
    uint32_t rank;
    if (!lora_open(d, path, &h, &rank, error, error_size)) return 0; /* old one stays */
    char *copy = strdup(path);
    if (!copy) {
        h3_st_free_header(&h);
        return set_error(error, error_size, "out of memory");
    }
    free(d->lora[0].path);
    h3_st_free_header(&d->lora[0].header);
    d->lora[0] = (struct qw_lora){copy, scale, rank, h};
    return lora_rebuild(d, error, error_size);
}

int qw_dit_remove_lora(qw_dit *d, const char *path, char *error, size_t error_size) {
    if (!d) return set_error(error, error_size, "no dit");
    if (!path || !*path) return qw_dit_clear_lora(d, error, error_size);
    for (int i = 0; i < d->n_lora; i++)
        if (strcmp(d->lora[i].path, path) == 0) {
            free(d->lora[i].path);
            h3_st_free_header(&d->lora[i].header);
            memmove(&d->lora[i], &d->lora[i + 1], sizeof(d->lora[0]) * (size_t)(d->n_lora - i - 1));
            d->n_lora--;
            if (!d->n_lora) {
                lora_reset(d);
                return 1;
            }
            return lora_rebuild(d, error, error_size);
        }
    return 1; /* unknown path: nothing to remove */
}

int qw_dit_clear_lora(qw_dit *d, char *error, size_t error_size) {
    if (!d) return set_error(error, error_size, "no dit");
    lora_reset(d);
    return 1;
}

int qw_dit_lora_count(const qw_dit *d) { return d ? d->n_lora : 0; }

const char *qw_dit_lora_path_at(const qw_dit *d, int index) {
    return d && index >= 0 && index < d->n_lora ? d->lora[index].path : NULL;
}

float qw_dit_lora_scale_at(const qw_dit *d, int index) {
    return d && index >= 0 && index < d->n_lora ? d->lora[index].scale : 0.0f;
}

void qw_dit_free(qw_dit *d) {
    if (!d) return;
    lora_reset(d);
    if (d->layer)
        for (uint32_t l = 0; l < d->cfg.layers; l++) {
            lin_free(&d->layer[l].qkv);
            lin_free(&d->layer[l].out);
            lin_free(&d->layer[l].fc1);
            lin_free(&d->layer[l].fc2);
            h3_gpu_tensor_free(d->layer[l].norm_q);
            h3_gpu_tensor_free(d->layer[l].norm_k);
        }
    free(d->layer);
    qkv_views_free(d);
    lin_free(&d->img_in);
    lin_free(&d->txt_in1);
    lin_free(&d->txt_in2);
    lin_free(&d->time_l1);
    lin_free(&d->time_l2);
    lin_free(&d->mod);
    lin_free(&d->norm_out);
    lin_free(&d->proj_out);
    h3_gpu_tensor *t[] = {d->txt_norm, d->ws_mod, d->ws_qkv, d->ws_attn, d->ws_wide, d->ws_act,
                          d->ws_tnorm, d->ws_twide, d->feat, d->feat_bf16, d->c_wide, d->c_silu,
                          d->temb, d->mod_raw, d->modulation, d->norm_out_mod, d->joint,
                          d->row_map};
    for (size_t i = 0; i < sizeof(t) / sizeof(t[0]); i++) h3_gpu_tensor_free(t[i]);
    qw_dit_ti2i_cache_clear(d);
    free(d);
}

/* View of rows [part H, (part + 1) H) of the fused qkv weight (scales: 0)
 * or of its row scales (scales: 1), rebuilt if the live tensor changed. */
static const h3_gpu_tensor *qkv_part(qw_dit *d, int block, int part, int scales) {
    const uint32_t H = d->cfg.hidden;
    const qw_layer *L = &d->layer[block];
    const h3_gpu_tensor *src = scales ? L->qkv.scales : L->qkv.w;
    if (!src) return NULL;
    if (!d->qkv_views) {
        d->qkv_views = calloc(d->cfg.layers, sizeof(*d->qkv_views));
        if (!d->qkv_views) return NULL;
    }
    struct qw_qkv_views *v = &d->qkv_views[block];
    const h3_gpu_tensor **have = scales ? &v->src_s : &v->src_w;
    h3_gpu_tensor **views = scales ? v->s : v->w;
    if (*have != src) {
        for (int i = 0; i < 3; i++) {
            h3_gpu_tensor_free(views[i]);
            views[i] = NULL;
        }
        *have = src;
    }
    if (!views[part]) {
        const size_t per = scales ? H : (size_t)H * L->qkv.k;
        views[part] = h3_gpu_tensor_view(src, per * (size_t)part, per);
    }
    return views[part];
}

static void qkv_views_free(qw_dit *d) {
    if (!d->qkv_views) return;
    for (uint32_t l = 0; l < d->cfg.layers; l++)
        for (int i = 0; i < 3; i++) {
            h3_gpu_tensor_free(d->qkv_views[l].w[i]);
            h3_gpu_tensor_free(d->qkv_views[l].s[i]);
        }
    free(d->qkv_views);
    d->qkv_views = NULL;
}

/* Fields as reference qwen_dit.h:84-86: 0 = to_q, 1 = to_k, 2 = to_v (row
 * views of the fused [3H, H] weight), 3 = to_out, 4 = fc1, 5 = fc2. The
 * views belong to the model (valid until the next LoRA change or
 * qw_dit_free); the caller frees nothing. */
const h3_gpu_tensor *qw_dit_block_tensor(const qw_dit *d, int block, int field) {
    if (!d || block < 0 || (uint32_t)block >= d->cfg.layers) return NULL;
    const qw_layer *L = &d->layer[block];
    switch (field) {
    case 0: case 1: case 2: return qkv_part((qw_dit *)d, block, field, 0);
    case 3: return L->out.w;
    case 4: return L->fc1.w;
    case 5: return L->fc2.w;
    default: return NULL;
    }
}

const h3_gpu_tensor *qw_dit_block_scales(const qw_dit *d, int block, int field) {
    if (!d || block < 0 || (uint32_t)block >= d->cfg.layers) return NULL;
    const qw_layer *L = &d->layer[block];
    switch (field) {
    case 0: case 1: case 2: return qkv_part((qw_dit *)d, block, field, 1);
    case 3: return L->out.scales;
    case 4: return L->fc1.scales;
    case 5: return L->fc2.scales;
    default: return NULL;
    }
}

/* ---------------------------------------------------------------------- */
/* helpers                                                                */

static int linear(qw_dit *d, const qw_lin *l, h3_gpu_tensor *out, size_t out_off, uint32_t ldc,
                  const h3_gpu_tensor *in, size_t in_off, uint32_t lda, uint32_t rows, int epi,
                  const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, uint32_t slots,
                  uint32_t gate_slot) {
    qw_linear_desc desc;
    memset(&desc, 0, sizeof(desc));
    desc.out = out;
    desc.out_offset = out_off;
    desc.ldc = ldc;
    desc.in = in;
    desc.in_offset = in_off;
    desc.lda = lda;
    desc.weight = l->w;
    desc.wscale = l->scales;
    desc.bias = l->bias;
    desc.rows = rows;
    desc.k = l->k;
    desc.cols = l->n;
    desc.epilogue = epi;
    desc.modulation = modulation;
    desc.row_map = row_map;
    desc.slots = slots;
    desc.gate_slot = gate_slot;
    return qw_gpu_linear(d->gpu, &desc);
}

static int plain(qw_dit *d, const qw_lin *l, h3_gpu_tensor *out, const h3_gpu_tensor *in,
                 uint32_t rows, int epi) {
    return linear(d, l, out, 0, l->n, in, 0, l->k, rows, epi, NULL, NULL, 0, 0);
}

static void free_ws(qw_dit *d) {
    h3_gpu_tensor_free(d->ws_mod);
    h3_gpu_tensor_free(d->ws_qkv);
    h3_gpu_tensor_free(d->ws_attn);
    h3_gpu_tensor_free(d->ws_wide);
    h3_gpu_tensor_free(d->ws_act);
    d->ws_mod = d->ws_qkv = d->ws_attn = d->ws_wide = d->ws_act = NULL;
    d->ws_rows = 0;
}

/* Block workspaces for `rows` rows (grow-only). */
static int ensure_ws(qw_dit *d, uint32_t rows) {
    if (d->ws_rows >= rows) return 1;
    free_ws(d);
    h3_gpu *g = d->gpu;
    const size_t H = d->cfg.hidden, F = d->cfg.mlp_width;
    const int swiglu = d->cfg.mlp_act == QW_MLP_SWIGLU;
    d->ws_mod = h3_gpu_tensor_new_bf16(g, rows * H);
    d->ws_qkv = h3_gpu_tensor_new_bf16(g, rows * 3 * H);
    d->ws_attn = h3_gpu_tensor_new_bf16(g, rows * H);
    d->ws_wide = h3_gpu_tensor_new_bf16(g, rows * (swiglu ? 2 * F : F));
    d->ws_act = swiglu ? h3_gpu_tensor_new_bf16(g, rows * F) : NULL;
    if (!d->ws_mod || !d->ws_qkv || !d->ws_attn || !d->ws_wide || (swiglu && !d->ws_act)) {
        free_ws(d);
        return 0;
    }
    d->ws_rows = rows;
    return 1;
}

static int ensure_text_ws(qw_dit *d, uint32_t rows) {
    if (d->ws_text_rows >= rows) return 1;
    h3_gpu_tensor_free(d->ws_tnorm);
    h3_gpu_tensor_free(d->ws_twide);
    d->ws_tnorm = h3_gpu_tensor_new_bf16(d->gpu, (size_t)rows * d->cfg.text_dim);
    d->ws_twide = h3_gpu_tensor_new_bf16(d->gpu, (size_t)rows * d->cfg.hidden);
    d->ws_text_rows = d->ws_tnorm && d->ws_twide ? rows : 0;
    return d->ws_text_rows != 0;
}

static void prof_begin(qw_dit *d) {
    if (d->profile) h3_gpu_timer_begin(d->gpu);
}

static void prof_end(qw_dit *d, int stage) {
    if (d->profile) {
        double ms = h3_gpu_timer_end(d->gpu);
        if (ms > 0) d->prof_ms[stage] += ms;
    }
}

static void span_b(qw_dit *d, int tag) {
    if (d->spans) qw_gpu_span_begin(d->gpu, tag);
}

static void span_e(qw_dit *d) {
    if (d->spans) qw_gpu_span_end(d->gpu);
}

int qw_dit_set_spans(qw_dit *d, int on) {
    if (!d) return 0;
    d->spans = on != 0;
    return 1;
}

int qw_dit_block_profile(const qw_dit *d, double *ms, int max_stages) {
    if (!d || !ms) return 0;
    int n = max_stages < P_COUNT ? max_stages : P_COUNT;
    for (int i = 0; i < n; i++) ms[i] = d->prof_ms[i];
    return n;
}

/* ---------------------------------------------------------------------- */
/* embed / conditioning                                                   */

/* Text rows of one batch entry -> joint rows [joint_off, +text_rows):
 * rms_norm_one -> txt_in1 (GELU epilogue) -> txt_in2 (qwen_dit.m:1031-1062). */
static int embed_one(qw_dit *d, const h3_gpu_tensor *text_in, size_t text_off,
                     uint32_t text_rows, const h3_gpu_tensor *latents, size_t lat_off,
                     uint32_t image_rows, h3_gpu_tensor *joint, size_t joint_off) {
    h3_gpu *g = d->gpu;
    const uint32_t H = d->cfg.hidden;
    if (text_rows) {
        if (!ensure_text_ws(d, text_rows)) return 0;
        h3_gpu_tensor *tv = h3_gpu_tensor_view(text_in, text_off, (size_t)text_rows * d->cfg.text_dim);
        int ok = tv && qw_gpu_rms_norm_one_bf16(g, d->ws_tnorm, tv, d->txt_norm, text_rows,
                                                d->cfg.text_dim, 1e-6f);
        h3_gpu_tensor_free(tv);
        ok = ok && plain(d, &d->txt_in1, d->ws_twide, d->ws_tnorm, text_rows, QW_LINEAR_GELU) &&
             linear(d, &d->txt_in2, joint, joint_off, H, d->ws_twide, 0, H, text_rows,
                    QW_LINEAR_STORE, NULL, NULL, 0, 0);
        if (!ok) return 0;
    }
    if (image_rows)
        return linear(d, &d->img_in, joint, joint_off + (size_t)text_rows * H, H, latents, lat_off,
                      d->cfg.z_dim, image_rows, QW_LINEAR_STORE, NULL, NULL, 0, 0);
    return 1;
}

int qw_dit_embed(qw_dit *d, const h3_gpu_tensor *text_in, uint32_t text_rows,
                 const h3_gpu_tensor *latents, uint32_t image_rows, h3_gpu_tensor *joint,
                 char *error, size_t error_size) {
    if (!d) return set_error(error, error_size, "no dit");
    if (h3_gpu_tensor_elements(joint) < (size_t)(text_rows + image_rows) * d->cfg.hidden)
        return set_error(error, error_size, "joint tensor too small");
    if (text_rows && (!text_in || h3_gpu_tensor_elements(text_in) < (size_t)text_rows * d->cfg.text_dim))
        return set_error(error, error_size, "text_in too small");
    if (image_rows && (!latents || h3_gpu_tensor_elements(latents) < (size_t)image_rows * d->cfg.z_dim))
        return set_error(error, error_size, "latents too small");
    if (!embed_one(d, text_in, 0, text_rows, latents, 0, image_rows, joint, 0))
        return set_error(error, error_size, "embed failed: %s", h3_gpu_error(d->gpu));
    return 1;
}

void qw_dit_timestep_features(const float *row_sigmas, size_t count, float *features) {
    /* qwen_dit.m:1085-1096: [cos(1000 s f_i) | sin(1000 s f_i)],
     * f_i = 10000^(-i/128), computed in double, stored fp32. */
    for (size_t r = 0; r < count; r++) {
        const double t = (double)row_sigmas[r] * 1000.0;
        for (int i = 0; i < 128; i++) {
            const double arg = t * pow(10000.0, -(double)i / 128.0);
            features[r * 256 + i] = (float)cos(arg);
            features[r * 256 + 128 + i] = (float)sin(arg);
        }
    }
}

int qw_dit_conditioning(qw_dit *d, const h3_gpu_tensor *features, uint32_t mod_rows,
                        h3_gpu_tensor *temb, h3_gpu_tensor *modulation,
                        h3_gpu_tensor *norm_out_scale, char *error, size_t error_size) {
    /* qwen_dit.m:1098-1192 */
    if (!d) return set_error(error, error_size, "no dit");
    h3_gpu *g = d->gpu;
    const uint32_t H = d->cfg.hidden, S = slots_of(&d->cfg);
    if (mod_rows == 0 || mod_rows > 2) return set_error(error, error_size, "mod_rows must be 1 or 2");
    if (h3_gpu_tensor_elements(features) < (size_t)mod_rows * 256 ||
        h3_gpu_tensor_elements(temb) < (size_t)mod_rows * H ||
        h3_gpu_tensor_elements(modulation) < (size_t)mod_rows * S * H ||
        h3_gpu_tensor_elements(norm_out_scale) < (size_t)mod_rows * d->norm_out.n)
        return set_error(error, error_size, "conditioning tensors too small");
    size_t n = (size_t)mod_rows * H;
    int ok = h3_gpu_cast_f32_to_bf16(g, d->feat_bf16, features, mod_rows * 256) &&
             plain(d, &d->time_l1, d->c_wide, d->feat_bf16, mod_rows, QW_LINEAR_STORE) &&
             h3_gpu_silu_bf16(g, d->c_wide, d->c_wide, (uint32_t)n) &&
             plain(d, &d->time_l2, temb, d->c_wide, mod_rows, QW_LINEAR_STORE) &&
             h3_gpu_silu_bf16(g, d->c_silu, temb, (uint32_t)n) &&
             plain(d, &d->norm_out, norm_out_scale, d->c_silu, mod_rows, QW_LINEAR_STORE) &&
             plain(d, &d->mod, d->mod_raw, d->c_silu, mod_rows, QW_LINEAR_STORE) &&
             qw_gpu_modulation_reorder_bf16(g, modulation, d->mod_raw, mod_rows, H,
                                            d->cfg.adaln_shift);
    if (!ok) return set_error(error, error_size, "conditioning failed: %s", h3_gpu_error(g));
    return 1;
}

/* ---------------------------------------------------------------------- */
/* block                                                                  */

/* Attention of a block's rows against cached keys (ti2i target-only
 * steps): the rows' own K/V are written at `base` of the [rows, H] caches,
 * then their queries attend to all cache rows. */
typedef struct {
    h3_gpu_tensor *k, *v;
    uint32_t base, rows;
} qw_kv_cache;

/* The fused q|k|v projection with the per-head RMS norm of q and k
 * (h3_shaders.metal:4309-4329) and their RoPE (4864-4896) in its epilogue:
 * one launch, the same result as the linear followed by
 * qw_gpu_qk_norm_rope_bf16. */
static int qkv_linear(qw_dit *d, const qw_layer *L, uint32_t M, const h3_gpu_tensor *rope_cos,
                      const h3_gpu_tensor *rope_sin, uint32_t rope_rows) {
    const uint32_t H = d->cfg.hidden;
    qw_linear_desc desc;
    memset(&desc, 0, sizeof(desc));
    desc.out = d->ws_qkv;
    desc.ldc = 3 * H;
    desc.in = d->ws_mod;
    desc.lda = H;
    desc.weight = L->qkv.w;
    desc.wscale = L->qkv.scales;
    desc.bias = L->qkv.bias;
    desc.rows = M;
    desc.k = H;
    desc.cols = 3 * H;
    desc.epilogue = QW_LINEAR_QKNORM;
    desc.norm_q = L->norm_q;
    desc.norm_k = L->norm_k;
    desc.rope_cos = rope_cos;
    desc.rope_sin = rope_sin;
    desc.rope_rows = rope_rows;
    desc.eps = 1e-6f;
    return qw_gpu_linear(d->gpu, &desc);
}

static int block_run(qw_dit *d, int li, h3_gpu_tensor *hidden, uint32_t batch, uint32_t rows,
                     uint32_t text_rows, const h3_gpu_tensor *modulation,
                     const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin,
                     const h3_gpu_tensor *row_map, const h3_gpu_tensor *kv_limit,
                     h3_gpu_tensor *k_out, h3_gpu_tensor *v_out, h3_gpu_tensor *debug_attn,
                     const qw_kv_cache *kvc) {
    h3_gpu *g = d->gpu;
    const qw_layer *L = &d->layer[li];
    const uint32_t H = d->cfg.hidden, F = d->cfg.mlp_width, S = slots_of(&d->cfg);
    const uint32_t M = batch * rows;
    const int sh = d->cfg.adaln_shift;
    int ok;

    prof_begin(d);
    span_b(d, QW_SPAN_LN1);
    ok = qw_gpu_layer_norm_mod_shift_bf16(g, d->ws_mod, hidden, modulation, row_map, M, H, S, 0,
                                          sh ? 4 : -1, 1e-6f);
    span_e(d);
    span_b(d, QW_SPAN_QKV);
    ok = ok && qkv_linear(d, L, M, rope_cos, rope_sin, rows);
    span_e(d);
    prof_end(d, P_INPUT);
    if (!ok) return 0;

    prof_begin(d);
    qw_attention_desc ad;
    memset(&ad, 0, sizeof(ad));
    ad.out = d->ws_attn;
    ad.ldo = H;
    ad.q = ad.k = ad.v = d->ws_qkv;
    ad.q_offset = 0;
    ad.k_offset = H;
    ad.v_offset = 2 * (size_t)H;
    ad.ldq = ad.ldk = ad.ldv = 3 * H;
    ad.kv_limit = kv_limit;
    ad.batch = batch;
    ad.q_rows = ad.kv_rows = rows;
    ad.heads = d->cfg.heads;
    ad.text_rows = text_rows;
    ad.text_causal = d->cfg.text_causal;
    ad.scale = 1.0f / sqrtf(128.0f);
    if (kvc) { /* this step's rows into the cache, then attend to all of it */
        ok = qw_gpu_copy_rows(g, kvc->k, (size_t)kvc->base * H, H, d->ws_qkv, H, 3 * H, M, H) &&
             qw_gpu_copy_rows(g, kvc->v, (size_t)kvc->base * H, H, d->ws_qkv, 2 * (size_t)H,
                              3 * H, M, H);
        if (!ok) return 0;
        ad.k = kvc->k;
        ad.v = kvc->v;
        ad.k_offset = ad.v_offset = 0;
        ad.ldk = ad.ldv = H;
        ad.kv_rows = kvc->rows;
        ad.kv_limit = NULL;
        ad.text_rows = 0; /* every query sees every cached key */
    }
    span_b(d, QW_SPAN_ATTN);
    ok = qw_gpu_attention_bf16(g, &ad);
    span_e(d);
    if (ok && k_out) ok = qw_gpu_copy_rows(g, k_out, 0, H, d->ws_qkv, H, 3 * H, M, H);
    if (ok && v_out) ok = qw_gpu_copy_rows(g, v_out, 0, H, d->ws_qkv, 2 * (size_t)H, 3 * H, M, H);
    if (ok && debug_attn) ok = h3_gpu_copy_bf16(g, debug_attn, 0, d->ws_attn, 0, (size_t)M * H);
    prof_end(d, P_ATTN);
    if (!ok) return 0;

    prof_begin(d);
    span_b(d, QW_SPAN_OUT);
    ok = linear(d, &L->out, hidden, 0, H, d->ws_attn, 0, H, M, QW_LINEAR_GATE, modulation, row_map,
                S, 2);
    span_e(d);
    prof_end(d, P_OUT);
    if (!ok) return 0;

    prof_begin(d);
    span_b(d, QW_SPAN_LN2);
    ok = qw_gpu_layer_norm_mod_shift_bf16(g, d->ws_mod, hidden, modulation, row_map, M, H, S, 1,
                                          sh ? 5 : -1, 1e-6f);
    span_e(d);
    prof_end(d, P_LN);
    if (!ok) return 0;

    prof_begin(d);
    if (d->cfg.mlp_act == QW_MLP_GELU_TANH) {
        span_b(d, QW_SPAN_UP);
        ok = plain(d, &L->fc1, d->ws_wide, d->ws_mod, M, QW_LINEAR_GELU);
        span_e(d);
        span_b(d, QW_SPAN_DOWN);
        ok = ok && linear(d, &L->fc2, hidden, 0, H, d->ws_wide, 0, F, M, QW_LINEAR_GATE,
                          modulation, row_map, S, 3);
        span_e(d);
    } else {
        span_b(d, QW_SPAN_UP);
        ok = plain(d, &L->fc1, d->ws_wide, d->ws_mod, M, QW_LINEAR_STORE) &&
             qw_gpu_swiglu_bf16(g, d->ws_act, d->ws_wide, M, F);
        span_e(d);
        span_b(d, QW_SPAN_DOWN);
        ok = ok && linear(d, &L->fc2, hidden, 0, H, d->ws_act, 0, F, M, QW_LINEAR_GATE,
                          modulation, row_map, S, 3);
        span_e(d);
    }
    prof_end(d, P_MLP);
    return ok;
}

static int check_row_map(const h3_gpu_tensor *row_map, uint32_t rows) {
    return row_map && h3_gpu_tensor_dtype(row_map) == H3_GPU_U32 &&
           h3_gpu_tensor_elements(row_map) >= rows;
}

int qw_dit_block(qw_dit *d, int layer, h3_gpu_tensor *hidden, const h3_gpu_tensor *modulation,
                 const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin,
                 const h3_gpu_tensor *row_map, uint32_t rows, uint32_t text_rows,
                 const h3_gpu_tensor *kv_limit, const qw_dit_segment *segs, uint32_t seg_count,
                 h3_gpu_tensor *k_out, h3_gpu_tensor *v_out, h3_gpu_tensor *debug_attn,
                 char *error, size_t error_size) {
    (void)segs;
    (void)seg_count;
    if (!d) return set_error(error, error_size, "no dit");
    if (layer < 0 || (uint32_t)layer >= d->cfg.layers)
        return set_error(error, error_size, "layer %d out of range", layer);
    const size_t n = (size_t)rows * d->cfg.hidden;
    if (text_rows > rows) return set_error(error, error_size, "text_rows > rows");
    if (h3_gpu_tensor_elements(hidden) < n || !check_row_map(row_map, rows))
        return set_error(error, error_size, "block %d: hidden/row_map too small", layer);
    if ((k_out && h3_gpu_tensor_elements(k_out) < n) || (v_out && h3_gpu_tensor_elements(v_out) < n) ||
        (debug_attn && h3_gpu_tensor_elements(debug_attn) < n))
        return set_error(error, error_size, "block %d: output tensors too small", layer);
    if (!ensure_ws(d, rows)) return set_error(error, error_size, "workspace allocation failed");
    if (!block_run(d, layer, hidden, 1, rows, text_rows, modulation, rope_cos, rope_sin, row_map,
                   kv_limit, k_out, v_out, debug_attn, NULL))
        return set_error(error, error_size, "block %d kernel failed: %s", layer,
                         h3_gpu_error(d->gpu));
    return 1;
}

void qw_dit_prefix_limits(const qw_dit_segment *segs, uint32_t seg_count, uint32_t *limits) {
    /* qwen_dit.m:1651-1665: text runs causal (run start + r + 1), image
     * runs see every key up to their run end. */
    uint32_t start = 0;
    for (uint32_t s = 0; s < seg_count; s++) {
        const uint32_t end = start + segs[s].rows;
        for (uint32_t r = 0; r < segs[s].rows; r++)
            limits[start + r] = segs[s].is_image ? end : start + r + 1;
        start = end;
    }
}

int qw_dit_final(qw_dit *d, h3_gpu_tensor *hidden, const h3_gpu_tensor *norm_out_scale,
                 const h3_gpu_tensor *row_map, uint32_t rows, h3_gpu_tensor *output, char *error,
                 size_t error_size) {
    /* qwen_dit.m:1478-1496 */
    if (!d) return set_error(error, error_size, "no dit");
    const uint32_t H = d->cfg.hidden;
    if (h3_gpu_tensor_elements(hidden) < (size_t)rows * H || !check_row_map(row_map, rows) ||
        h3_gpu_tensor_elements(output) < (size_t)rows * d->cfg.z_dim)
        return set_error(error, error_size, "final: tensors too small");
    if (!ensure_ws(d, rows)) return set_error(error, error_size, "workspace allocation failed");
    const int sh = d->cfg.adaln_shift;
    int ok = qw_gpu_layer_norm_mod_shift_bf16(d->gpu, d->ws_mod, hidden, norm_out_scale, row_map,
                                              rows, H, sh ? 2 : 1, 0, sh ? 1 : -1, 1e-6f) &&
             plain(d, &d->proj_out, output, d->ws_mod, rows, QW_LINEAR_STORE);
    if (!ok) return set_error(error, error_size, "final projection failed: %s", h3_gpu_error(d->gpu));
    return 1;
}

/* ---------------------------------------------------------------------- */
/* forward                                                                */

static int ensure_row_map(qw_dit *d, uint32_t rows, uint32_t text_rows, uint32_t batch) {
    if (d->row_map && d->rm_rows == rows && d->rm_text == text_rows && d->rm_batch == batch)
        return 1;
    h3_gpu_tensor_free(d->row_map);
    d->row_map = NULL;
    uint32_t *host = malloc(sizeof(uint32_t) * (size_t)rows * batch);
    if (!host) return 0;
    /* qwen_dit.m:1510-1516: text rows ride the t = 0 modulation row */
    for (uint32_t b = 0; b < batch; b++)
        for (uint32_t i = 0; i < rows; i++) host[(size_t)b * rows + i] = i < text_rows ? 1u : 0u;
    d->row_map = h3_gpu_tensor_from_u32(d->gpu, host, (size_t)rows * batch);
    free(host);
    if (!d->row_map) return 0;
    d->rm_rows = rows;
    d->rm_text = text_rows;
    d->rm_batch = batch;
    return 1;
}

/* features: NULL = compute them for {sigma, 0} on the host and upload;
 * else copy the [2, 256] f32 rows at feat_off of that device table */
static int forward_impl(qw_dit *d, const h3_gpu_tensor *text_in, uint32_t text_rows,
                        const h3_gpu_tensor *latents, uint32_t image_rows, uint32_t batch,
                        float sigma, const h3_gpu_tensor *features, size_t feat_off,
                        const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin,
                        h3_gpu_tensor *output, char *error, size_t error_size) {
    if (!d) return set_error(error, error_size, "no dit");
    h3_gpu *g = d->gpu;
    const uint32_t rows = text_rows + image_rows, H = d->cfg.hidden, S = slots_of(&d->cfg);
    if (!batch || !rows) return set_error(error, error_size, "empty forward");
    const uint32_t M = batch * rows;
    if (text_rows && (!text_in || h3_gpu_tensor_elements(text_in) < (size_t)batch * text_rows * d->cfg.text_dim))
        return set_error(error, error_size, "text_in too small");
    if (image_rows && (!latents || h3_gpu_tensor_elements(latents) < (size_t)batch * image_rows * d->cfg.z_dim))
        return set_error(error, error_size, "latents too small");
    if (!output || h3_gpu_tensor_elements(output) < (size_t)M * d->cfg.z_dim)
        return set_error(error, error_size, "output too small");
    if (!rope_cos || !rope_sin || h3_gpu_tensor_elements(rope_cos) < (size_t)rows * 64 ||
        h3_gpu_tensor_elements(rope_sin) < (size_t)rows * 64)
        return set_error(error, error_size, "rope tables must cover %u rows", rows);
    if (!ensure_ws(d, M) || !ensure_row_map(d, rows, text_rows, batch))
        return set_error(error, error_size, "forward allocation failed: %s", h3_gpu_error(g));
    if (d->joint_rows < M) {
        h3_gpu_tensor_free(d->joint);
        d->joint = h3_gpu_tensor_new_bf16(g, (size_t)M * H);
        d->joint_rows = d->joint ? M : 0;
        if (!d->joint) return set_error(error, error_size, "joint allocation failed");
    }
    if (d->profile) memset(d->prof_ms, 0, sizeof(d->prof_ms));

    prof_begin(d);
    for (uint32_t b = 0; b < batch; b++)
        if (!embed_one(d, text_in, (size_t)b * text_rows * d->cfg.text_dim, text_rows, latents,
                       (size_t)b * image_rows * d->cfg.z_dim, image_rows, d->joint,
                       (size_t)b * rows * H))
            return set_error(error, error_size, "embed failed: %s", h3_gpu_error(g));
    prof_end(d, P_EMBED);

    prof_begin(d);
    int fok;
    if (features) {
        fok = qw_gpu_copy_rows(g, d->feat, 0, 512, features, feat_off, 512, 1, 512);
    } else {
        const float sigmas[2] = {sigma, 0.0f};
        float feats[512];
        qw_dit_timestep_features(sigmas, 2, feats);
        fok = h3_gpu_tensor_write_f32(d->feat, feats, 512);
    }
    if (!fok || !qw_dit_conditioning(d, d->feat, 2, d->temb, d->modulation, d->norm_out_mod,
                                     error, error_size))
        return error && *error ? 0 : set_error(error, error_size, "conditioning failed");
    prof_end(d, P_COND);

    const size_t MH = (size_t)M * H;
    if (d->trace_hidden) {
        if (h3_gpu_tensor_elements(d->trace_hidden) < (size_t)(d->cfg.layers + 1) * MH ||
            (d->trace_mod && h3_gpu_tensor_elements(d->trace_mod) < (size_t)2 * S * H))
            return set_error(error, error_size, "trace tensors too small for %u layers of %u rows",
                             d->cfg.layers, M);
        if (!h3_gpu_copy_bf16(g, d->trace_hidden, 0, d->joint, 0, MH) ||
            (d->trace_mod &&
             !h3_gpu_copy_bf16(g, d->trace_mod, 0, d->modulation, 0, (size_t)2 * S * H)))
            return set_error(error, error_size, "trace copy failed: %s", h3_gpu_error(g));
    }
    for (uint32_t l = 0; l < d->cfg.layers; l++) {
        if (!block_run(d, (int)l, d->joint, batch, rows, text_rows, d->modulation, rope_cos,
                       rope_sin, d->row_map, NULL, NULL, NULL, NULL, NULL))
            return set_error(error, error_size, "block %u kernel failed: %s", l, h3_gpu_error(g));
        if (d->trace_hidden &&
            !h3_gpu_copy_bf16(g, d->trace_hidden, (size_t)(l + 1) * MH, d->joint, 0, MH))
            return set_error(error, error_size, "trace copy failed: %s", h3_gpu_error(g));
    }

    prof_begin(d);
    const int sh = d->cfg.adaln_shift;
    int ok = qw_gpu_layer_norm_mod_shift_bf16(g, d->ws_mod, d->joint, d->norm_out_mod, d->row_map,
                                              M, H, sh ? 2 : 1, 0, sh ? 1 : -1, 1e-6f) &&
             plain(d, &d->proj_out, output, d->ws_mod, M, QW_LINEAR_STORE);
    prof_end(d, P_FINAL);
    if (!ok) return set_error(error, error_size, "final projection failed: %s", h3_gpu_error(g));
    return 1;
}

int qw_dit_set_trace(qw_dit *d, h3_gpu_tensor *hidden, h3_gpu_tensor *modulation) {
    if (!d) return 0;
    if (!hidden && modulation) return 0;
    if ((hidden && h3_gpu_tensor_dtype(hidden) != H3_GPU_BF16) ||
        (modulation && h3_gpu_tensor_dtype(modulation) != H3_GPU_BF16))
        return 0;
    d->trace_hidden = hidden;
    d->trace_mod = modulation;
    return 1;
}

int qw_dit_forward_batch(qw_dit *d, const h3_gpu_tensor *text_in, uint32_t text_rows,
                         const h3_gpu_tensor *latents, uint32_t image_rows, uint32_t batch,
                         float sigma, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin,
                         h3_gpu_tensor *output, char *error, size_t error_size) {
    return forward_impl(d, text_in, text_rows, latents, image_rows, batch, sigma, NULL, 0,
                        rope_cos, rope_sin, output, error, error_size);
}

int qw_dit_forward_batch_features(qw_dit *d, const h3_gpu_tensor *text_in, uint32_t text_rows,
                                  const h3_gpu_tensor *latents, uint32_t image_rows,
                                  uint32_t batch, const h3_gpu_tensor *features,
                                  size_t feature_offset, const h3_gpu_tensor *rope_cos,
                                  const h3_gpu_tensor *rope_sin, h3_gpu_tensor *output,
                                  char *error, size_t error_size) {
    if (!features || h3_gpu_tensor_dtype(features) != H3_GPU_F32 ||
        h3_gpu_tensor_elements(features) < feature_offset + 512)
        return set_error(error, error_size, "features must be f32 [2, 256] at the offset");
    return forward_impl(d, text_in, text_rows, latents, image_rows, batch, 0.0f, features,
                        feature_offset, rope_cos, rope_sin, output, error, error_size);
}

int qw_dit_forward(qw_dit *d, const h3_gpu_tensor *text_in, uint32_t text_rows,
                   const h3_gpu_tensor *latents, uint32_t image_rows, float sigma,
                   const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin,
                   h3_gpu_tensor *output, char *error, size_t error_size) {
    /* qwen_dit.m:1498-1568 (the reference submits inside; so do we, at the
     * end, so the caller's read sees the result) */
    return qw_dit_forward_batch(d, text_in, text_rows, latents, image_rows, 1, sigma, rope_cos,
                                rope_sin, output, error, error_size) &&
           (h3_gpu_submit(d->gpu) && h3_gpu_begin(d->gpu)
                ? 1
                : set_error(error, error_size, "forward failed: %s", h3_gpu_error(d->gpu)));
}

/* ---------------------------------------------------------------------- */
/* ti2i: segmented joint sequence, block-causal prefix attention, and the  */
/* cross-step K/V cache (qwen_dit.m:1572-1665, 1667-1967)                  */

static int segs_valid(const qw_dit *d, const h3_gpu_tensor *text_in, const h3_gpu_tensor *latents,
                      const qw_dit_segment *segs, uint32_t seg_count, uint32_t *rows, char *error,
                      size_t error_size) {
    const size_t text_total = text_in ? h3_gpu_tensor_elements(text_in) / d->cfg.text_dim : 0;
    const size_t image_total = latents ? h3_gpu_tensor_elements(latents) / d->cfg.z_dim : 0;
    uint64_t n = 0;
    if (!segs || !seg_count) return set_error(error, error_size, "ti2i: no runs");
    for (uint32_t s = 0; s < seg_count; s++) {
        const size_t have = segs[s].is_image ? image_total : text_total;
        if (!segs[s].rows || segs[s].src_offset > have || segs[s].rows > have - segs[s].src_offset)
            return set_error(error, error_size, "ti2i: run %u (%u %s rows at %u) outside its source",
                             s, segs[s].rows, segs[s].is_image ? "image" : "text",
                             segs[s].src_offset);
        n += segs[s].rows;
    }
    if (n > (1u << 24)) return set_error(error, error_size, "ti2i: %llu rows", (unsigned long long)n);
    *rows = (uint32_t)n;
    return 1;
}

int qw_dit_embed_segments(qw_dit *d, const h3_gpu_tensor *text_in, const h3_gpu_tensor *latents,
                          const qw_dit_segment *segs, uint32_t seg_count, h3_gpu_tensor *joint,
                          char *error, size_t error_size) {
    /* qwen_dit.m:1572-1648: the embedding is row-wise, so each run is
     * embedded straight into its joint rows (no projection of unused rows,
     * no scatter copies) */
    if (!d) return set_error(error, error_size, "no dit");
    uint32_t rows;
    if (!segs_valid(d, text_in, latents, segs, seg_count, &rows, error, error_size)) return 0;
    const uint32_t H = d->cfg.hidden;
    if (!joint || h3_gpu_tensor_elements(joint) < (size_t)rows * H)
        return set_error(error, error_size, "joint tensor too small");
    uint32_t at = 0;
    for (uint32_t s = 0; s < seg_count; s++) {
        const int img = segs[s].is_image;
        const int ok =
            img ? embed_one(d, NULL, 0, 0, latents, (size_t)segs[s].src_offset * d->cfg.z_dim,
                            segs[s].rows, joint, (size_t)at * H)
                : embed_one(d, text_in, (size_t)segs[s].src_offset * d->cfg.text_dim, segs[s].rows,
                            NULL, 0, 0, joint, (size_t)at * H);
        if (!ok) return set_error(error, error_size, "embed of run %u failed: %s", s,
                                  h3_gpu_error(d->gpu));
        at += segs[s].rows;
    }
    return 1;
}

static void cache_drop(qw_dit *d, struct qw_ti2i_cache *t) {
    for (uint32_t l = 0; l < d->cfg.layers; l++) {
        if (t->k) h3_gpu_tensor_free(t->k[l]);
        if (t->v) h3_gpu_tensor_free(t->v[l]);
    }
    free(t->k);
    free(t->v);
    free(t->segs);
    h3_gpu_tensor_free(t->th);
    h3_gpu_tensor_free(t->row0);
    memset(t, 0, sizeof(*t));
}

void qw_dit_ti2i_cache_clear(qw_dit *d) {
    if (!d) return;
    cache_drop(d, &d->ti2i[0]);
    cache_drop(d, &d->ti2i[1]);
}

static int cache_alloc(qw_dit *d, struct qw_ti2i_cache *t, uint32_t rows, uint32_t target,
                       const qw_dit_segment *segs, uint32_t seg_count) {
    cache_drop(d, t);
    const size_t n = (size_t)rows * d->cfg.hidden;
    t->k = calloc(d->cfg.layers, sizeof(*t->k));
    t->v = calloc(d->cfg.layers, sizeof(*t->v));
    t->segs = malloc(sizeof(*segs) * seg_count);
    uint32_t *zero = calloc(target, sizeof(uint32_t));
    int ok = t->k && t->v && t->segs && zero;
    for (uint32_t l = 0; ok && l < d->cfg.layers; l++)
        ok = (t->k[l] = h3_gpu_tensor_new_bf16(d->gpu, n)) &&
             (t->v[l] = h3_gpu_tensor_new_bf16(d->gpu, n));
    ok = ok && (t->th = h3_gpu_tensor_new_bf16(d->gpu, (size_t)target * d->cfg.hidden)) &&
         (t->row0 = h3_gpu_tensor_from_u32(d->gpu, zero, target));
    free(zero);
    if (!ok) {
        cache_drop(d, t);
        return 0;
    }
    memcpy(t->segs, segs, sizeof(*segs) * seg_count);
    t->rows = rows;
    t->target_rows = target;
    t->seg_count = seg_count;
    return 1;
}

int qw_dit_forward_ti2i(qw_dit *d, const h3_gpu_tensor *text_in, const h3_gpu_tensor *latents,
                        const qw_dit_segment *segs, uint32_t seg_count, uint32_t cache_slot,
                        const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, float sigma,
                        h3_gpu_tensor *output, char *error, size_t error_size) {
    if (error && error_size) error[0] = '\0';
    if (!d) return set_error(error, error_size, "no dit");
    h3_gpu *g = d->gpu;
    uint32_t rows;
    if (!segs_valid(d, text_in, latents, segs, seg_count, &rows, error, error_size)) return 0;
    if (!segs[seg_count - 1].is_image)
        return set_error(error, error_size, "ti2i: last run must be image");
    const uint32_t H = d->cfg.hidden, Z = d->cfg.z_dim, S = slots_of(&d->cfg);
    const uint32_t t_rows = segs[seg_count - 1].rows, t_base = rows - t_rows;
    if (!rope_cos || !rope_sin || h3_gpu_tensor_elements(rope_cos) < (size_t)rows * 64 ||
        h3_gpu_tensor_elements(rope_sin) < (size_t)rows * 64)
        return set_error(error, error_size, "rope tables must cover %u rows", rows);
    if (!output || h3_gpu_tensor_elements(output) < (size_t)rows * Z)
        return set_error(error, error_size, "output too small");
    struct qw_ti2i_cache *c = &d->ti2i[cache_slot ? 1 : 0];
    /* qwen_dit.m:1694-1699: the cond rows' inputs do not change across
     * sampling steps, so a filled cache with the same run layout serves
     * their K/V and only the target rows are recomputed */
    const int reuse = c->filled && c->rows == rows && c->target_rows == t_rows &&
                      c->seg_count == seg_count &&
                      memcmp(c->segs, segs, sizeof(*segs) * seg_count) == 0;
    if (!reuse && !cache_alloc(d, c, rows, t_rows, segs, seg_count))
        return set_error(error, error_size, "ti2i: cache allocation failed");
    if (!ensure_ws(d, reuse ? t_rows : rows))
        return set_error(error, error_size, "workspace allocation failed");
    /* conditioning: row 0 = sigma (target rows), row 1 = t = 0 (the rest) */
    const float sigmas[2] = {sigma, 0.0f};
    float feats[512];
    qw_dit_timestep_features(sigmas, 2, feats);
    int ok = h3_gpu_tensor_write_f32(d->feat, feats, 512) &&
             qw_dit_conditioning(d, d->feat, 2, d->temb, d->modulation, d->norm_out_mod, error,
                                 error_size);
    const int sh = d->cfg.adaln_shift;
    if (ok && !reuse) {
        if (d->joint_rows < rows) {
            h3_gpu_tensor_free(d->joint);
            d->joint = h3_gpu_tensor_new_bf16(g, (size_t)rows * H);
            d->joint_rows = d->joint ? rows : 0;
        }
        uint32_t *rm = malloc(sizeof(uint32_t) * rows), *lim = malloc(sizeof(uint32_t) * rows);
        h3_gpu_tensor *rm_t = NULL, *lim_t = NULL;
        ok = d->joint && rm && lim;
        if (ok) {
            for (uint32_t i = 0; i < rows; i++) rm[i] = i < t_base ? 1u : 0u;
            qw_dit_prefix_limits(segs, seg_count, lim);
            rm_t = h3_gpu_tensor_from_u32(g, rm, rows);
            lim_t = h3_gpu_tensor_from_u32(g, lim, rows);
            ok = rm_t && lim_t &&
                 qw_dit_embed_segments(d, text_in, latents, segs, seg_count, d->joint, error,
                                       error_size);
        }
        for (uint32_t l = 0; ok && l < d->cfg.layers; l++)
            ok = block_run(d, (int)l, d->joint, 1, rows, 0, d->modulation, rope_cos, rope_sin,
                           rm_t, lim_t, c->k[l], c->v[l], NULL, NULL);
        ok = ok &&
             qw_gpu_layer_norm_mod_shift_bf16(g, d->ws_mod, d->joint, d->norm_out_mod, rm_t, rows,
                                              H, sh ? 2 : 1, 0, sh ? 1 : -1, 1e-6f) &&
             plain(d, &d->proj_out, output, d->ws_mod, rows, QW_LINEAR_STORE) &&
             h3_gpu_submit(g) && h3_gpu_begin(g);
        free(rm);
        free(lim);
        h3_gpu_tensor_free(rm_t);
        h3_gpu_tensor_free(lim_t);
        if (!ok) {
            cache_drop(d, c); /* half-filled K/V must not be served later */
            if (error && !*error) set_error(error, error_size, "%s", h3_gpu_error(g));
            return error && *error ? 0 : set_error(error, error_size, "ti2i full pass failed");
        }
        c->filled = 1;
        return 1;
    }
    if (ok) { /* target-only pass: the target run's rows against the cached K/V */
        const qw_dit_segment *ts = &segs[seg_count - 1];
        h3_gpu_tensor *cv = h3_gpu_tensor_view(rope_cos, (size_t)t_base * 64, (size_t)t_rows * 64);
        h3_gpu_tensor *sv = h3_gpu_tensor_view(rope_sin, (size_t)t_base * 64, (size_t)t_rows * 64);
        h3_gpu_tensor *ov = h3_gpu_tensor_view(output, (size_t)t_base * Z, (size_t)t_rows * Z);
        ok = cv && sv && ov &&
             embed_one(d, NULL, 0, 0, latents, (size_t)ts->src_offset * Z, t_rows, c->th, 0);
        for (uint32_t l = 0; ok && l < d->cfg.layers; l++) {
            const qw_kv_cache kvc = {c->k[l], c->v[l], t_base, rows};
            ok = block_run(d, (int)l, c->th, 1, t_rows, 0, d->modulation, cv, sv, c->row0, NULL,
                           NULL, NULL, NULL, &kvc);
        }
        ok = ok &&
             qw_gpu_layer_norm_mod_shift_bf16(g, d->ws_mod, c->th, d->norm_out_mod, c->row0,
                                              t_rows, H, sh ? 2 : 1, 0, sh ? 1 : -1, 1e-6f) &&
             plain(d, &d->proj_out, ov, d->ws_mod, t_rows, QW_LINEAR_STORE) &&
             h3_gpu_submit(g) && h3_gpu_begin(g);
        h3_gpu_tensor_free(cv);
        h3_gpu_tensor_free(sv);
        h3_gpu_tensor_free(ov);
    }
    (void)S;
    if (!ok) return error && *error ? 0 : set_error(error, error_size, "ti2i target pass failed: %s",
                                                    h3_gpu_error(g));
    return 1;
}

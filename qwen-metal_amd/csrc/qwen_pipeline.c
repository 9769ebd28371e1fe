/* qwen_pipeline.c — scheduler, joint RoPE tables and the FlowMatch Euler
 * denoise loop around the DiT forward (reference qwen_pipeline.m:130-486).
 * With guidance, the cond and uncond branches run as one batch-2 forward
 * (M = 2 * rows in every linear) when their text lengths match. */
#include "../../include/qwen_pipeline.h"
#include "../../include/qwen_gpu_ext.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void qw_sched_cfg_default(qw_sched_cfg *c) {
    c->dynamic_shifting = 1;
    c->base_seq = 256.0;
    c->max_seq = 8192.0;
    c->base_shift = 0.5;
    c->max_shift = 0.9;
    c->has_terminal = 1;
    c->shift_terminal = 0.02;
}

/* FlowMatch sigma schedule (semantics of reference qwen_pipeline.m:130-205).
 *
 * Each step's timestep t_i (linear from 1 down to 1/steps, or the caller's
 * turbo list) is a float32. With dynamic shifting it maps to
 *     sigma_i = e^mu / (e^mu + (1 / t_i - 1)),
 * mu = slope * seq_len + intercept on the line through (base_seq,
 * base_shift) and (max_seq, max_shift), e^mu in double; 1 / t_i is taken
 * in double and rounded to float32, the "- 1" is a float32 subtraction and
 * the quotient is rounded to float32. The optional terminal stretch then
 * rescales every 1 - sigma_i so the last sigma lands on shift_terminal:
 *     k = fl32(fl32(1 - sigma_last) / (1 - shift_terminal)),
 *     sigma_i = fl32(1 - fl32(1 - sigma_i) / k).
 * Every listed fl32 is a rounding point of the released schedule; the
 * float32 values are exact in the double output, which ends with 0. */
static float fl32(double v) { return (float)v; }

static double shift_exp_mu(const qw_sched_cfg *c, uint32_t seq_len) {
    const double slope = c->max_seq == c->base_seq
                             ? 0.0
                             : (c->max_shift - c->base_shift) / (c->max_seq - c->base_seq);
    const double intercept = c->base_shift - slope * c->base_seq;
    return exp(slope * (double)seq_len + intercept);
}

static float base_timestep(uint32_t i, uint32_t steps, const double *turbo) {
    if (turbo) return fl32(turbo[i]);
    if (steps == 1) return 1.0f;
    const double stride = (1.0 / steps - 1.0) / (double)(steps - 1);
    return fl32(1.0 + (double)i * stride);
}

int qw_pipe_schedule(uint32_t steps, uint32_t seq_len, const double *turbo_sigmas,
                     uint32_t turbo_count, const qw_sched_cfg *cfg, double *sigmas_out,
                     char *error, size_t error_size) {
    if (!cfg || !sigmas_out || steps == 0 || seq_len == 0) {
        snprintf(error, error_size, "qw_pipe_schedule: need a config, an output array, "
                 "steps > 0 and seq_len > 0");
        return 0;
    }
    if (turbo_sigmas && turbo_count != steps) {
        snprintf(error, error_size,
                 "qw_pipe_schedule: %u turbo timesteps given for a %u-step schedule",
                 turbo_count, steps);
        return 0;
    }
    const double e_mu = cfg->dynamic_shifting ? shift_exp_mu(cfg, seq_len) : 0.0;
    for (uint32_t i = 0; i < steps; i++) {
        const float t = base_timestep(i, steps, turbo_sigmas);
        float sigma = t;
        if (cfg->dynamic_shifting) {
            const float odds = fl32(1.0 / t) - 1.0f;
            sigma = fl32(e_mu / (e_mu + (double)odds));
        }
        sigmas_out[i] = sigma;
    }
    if (cfg->has_terminal && cfg->shift_terminal < 1.0) {
        const float k =
            fl32((double)fl32(1.0 - sigmas_out[steps - 1]) / (1.0 - cfg->shift_terminal));
        if (k != 0.0f)
            for (uint32_t i = 0; i < steps; i++) {
                const float rest = fl32(1.0 - sigmas_out[i]);
                sigmas_out[i] = fl32(1.0 - (double)rest / (double)k);
            }
    }
    sigmas_out[steps] = 0.0;
    return 1;
}

/* one table row: the 64 (cos, sin) pairs of position (frame, h, w) over the
 * axes (16, 56, 56), angle = position x 10000^(-2p / dim) in double */
static void rope_row(const double pos[3], float *cos_row, float *sin_row) {
    static const int dims[3] = {16, 56, 56};
    size_t col = 0;
    for (int a = 0; a < 3; a++)
        for (int p = 0; p < dims[a] / 2; p++, col++) {
            const double ang = pos[a] * pow(10000.0, -2.0 * (double)p / (double)dims[a]);
            cos_row[col] = (float)cos(ang);
            sin_row[col] = (float)sin(ang);
        }
}

size_t qw_pipe_rope_tables_blocks_host(const uint32_t *block_h, const uint32_t *block_w,
                                       const uint32_t *text_before, uint32_t n_blocks,
                                       float *cos_out, float *sin_out) {
    /* qwen_pipeline.m:611-680. One running position: each text row takes
     * it on all three axes and advances it by one; an image block keeps its
     * frame at the position it starts at, its rows sit on the centred grid
     * (h - ceil(gh/2), w - ceil(gw/2)), and the position then advances by
     * the block's longer side. */
    double position = 0.0;
    size_t row = 0;
    for (uint32_t b = 0; b < n_blocks; b++) {
        for (uint32_t t = 0; t < text_before[b]; t++, row++, position += 1.0) {
            const double pos[3] = {position, position, position};
            if (cos_out) rope_row(pos, cos_out + row * 64, sin_out + row * 64);
        }
        const uint32_t gh = block_h[b], gw = block_w[b];
        const long ch = (long)(gh - gh / 2), cw = (long)(gw - gw / 2);
        for (uint32_t y = 0; y < gh; y++)
            for (uint32_t x = 0; x < gw; x++, row++) {
                const double pos[3] = {position, (double)((long)y - ch),
                                       (double)((long)x - cw)};
                if (cos_out) rope_row(pos, cos_out + row * 64, sin_out + row * 64);
            }
        position += (double)(gh > gw ? gh : gw);
    }
    return row;
}

int qw_pipe_rope_tables_blocks(h3_gpu *gpu, const uint32_t *block_h, const uint32_t *block_w,
                               const uint32_t *text_before, uint32_t n_blocks,
                               h3_gpu_tensor **rope_cos, h3_gpu_tensor **rope_sin, char *error,
                               size_t error_size) {
    if (!rope_cos || !rope_sin || (n_blocks && (!block_h || !block_w || !text_before))) {
        snprintf(error, error_size, "rope blocks: need the block arrays and two outputs");
        return 0;
    }
    const size_t rows = qw_pipe_rope_tables_blocks_host(block_h, block_w, text_before, n_blocks,
                                                        NULL, NULL);
    if (!rows) {
        snprintf(error, error_size, "rope blocks: empty layout");
        return 0;
    }
    float *c = malloc(sizeof(float) * rows * 64), *s = malloc(sizeof(float) * rows * 64);
    h3_gpu_tensor *ct = NULL, *st = NULL;
    int ok = c && s;
    if (ok) {
        qw_pipe_rope_tables_blocks_host(block_h, block_w, text_before, n_blocks, c, s);
        ct = h3_gpu_tensor_from_f32(gpu, c, rows * 64);
        st = h3_gpu_tensor_from_f32(gpu, s, rows * 64);
        ok = ct && st;
    }
    free(c);
    free(s);
    if (!ok) {
        h3_gpu_tensor_free(ct);
        h3_gpu_tensor_free(st);
        snprintf(error, error_size, "rope blocks: host or device allocation failed");
        return 0;
    }
    *rope_cos = ct;
    *rope_sin = st;
    return 1;
}

void qw_pipe_rope_tables_host(uint32_t text_rows, uint32_t gh, uint32_t gw, float *cos_out,
                              float *sin_out) {
    /* qwen_pipeline.m:212-273: axes (16, 56, 56), text row t at (t, t, t),
     * image row (h, w) at (text_rows, h - ceil(gh/2), w - ceil(gw/2)). */
    const uint32_t rows = text_rows + gh * gw;
    const long ch = (long)(gh - gh / 2), cw = (long)(gw - gw / 2);
    for (uint32_t t = 0; t < rows; t++) {
        double pos[3];
        if (t < text_rows) {
            pos[0] = pos[1] = pos[2] = (double)t;
        } else {
            const uint32_t idx = t - text_rows;
            pos[0] = (double)text_rows;
            pos[1] = (double)((long)(idx / gw) - ch);
            pos[2] = (double)((long)(idx % gw) - cw);
        }
        rope_row(pos, cos_out + (size_t)t * 64, sin_out + (size_t)t * 64);
    }
}

int qw_pipe_rope_tables(h3_gpu *gpu, uint32_t text_rows, uint32_t gh, uint32_t gw,
                        h3_gpu_tensor **rope_cos, h3_gpu_tensor **rope_sin, char *error,
                        size_t error_size) {
    if (!gh || !gw || !rope_cos || !rope_sin) {
        snprintf(error, error_size, "qw_pipe_rope_tables: need gh, gw > 0 and two outputs");
        return 0;
    }
    const size_t n = (size_t)(text_rows + gh * gw) * 64;
    float *c = malloc(sizeof(float) * n), *s = malloc(sizeof(float) * n);
    h3_gpu_tensor *ct = NULL, *st = NULL;
    int ok = c && s;
    if (ok) {
        qw_pipe_rope_tables_host(text_rows, gh, gw, c, s);
        ct = h3_gpu_tensor_from_f32(gpu, c, n);
        st = h3_gpu_tensor_from_f32(gpu, s, n);
        ok = ct && st;
    }
    free(c);
    free(s);
    if (!ok) {
        h3_gpu_tensor_free(ct);
        h3_gpu_tensor_free(st);
        snprintf(error, error_size, "qw_pipe_rope_tables: host or device allocation failed");
        return 0;
    }
    *rope_cos = ct;
    *rope_sin = st;
    return 1;
}

static uint16_t bf16_rne(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

static float bf16_f32(uint16_t v) {
    uint32_t b = (uint32_t)v << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* The denoise loop with the latents resident on the device (fp32): per step
 * a bf16 cast (copied for the stacked CFG batch), the forward with its
 * timestep features from a table uploaded once, and the CFG + Euler kernel
 * -- no host transfer and no synchronisation until the final read-back. The
 * arithmetic is the host loop's (qwen_pipeline.m:385-429). */
static int denoise_device(qw_dit *dit, h3_gpu *gpu, const h3_gpu_tensor *text,
                          uint32_t text_rows, const h3_gpu_tensor *neg_text_in,
                          uint32_t neg_rows, float *latents, uint32_t image_rows, uint32_t z,
                          uint32_t steps, float cfg_scale, const double *sigmas, int guided,
                          int stacked, const h3_gpu_tensor *cos_t, const h3_gpu_tensor *sin_t,
                          const h3_gpu_tensor *ncos, const h3_gpu_tensor *nsin,
                          h3_gpu_tensor *lat, h3_gpu_tensor *pred, h3_gpu_tensor *npred,
                          char *error, size_t error_size) {
    const size_t count = (size_t)image_rows * z;
    const uint32_t rows = text_rows + image_rows;
    float *ft = malloc(sizeof(float) * 512 * steps);
    if (!ft) {
        snprintf(error, error_size, "denoise: out of memory");
        return 0;
    }
    for (uint32_t s = 0; s < steps; s++) {
        const float sg[2] = {(float)sigmas[s], 0.0f};
        qw_dit_timestep_features(sg, 2, ft + (size_t)s * 512);
    }
    h3_gpu_tensor *x = h3_gpu_tensor_from_f32(gpu, latents, count);
    h3_gpu_tensor *feat = h3_gpu_tensor_from_f32(gpu, ft, (size_t)512 * steps);
    free(ft);
    int ok = x && feat;
    if (!ok) snprintf(error, error_size, "denoise: allocation failed: %s", h3_gpu_error(gpu));
    for (uint32_t step = 0; ok && step < steps; step++) {
        const size_t fo = (size_t)step * 512;
        const float dt = (float)(sigmas[step + 1] - sigmas[step]);
        ok = h3_gpu_cast_f32_to_bf16(gpu, lat, x, (uint32_t)count) &&
             (!stacked || h3_gpu_copy_bf16(gpu, lat, count, lat, 0, count));
        if (ok && stacked) {
            ok = qw_dit_forward_batch_features(dit, text, text_rows, lat, image_rows, 2, feat, fo,
                                               cos_t, sin_t, pred, error, error_size) &&
                 qw_gpu_cfg_euler_f32(gpu, x, pred, (size_t)text_rows * z, pred,
                                      (size_t)(rows + text_rows) * z, count, dt, cfg_scale);
        } else if (ok) {
            ok = qw_dit_forward_batch_features(dit, text, text_rows, lat, image_rows, 1, feat, fo,
                                               cos_t, sin_t, pred, error, error_size) &&
                 (!guided ||
                  qw_dit_forward_batch_features(dit, neg_text_in, neg_rows, lat, image_rows, 1,
                                                feat, fo, ncos, nsin, npred, error,
                                                error_size)) &&
                 qw_gpu_cfg_euler_f32(gpu, x, pred, (size_t)text_rows * z, guided ? npred : NULL,
                                      (size_t)neg_rows * z, count, dt, cfg_scale);
        }
        if (!ok && error && !*error)
            snprintf(error, error_size, "denoise step %u: %s", step, h3_gpu_error(gpu));
    }
    if (ok) ok = h3_gpu_submit(gpu) && h3_gpu_begin(gpu) && h3_gpu_tensor_read_f32(x, latents, count);
    if (!ok && error && !*error) snprintf(error, error_size, "denoise: %s", h3_gpu_error(gpu));
    h3_gpu_tensor_free(x);
    h3_gpu_tensor_free(feat);
    return ok;
}

int qw_pipe_denoise(qw_dit *dit, h3_gpu *gpu, const h3_gpu_tensor *text_in, uint32_t text_rows,
                    const h3_gpu_tensor *neg_text_in, uint32_t neg_rows, float *latents,
                    uint32_t gh, uint32_t gw, uint32_t steps, float cfg_scale,
                    const double *turbo_sigmas, uint32_t turbo_count, const qw_sched_cfg *sched,
                    char *error, size_t error_size) {
    /* qwen_pipeline.m:289-486 */
    const qw_dit_config *cfg = qw_dit_get_config(dit);
    if (!cfg || !gpu || !latents || !gh || !gw || !steps) {
        snprintf(error, error_size, "denoise: bad arguments");
        return 0;
    }
    const uint32_t z = cfg->z_dim, image_rows = gh * gw;
    const size_t count = (size_t)image_rows * z;
    const int guided = cfg_scale > 1.0f && neg_text_in && neg_rows;
    const int stacked = guided && neg_rows == text_rows;
    const uint32_t rows = text_rows + image_rows, nrows = neg_rows + image_rows;
    double *sigmas = malloc(sizeof(double) * (steps + 1));
    uint16_t *lat_host = malloc(sizeof(uint16_t) * count * 2);
    uint16_t *pred_host = malloc(sizeof(uint16_t) * (size_t)(rows + (guided ? nrows : 0)) * z);
    h3_gpu_tensor *cos_t = NULL, *sin_t = NULL, *ncos = NULL, *nsin = NULL;
    h3_gpu_tensor *lat = NULL, *pred = NULL, *npred = NULL, *text2 = NULL;
    int ok = sigmas && lat_host && pred_host;
    if (!ok) {
        snprintf(error, error_size, "denoise: out of memory");
        goto done;
    }
    ok = qw_pipe_schedule(steps, image_rows, turbo_sigmas, turbo_count, sched, sigmas, error,
                          error_size) &&
         qw_pipe_rope_tables(gpu, text_rows, gh, gw, &cos_t, &sin_t, error, error_size);
    if (ok && guided && !stacked)
        ok = qw_pipe_rope_tables(gpu, neg_rows, gh, gw, &ncos, &nsin, error, error_size);
    if (!ok) goto done;
    lat = h3_gpu_tensor_new_bf16(gpu, count * (stacked ? 2 : 1));
    pred = h3_gpu_tensor_new_bf16(gpu, (size_t)rows * z * (stacked ? 2 : 1));
    if (guided && !stacked) npred = h3_gpu_tensor_new_bf16(gpu, (size_t)nrows * z);
    if (stacked && text_rows) {
        /* [cond text; uncond text] stacked for the batch-2 forward */
        text2 = h3_gpu_tensor_new_bf16(gpu, (size_t)2 * text_rows * cfg->text_dim);
        ok = text2 &&
             h3_gpu_copy_bf16(gpu, text2, 0, text_in, 0, (size_t)text_rows * cfg->text_dim) &&
             h3_gpu_copy_bf16(gpu, text2, (size_t)text_rows * cfg->text_dim, neg_text_in, 0,
                              (size_t)text_rows * cfg->text_dim);
    }
    ok = ok && lat && pred && (!guided || stacked || npred);
    if (!ok) {
        snprintf(error, error_size, "denoise: allocation failed: %s", h3_gpu_error(gpu));
        goto done;
    }
    h3_gpu_begin(gpu);
    const char *hl = getenv("QW_PIPE_HOST_LOOP");
    if (!(hl && hl[0] == '1')) {
        ok = denoise_device(dit, gpu, text_rows ? (stacked ? text2 : text_in) : NULL, text_rows,
                            neg_text_in, neg_rows, latents, image_rows, z, steps, cfg_scale,
                            sigmas, guided, stacked, cos_t, sin_t, ncos, nsin, lat, pred, npred,
                            error, error_size);
        goto done;
    }
    /* QW_PIPE_HOST_LOOP=1: the reference's own loop shape, a host round
     * trip per step (bf16 upload, prediction read-back, CFG + Euler on the
     * host); kept to check the device loop against */
    for (uint32_t step = 0; ok && step < steps; step++) {
        for (size_t i = 0; i < count; i++) lat_host[i] = bf16_rne(latents[i]);
        if (stacked) memcpy(lat_host + count, lat_host, sizeof(uint16_t) * count);
        const float sigma = (float)sigmas[step];
        ok = h3_gpu_tensor_write_bf16(lat, lat_host, count * (stacked ? 2 : 1));
        if (ok && stacked) {
            ok = qw_dit_forward_batch(dit, text_rows ? text2 : NULL, text_rows, lat, image_rows, 2,
                                      sigma, cos_t, sin_t, pred, error, error_size) &&
                 h3_gpu_submit(gpu) && h3_gpu_begin(gpu) &&
                 h3_gpu_tensor_read_bf16(pred, pred_host, (size_t)2 * rows * z);
        } else if (ok) {
            ok = qw_dit_forward(dit, text_in, text_rows, lat, image_rows, sigma, cos_t, sin_t, pred,
                                error, error_size) &&
                 h3_gpu_tensor_read_bf16(pred, pred_host, (size_t)rows * z);
            if (ok && guided)
                ok = qw_dit_forward(dit, neg_text_in, neg_rows, lat, image_rows, sigma, ncos, nsin,
                                    npred, error, error_size) &&
                     h3_gpu_tensor_read_bf16(npred, pred_host + (size_t)rows * z,
                                             (size_t)nrows * z);
        }
        if (!ok) {
            if (error && !*error) snprintf(error, error_size, "denoise step %u: %s", step,
                                           h3_gpu_error(gpu));
            break;
        }
        /* x += (sigma_next - sigma) * (neg + cfg (pos - neg)), fp32 on host */
        const float dt = (float)(sigmas[step + 1] - sigmas[step]);
        const uint16_t *pos = pred_host + (size_t)text_rows * z;
        const uint16_t *neg =
            pred_host + (size_t)rows * z + (size_t)(stacked ? text_rows : neg_rows) * z;
        for (size_t i = 0; i < count; i++) {
            float p = bf16_f32(pos[i]);
            if (guided) {
                float n = bf16_f32(neg[i]);
                p = n + cfg_scale * (p - n);
            }
            latents[i] += dt * p;
        }
    }
done:
    h3_gpu_tensor_free(cos_t);
    h3_gpu_tensor_free(sin_t);
    h3_gpu_tensor_free(ncos);
    h3_gpu_tensor_free(nsin);
    h3_gpu_tensor_free(lat);
    h3_gpu_tensor_free(pred);
    h3_gpu_tensor_free(npred);
    h3_gpu_tensor_free(text2);
    free(sigmas);
    free(lat_host);
    free(pred_host);
    return ok;
}

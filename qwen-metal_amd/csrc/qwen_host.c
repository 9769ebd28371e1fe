/* Host math of the DiT path: schedule, Euler, RoPE tables, PCG32 RNG.
 * Semantics of the reference qwen_host.c (cited per function); float32
 * intermediates exactly where the released scheduler keeps them. Built with
 * -ffp-contract=off so no multiply-add is fused behind the source's back. */
#include "../../include/qwen_host.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int qw_latent_grid(int width, int height, int *latent_w, int *latent_h) {
    /* qwen_host.c:7-16: one latent token per 16x16 pixels. */
    if (!latent_w || !latent_h || width < QWEN_VAE_SPATIAL_RATIO ||
        height < QWEN_VAE_SPATIAL_RATIO || width % QWEN_VAE_SPATIAL_RATIO ||
        height % QWEN_VAE_SPATIAL_RATIO)
        return 0;
    *latent_w = width / QWEN_VAE_SPATIAL_RATIO;
    *latent_h = height / QWEN_VAE_SPATIAL_RATIO;
    return 1;
}

double qw_calculate_shift(int image_seq_len) {
    /* qwen_host.c:18-26: linear in the sequence length between
     * (base_seq, base_shift) and (max_seq, max_shift). */
    double slope = (QWEN_SCHED_MAX_SHIFT - QWEN_SCHED_BASE_SHIFT) /
                   ((double)QWEN_SCHED_MAX_SEQ_LEN - QWEN_SCHED_BASE_SEQ_LEN);
    double intercept = QWEN_SCHED_BASE_SHIFT - slope * QWEN_SCHED_BASE_SEQ_LEN;
    return slope * (double)image_seq_len + intercept;
}

int qw_schedule_build(int steps, int image_seq_len, qw_sigma_schedule *s) {
    /* qwen_host.c:335-370. */
    if (!s || steps < 1 || steps > QWEN_MAX_STEPS || image_seq_len < 1) return 0;
    const float exp_mu = (float)exp(qw_calculate_shift(image_seq_len));
    const double stop = 1.0 / (double)steps;
    const double delta = steps > 1 ? (stop - 1.0) / (double)(steps - 1) : 0.0;
    for (int i = 0; i < steps; i++) {
        double t = i == steps - 1 ? stop : 1.0 + (double)i * delta;
        float base = (float)t;
        float inv = 1.0f / base;
        s->sigma[i] = exp_mu / (exp_mu + (inv - 1.0f));
    }
    const float scale = (1.0f - s->sigma[steps - 1]) /
                        (1.0f - (float)QWEN_SCHED_SHIFT_TERMINAL);
    for (int i = 0; i < steps; i++) s->sigma[i] = 1.0f - (1.0f - s->sigma[i]) / scale;
    s->steps = steps;
    s->sigma[steps] = 0.0f;
    return 1;
}

int qw_schedule_from_sigmas(const float *sigmas, int steps, qw_sigma_schedule *s) {
    /* qwen_host.c:372 (explicit list + terminal zero). */
    if (!sigmas || !s || steps < 1 || steps > QWEN_MAX_STEPS) return 0;
    memcpy(s->sigma, sigmas, sizeof(float) * (size_t)steps);
    s->sigma[steps] = 0.0f;
    s->steps = steps;
    return 1;
}

void qw_euler_velocity_step(float *sample, const float *velocity, size_t count,
                            float sigma, float sigma_next) {
    const float dt = sigma - sigma_next;
    for (size_t i = 0; i < count; i++) sample[i] += dt * velocity[i];
}

int qw_rope_row(int coordinate) {
    /* qwen_host.c:380-386: negative coordinates live in the tail rows. */
    if (coordinate >= 0) return coordinate < QWEN_ROPE_POS_ROWS ? coordinate : -1;
    return -coordinate <= QWEN_ROPE_NEG_ROWS ? QWEN_ROPE_ROWS + coordinate : -1;
}

int qw_rope_build(const int *axis_dim, int axes, qw_rope_tables *t) {
    /* qwen_host.c:388-430: per axis, rows = coordinates 0..8191 then
     * -1024..-1, pair frequency theta^(-2 p / dim) in float32. */
    if (!axis_dim || !t || axes < 1 || axes > QWEN_ROPE_AXES) return 0;
    size_t total = 0;
    for (int a = 0; a < axes; a++) {
        if (axis_dim[a] < 2 || axis_dim[a] % 2) return 0;
        total += (size_t)QWEN_ROPE_ROWS * (size_t)(axis_dim[a] / 2);
    }
    t->cos = malloc(sizeof(float) * total);
    t->sin = malloc(sizeof(float) * total);
    if (!t->cos || !t->sin) {
        free(t->cos);
        free(t->sin);
        t->cos = t->sin = NULL;
        return 0;
    }
    t->axes = axes;
    size_t base = 0;
    for (int a = 0; a < axes; a++) {
        const int pairs = axis_dim[a] / 2;
        t->axis_dim[a] = axis_dim[a];
        for (int p = 0; p < pairs; p++) {
            float freq = (float)pow(QWEN_ROPE_THETA, -2.0 * p / (double)axis_dim[a]);
            for (int row = 0; row < QWEN_ROPE_ROWS; row++) {
                int coord = row < QWEN_ROPE_POS_ROWS ? row : row - QWEN_ROPE_ROWS;
                float ang = (float)coord * freq;
                t->cos[base + (size_t)row * pairs + p] = cosf(ang);
                t->sin[base + (size_t)row * pairs + p] = sinf(ang);
            }
        }
        base += (size_t)QWEN_ROPE_ROWS * (size_t)pairs;
    }
    return 1;
}

void qw_rope_free(qw_rope_tables *t) {
    if (!t) return;
    free(t->cos);
    free(t->sin);
    t->cos = t->sin = NULL;
}

uint32_t qw_rng_u32(qw_rng *r) {
    /* qwen_host.c:440-446: PCG32, XSH-RR output of the old state. */
    const uint64_t old = r->state;
    r->state = old * UINT64_C(6364136223846793005) + r->increment;
    const uint32_t x = (uint32_t)(((old >> 18u) ^ old) >> 27u);
    const uint32_t rot = (uint32_t)(old >> 59u);
    return (x >> rot) | (x << ((32u - rot) & 31u));
}

void qw_rng_seed(qw_rng *r, uint64_t seed) {
    /* qwen_host.c:452-458 */
    memset(r, 0, sizeof(*r));
    r->increment = (seed << 1u) | 1u;
    (void)qw_rng_u32(r);
    r->state += seed ^ UINT64_C(0x9e3779b97f4a7c15);
    (void)qw_rng_u32(r);
}

float qw_rng_normal(qw_rng *r) {
    /* qwen_host.c:460-471: Box-Muller in double, cosine branch first. */
    if (r->has_spare) {
        r->has_spare = 0;
        return r->spare;
    }
    const double u1 = ((double)qw_rng_u32(r) + 1.0) / 4294967297.0;
    const double u2 = ((double)qw_rng_u32(r) + 0.5) / 4294967296.0;
    const double rad = sqrt(-2.0 * log(u1));
    const double th = 6.283185307179586476925286766559 * u2;
    r->spare = (float)(rad * sin(th));
    r->has_spare = 1;
    return (float)(rad * cos(th));
}

void qw_rng_fill_normal(qw_rng *r, float *v, size_t n) {
    for (size_t i = 0; i < n; i++) v[i] = qw_rng_normal(r);
}

/* qwen_host — deterministic host math of the DiT path (reference
 * qwen_host.h:1-111): sigma schedule, Euler step, RoPE tables, latent grid
 * and the seeded PCG32 + Box-Muller RNG used for synthetic inputs. Same
 * names, constants and semantics as the reference; own implementation. */
#ifndef QWEN_HOST_H
#define QWEN_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWEN_TRAIN_TIMESTEPS 1000.0
#define QWEN_SCHED_BASE_SEQ_LEN 256
#define QWEN_SCHED_MAX_SEQ_LEN 8192
#define QWEN_SCHED_BASE_SHIFT 0.5
#define QWEN_SCHED_MAX_SHIFT 0.9
#define QWEN_SCHED_SHIFT_TERMINAL 0.02
#define QWEN_MAX_STEPS 1000

#define QWEN_VAE_SPATIAL_RATIO 16
#define QWEN_Z_DIM 64
#define QWEN_HIDDEN 4096
#define QWEN_HEADS 32
#define QWEN_HEAD_DIM 128
#define QWEN_DIT_LAYERS 32
#define QWEN_MLP_RATIO 3
#define QWEN_MLP_HIDDEN (QWEN_HIDDEN * QWEN_MLP_RATIO)
#define QWEN_TEXT_HIDDEN 4096
#define QWEN_EPS 1e-6f

#define QWEN_ROPE_AXES 3
#define QWEN_ROPE_THETA 10000.0
#define QWEN_ROPE_POS_ROWS 8192
#define QWEN_ROPE_NEG_ROWS 1024
#define QWEN_ROPE_ROWS (QWEN_ROPE_POS_ROWS + QWEN_ROPE_NEG_ROWS)

/* reference qwen_host.h:50 */
int qw_latent_grid(int width, int height, int *latent_w, int *latent_h);
/* reference qwen_host.h:55 */
double qw_calculate_shift(int image_seq_len);

typedef struct {
    int steps;
    float sigma[QWEN_MAX_STEPS + 1];
} qw_sigma_schedule;

/* reference qwen_host.h:66 */
int qw_schedule_build(int steps, int image_seq_len, qw_sigma_schedule *schedule);
/* reference qwen_host.h:70-71 */
int qw_schedule_from_sigmas(const float *sigmas, int steps,
                            qw_sigma_schedule *schedule);
/* reference qwen_host.h:75-76: sample += (sigma - sigma_next) * velocity */
void qw_euler_velocity_step(float *sample, const float *velocity,
                            size_t count, float sigma, float sigma_next);

typedef struct {
    int axes;
    int axis_dim[QWEN_ROPE_AXES];
    float *cos;
    float *sin;
} qw_rope_tables;

/* reference qwen_host.h:90-97 */
int qw_rope_build(const int *axis_dim, int axes, qw_rope_tables *tables);
void qw_rope_free(qw_rope_tables *tables);
int qw_rope_row(int coordinate);

typedef struct {
    uint64_t state;
    uint64_t increment;
    float spare;
    int has_spare;
} qw_rng;

/* reference qwen_host.h:106-109 */
void qw_rng_seed(qw_rng *rng, uint64_t seed);
uint32_t qw_rng_u32(qw_rng *rng);
float qw_rng_normal(qw_rng *rng);
void qw_rng_fill_normal(qw_rng *rng, float *values, size_t count);

#ifdef __cplusplus
}
#endif
#endif

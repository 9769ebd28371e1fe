/* qwen_pipeline — the denoise loop around the DiT forward (reference
 * qwen_pipeline.h:46-94): scheduler config, sigma schedule, joint RoPE
 * tables and the FlowMatch Euler loop with classifier-free guidance. */
#ifndef QWEN_PIPELINE_H
#define QWEN_PIPELINE_H

#include <stddef.h>
#include <stdint.h>

#include "h3_gpu.h"
#include "qwen_dit.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference qwen_pipeline.h:46-60 */
typedef struct {
    int dynamic_shifting;
    double base_seq;
    double max_seq;
    double base_shift;
    double max_shift;
    int has_terminal;
    double shift_terminal;
} qw_sched_cfg;

/* The released base-model scheduler config (dynamic shift, terminal 0.02). */
void qw_sched_cfg_default(qw_sched_cfg *cfg);

/* reference qwen_pipeline.h:69-72 */
int qw_pipe_schedule(uint32_t steps, uint32_t seq_len,
                     const double *turbo_sigmas, uint32_t turbo_count,
                     const qw_sched_cfg *cfg, double *sigmas_out,
                     char *error, size_t error_size);

/* reference qwen_pipeline.h:78-81 */
int qw_pipe_rope_tables(h3_gpu *gpu, uint32_t text_rows, uint32_t gh,
                        uint32_t gw, h3_gpu_tensor **rope_cos,
                        h3_gpu_tensor **rope_sin, char *error,
                        size_t error_size);
/* Host-side form of the same tables ([text_rows + gh*gw, 64] each). */
void qw_pipe_rope_tables_host(uint32_t text_rows, uint32_t gh, uint32_t gw,
                              float *cos_out, float *sin_out);

/* reference qwen_pipeline.h:115-122 (qwen_pipeline.m:611-680): the ti2i
 * multi-block tables. Block b is text_before[b] text rows, then a
 * block_h[b] x block_w[b] image grid. One running position: a text row
 * takes it on all three axes and advances it by 1; an image block's frame
 * is the position where it starts, its rows sit on the grid centred as in
 * qw_pipe_rope_tables, and the position then advances by max(h, w). Rows
 * = sum text_before + sum h*w, 64 (cos, sin) pairs each. 0 with a message
 * on an empty layout or a failed allocation. */
int qw_pipe_rope_tables_blocks(h3_gpu *gpu, const uint32_t *block_h,
                               const uint32_t *block_w,
                               const uint32_t *text_before,
                               uint32_t n_blocks, h3_gpu_tensor **rope_cos,
                               h3_gpu_tensor **rope_sin, char *error,
                               size_t error_size);
/* Host-side form: fills [rows, 64] cos / sin (both NULL: only counts) and
 * returns the row count. */
size_t qw_pipe_rope_tables_blocks_host(const uint32_t *block_h,
                                       const uint32_t *block_w,
                                       const uint32_t *text_before,
                                       uint32_t n_blocks, float *cos_out,
                                       float *sin_out);

/* reference qwen_pipeline.h:87-94. latents [gh*gw, 64] fp32 updated in
 * place. With guidance and neg_rows == text_rows the cond and uncond
 * branches run as ONE batch-2 forward (stacked rows); otherwise as two
 * forwards. */
int qw_pipe_denoise(qw_dit *dit, h3_gpu *gpu, const h3_gpu_tensor *text_in,
                    uint32_t text_rows, const h3_gpu_tensor *neg_text_in,
                    uint32_t neg_rows, float *latents, uint32_t gh,
                    uint32_t gw, uint32_t steps, float cfg_scale,
                    const double *turbo_sigmas, uint32_t turbo_count,
                    const qw_sched_cfg *sched, char *error,
                    size_t error_size);

#ifdef __cplusplus
}
#endif
#endif

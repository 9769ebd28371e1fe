/* h3_gpu — C-ABI GPU runtime of the qwen-metal DiT hot path on MI355X.
 *
 * Replaces the reference's Metal runtime h3_gpu.{h,m} for the DiT path:
 * same opaque handles, tensor calls, command-chain calls, error and stats
 * conventions (reference h3_gpu.h:7-112), implemented over HIP: tensors are
 * hipMalloc'd device buffers, the command chain is one hipStream_t, kernels
 * come from a gfx950 code object loaded with hipModuleLoad.
 *
 * Conventions kept from the reference:
 *   - every dispatch returns int (1 ok, 0 failure) and leaves the reason in
 *     h3_gpu_error(gpu); nothing aborts;
 *   - work is enqueued between h3_gpu_begin() and h3_gpu_submit(); submit
 *     waits for the chain and reports any device fault;
 *   - tensor reads/writes are synchronous with respect to queued work.
 * Dispatch entry points of the DiT path are declared here (h3_gpu_*) and in
 * qwen_gpu_ext.h (qw_gpu_*).
 */
#ifndef H3_GPU_H
#define H3_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct h3_gpu h3_gpu;
typedef struct h3_gpu_tensor h3_gpu_tensor;

/* reference h3_gpu.h:14-19 */
typedef enum {
    H3_GPU_F32 = 0,
    H3_GPU_BF16,
    H3_GPU_I8,
    H3_GPU_U32
} h3_gpu_dtype;

/* reference h3_gpu.h:21-37. mps_* counters stay zero (no MPSGraph here);
 * direct_dispatches counts kernel launches, gpu_seconds is the event-timed
 * duration of submitted chains. */
typedef struct {
    uint64_t allocated_bytes;
    uint64_t live_bytes;
    uint64_t peak_live_bytes;
    uint64_t tensor_allocations;
    uint64_t direct_dispatches;
    uint64_t mps_linear_dispatches;
    uint64_t mps_conv_dispatches;
    uint64_t mps_sdpa_dispatches;
    uint64_t blit_copies;
    uint64_t submissions;
    double command_encode_seconds;
    double command_wait_seconds;
    double gpu_seconds;
} h3_gpu_stats;

/* reference h3_gpu.h:39-40. The argument names the gfx950 code object
 * (qwen_kernels.hsaco) instead of a Metal shader source; NULL or "" loads
 * the one installed next to this library. Uses HIP device 0 unless
 * QW_HIP_DEVICE is set. */
h3_gpu *h3_gpu_create(const char *code_object_path, char *error,
                      size_t error_size);
void h3_gpu_free(h3_gpu *gpu);

/* reference h3_gpu.h:46-52 */
h3_gpu_tensor *h3_gpu_tensor_new_f32(h3_gpu *gpu, size_t elements);
h3_gpu_tensor *h3_gpu_tensor_new_bf16(h3_gpu *gpu, size_t elements);
h3_gpu_tensor *h3_gpu_tensor_new_i8(h3_gpu *gpu, size_t elements);
h3_gpu_tensor *h3_gpu_tensor_new_u32(h3_gpu *gpu, size_t elements);
/* reference h3_gpu.h:52-57 */
h3_gpu_tensor *h3_gpu_tensor_from_f32(h3_gpu *gpu, const float *values,
                                      size_t elements);
h3_gpu_tensor *h3_gpu_tensor_from_bf16(h3_gpu *gpu, const uint16_t *values,
                                       size_t elements);
h3_gpu_tensor *h3_gpu_tensor_from_u32(h3_gpu *gpu, const uint32_t *values,
                                      size_t elements);
/* Non-owning view of [offset, offset + elements) of a tensor (replaces the
 * reference's row-slice copies, qwen_dit.m:1384-1433). Free with
 * h3_gpu_tensor_free; the base must outlive the view. */
h3_gpu_tensor *h3_gpu_tensor_view(const h3_gpu_tensor *base, size_t offset,
                                  size_t elements);
/* reference h3_gpu.h:78-98 */
void h3_gpu_tensor_free(h3_gpu_tensor *tensor);
size_t h3_gpu_tensor_elements(const h3_gpu_tensor *tensor);
h3_gpu_dtype h3_gpu_tensor_dtype(const h3_gpu_tensor *tensor);
int h3_gpu_tensor_read_f32(const h3_gpu_tensor *tensor, float *values,
                           size_t elements);
int h3_gpu_tensor_read_f32_range(const h3_gpu_tensor *tensor,
                                 size_t source_offset, float *values,
                                 size_t elements);
int h3_gpu_tensor_read_bf16(const h3_gpu_tensor *tensor, uint16_t *values,
                            size_t elements);
int h3_gpu_tensor_write_f32(h3_gpu_tensor *tensor, const float *values,
                            size_t elements);
int h3_gpu_tensor_write_f32_range(h3_gpu_tensor *tensor,
                                  size_t destination_offset,
                                  const float *values, size_t elements);
int h3_gpu_tensor_write_bf16(h3_gpu_tensor *tensor, const uint16_t *values,
                             size_t elements);
int h3_gpu_tensor_write_bf16_range(h3_gpu_tensor *tensor,
                                   size_t destination_offset,
                                   const uint16_t *values, size_t elements);
/* Raw byte transfer for any dtype (i8 weights, u32 tables). */
int h3_gpu_tensor_read_bytes(const h3_gpu_tensor *tensor, void *bytes,
                             size_t byte_count);
int h3_gpu_tensor_write_bytes(h3_gpu_tensor *tensor, const void *bytes,
                              size_t byte_count);
/* Device address of the tensor's first element (for interop). */
void *h3_gpu_tensor_device_ptr(const h3_gpu_tensor *tensor);

/* reference h3_gpu.h:100-112 */
int h3_gpu_begin(h3_gpu *gpu);
int h3_gpu_continue(h3_gpu *gpu);
int h3_gpu_submit(h3_gpu *gpu);
const char *h3_gpu_error(const h3_gpu *gpu);
int h3_gpu_get_stats(const h3_gpu *gpu, h3_gpu_stats *stats);
void h3_gpu_profile_set_label(h3_gpu *gpu, const char *label);
void h3_gpu_profile_mark(h3_gpu *gpu, const char *phase);

/* Event timing on the runtime's stream (hipEventRecord pair): the elapsed
 * device time between timer_begin and timer_end, in milliseconds, or a
 * negative value on failure. timer_end waits for the end event. */
int h3_gpu_timer_begin(h3_gpu *gpu);
double h3_gpu_timer_end(h3_gpu *gpu);

/* ---- dispatch: DiT-path subset of the reference h3_gpu_* ops ----------- */
/* reference h3_gpu.h:295-299: Y = X W^T (+ bias), bf16 in/out, fp32 acc. */
int h3_gpu_linear_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                       const h3_gpu_tensor *input,
                       const h3_gpu_tensor *weight,
                       const h3_gpu_tensor *bias, uint32_t rows,
                       uint32_t input_dim, uint32_t output_dim);
/* reference h3_gpu.h:300-305: SwiGLU MLP, fc1 = [gate; up] [2*hidden, in],
 * fc2 [out, hidden]. */
int h3_gpu_mlp_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                    const h3_gpu_tensor *input,
                    const h3_gpu_tensor *fc1_weight,
                    const h3_gpu_tensor *fc2_weight, uint32_t rows,
                    uint32_t input_dim, uint32_t hidden_dim,
                    uint32_t output_dim);
/* reference h3_gpu.h:317-320 (kernel h3_shaders.metal:1320-1390, clip 1):
 * int8 [rows, columns] + fp32 scales [rows] from a bf16 weight. */
int h3_gpu_quantize_weight_int8(h3_gpu *gpu, h3_gpu_tensor *output,
                                h3_gpu_tensor *scales,
                                const h3_gpu_tensor *input, uint32_t rows,
                                uint32_t columns);
/* reference h3_gpu.h:358-359 */
int h3_gpu_silu_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                     const h3_gpu_tensor *input, uint32_t elements);
/* reference h3_gpu.h:369-371 (approximate must be 1: tanh form) */
int h3_gpu_gelu_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                     const h3_gpu_tensor *input, uint32_t elements,
                     int approximate);
/* reference h3_gpu.h:406-411 */
int h3_gpu_gate_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                     const h3_gpu_tensor *residual,
                     const h3_gpu_tensor *branch,
                     const h3_gpu_tensor *modulation,
                     const h3_gpu_tensor *row_map, uint32_t rows,
                     uint32_t width, uint32_t slots, uint32_t gate_slot);
/* reference h3_gpu.h:527-530 (head_dim 128) */
int h3_gpu_head_rms_norm_bf16(h3_gpu *gpu, h3_gpu_tensor *tensor,
                              const h3_gpu_tensor *weight,
                              uint32_t sequence, uint32_t heads,
                              uint32_t head_dim, float epsilon);
/* reference h3_gpu.h:537-542: causal self-attention (kv_heads == heads). */
int h3_gpu_gqa_causal_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                           const h3_gpu_tensor *query,
                           const h3_gpu_tensor *key,
                           const h3_gpu_tensor *value,
                           uint32_t sequence, uint32_t query_heads,
                           uint32_t kv_heads, uint32_t head_dim,
                           float scale);
/* reference h3_gpu.h:131-132 */
int h3_gpu_cast_f32_to_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                            const h3_gpu_tensor *input, uint32_t elements);
/* reference h3_gpu.h:135-138 */
int h3_gpu_copy_bf16(h3_gpu *gpu, h3_gpu_tensor *destination,
                     size_t destination_offset,
                     const h3_gpu_tensor *source, size_t source_offset,
                     size_t elements);

#ifdef __cplusplus
}
#endif
#endif

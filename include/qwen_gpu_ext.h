/* qwen_gpu_ext — DiT-path dispatch entry points (reference qwen_gpu_ext.h)
 * over the HIP runtime of h3_gpu.h, plus the fused MI355X entry points the
 * DiT host uses (declared after the reference-named ones).
 *
 * All activations are bf16 row-major [rows, features] with heads interleaved
 * as [row, head, 128]; RoPE tables are fp32 [rows, 64]; row_map is u32. */
#ifndef QWEN_GPU_EXT_H
#define QWEN_GPU_EXT_H

#include "h3_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference qwen_gpu_ext.h:11-16 (kernel h3_shaders.metal:4767-4815) */
int qw_gpu_layer_norm_mod_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                               const h3_gpu_tensor *input,
                               const h3_gpu_tensor *modulation,
                               const h3_gpu_tensor *row_map, uint32_t rows,
                               uint32_t width, uint32_t slots,
                               uint32_t scale_slot, float epsilon);
/* reference qwen_gpu_ext.h:19-22 (h3_shaders.metal:4817-4850) */
int qw_gpu_rms_norm_one_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                             const h3_gpu_tensor *input,
                             const h3_gpu_tensor *weight, uint32_t rows,
                             uint32_t width, float epsilon);
/* reference qwen_gpu_ext.h:25-26 */
int qw_gpu_tanh_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                     const h3_gpu_tensor *input, uint32_t elements);
/* reference qwen_gpu_ext.h:30-36 (h3_shaders.metal:4864-4896). In place
 * only (query_output == query_input, key_output == key_input). */
int qw_gpu_qk_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *query_output,
                        h3_gpu_tensor *key_output,
                        const h3_gpu_tensor *query_input,
                        const h3_gpu_tensor *key_input,
                        const h3_gpu_tensor *rope_cos,
                        const h3_gpu_tensor *rope_sin, uint32_t sequence,
                        uint32_t heads, uint32_t head_dim);
/* reference qwen_gpu_ext.h:65-67 (h3_shaders.metal:5078-5095) */
int qw_gpu_swiglu_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                       const h3_gpu_tensor *fc1, uint32_t rows,
                       uint32_t width);
/* reference qwen_gpu_ext.h:118-125: query rows against every key. */
int qw_gpu_flash_sdpa_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                           const h3_gpu_tensor *query,
                           const h3_gpu_tensor *key,
                           const h3_gpu_tensor *value, uint32_t q_rows,
                           uint32_t kv_rows, uint32_t heads,
                           uint32_t head_dim, float scale);
/* reference qwen_gpu_ext.h:131-138: per-row prefix limits (u32). Grouped
 * K/V heads are not on the DiT path: kv_heads must equal heads. */
int qw_gpu_flash_sdpa_prefix_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                                  const h3_gpu_tensor *query,
                                  const h3_gpu_tensor *key,
                                  const h3_gpu_tensor *value,
                                  const h3_gpu_tensor *kv_limit,
                                  uint32_t q_rows, uint32_t kv_rows,
                                  uint32_t heads, uint32_t kv_heads,
                                  uint32_t head_dim, float scale);
/* reference qwen_gpu_ext.h:204-210: q/k/v = X W_{q,k,v}^T, three outputs. */
int qw_gpu_qkv_bf16(h3_gpu *gpu, h3_gpu_tensor *query_out,
                    h3_gpu_tensor *key_out, h3_gpu_tensor *value_out,
                    const h3_gpu_tensor *input,
                    const h3_gpu_tensor *query_weight,
                    const h3_gpu_tensor *key_weight,
                    const h3_gpu_tensor *value_weight, uint32_t rows,
                    uint32_t dim);
/* reference qwen_gpu_ext.h:223-228: image rows against the full prefix. */
int qw_gpu_sdpa_rect_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                          const h3_gpu_tensor *query,
                          const h3_gpu_tensor *key,
                          const h3_gpu_tensor *value,
                          uint32_t query_sequence, uint32_t kv_sequence,
                          uint32_t heads, uint32_t head_dim, float scale);

/* ---- MI355X fused entry points (no reference counterpart) ------------- */

/* Shift-variant LayerNorm modulation: LN(x) * (1 + scale) + shift.
 * shift_slot < 0 disables the shift (then identical to the call above). */
int qw_gpu_layer_norm_mod_shift_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                                     const h3_gpu_tensor *input,
                                     const h3_gpu_tensor *modulation,
                                     const h3_gpu_tensor *row_map,
                                     uint32_t rows, uint32_t width,
                                     uint32_t slots, uint32_t scale_slot,
                                     int32_t shift_slot, float epsilon);

enum { QW_LINEAR_STORE = 0, QW_LINEAR_GELU = 1, QW_LINEAR_GATE = 2, QW_LINEAR_QKNORM = 3 };

/* One GEMM with a fused epilogue, on sub-ranges of tensors:
 *   y = bf16( X W^T * wscale + bias )                  (STORE)
 *   y = bf16( gelu_tanh( bf16(X W^T * wscale + bias) ) ) (GELU)
 *   out = bf16( out + bf16(X W^T * wscale + bias) * gate ) (GATE, in place;
 *         gate row = row_map[r], columns gate_slot*cols..)
 *   y, then per-head RMS norm + RoPE on the q and k thirds (QKNORM)
 * weight is bf16 [cols, k] or int8 [cols, k] (then wscale f32 [cols] is
 * required; without wscale a bf16 weight is unscaled). Offsets/strides are
 * in elements; k must be a multiple of 64. An int8 weight is widened to
 * bf16 inside the GEMM, once per workgroup into LDS, with the scale in the
 * epilogue. Where that measured slower (512 or more rows, k < 8192) the
 * weight is first widened to a bf16 copy (qw_gpu_widen_int8_bf16, into a
 * buffer the runtime keeps) and the bf16 GEMM runs: the same sums, the
 * same single rounding, the same bits. */
typedef struct {
    h3_gpu_tensor *out;
    size_t out_offset;
    uint32_t ldc;
    const h3_gpu_tensor *in;
    size_t in_offset;
    uint32_t lda;
    const h3_gpu_tensor *weight;
    const h3_gpu_tensor *wscale;
    const h3_gpu_tensor *bias;
    uint32_t rows, k, cols;
    int epilogue;
    const h3_gpu_tensor *modulation; /* GATE */
    const h3_gpu_tensor *row_map;    /* GATE */
    uint32_t slots, gate_slot;       /* GATE: row stride slots*cols */
    /* QKNORM: the fused q|k|v projection (cols = 3 heads 128, out_offset 0)
     * with qw_gpu_qk_norm_rope_bf16 applied to its q and k columns in the
     * epilogue (same result as the two calls); the RoPE table row is
     * row % rope_rows */
    const h3_gpu_tensor *norm_q, *norm_k, *rope_cos, *rope_sin;
    uint32_t rope_rows;
    float eps;
} qw_linear_desc;
int qw_gpu_linear(h3_gpu *gpu, const qw_linear_desc *desc);
/* No counterpart in the reference. For callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): qw_gpu_linear with every workspace in
 * one static per-GPU device buffer of 32 MiB + 4 KiB, held until the
 * process ends. It calls no hipMalloc / hipFree. int8 weights are always
 * widened inside the GEMM (no bf16 staging copy); split tiles are used only as
 * far as their fp32 partials fit the buffer (at most 128 pieces), so long-K
 * linears may split less than qw_gpu_linear does (same bar: within one
 * bf16 ulp of it, or of its cancellation bound). Calls on one GPU share
 * that buffer, whichever h3_gpu context or stream they come from: each call
 * makes its stream wait for the previous call's kernels (a per-device event)
 * and records its own, so calls issued one after another never overlap on
 * the buffer (a stream under graph capture skips that wait: the captured
 * graph's order is the caller's). The buffer keeps the last call's
 * contents. */
int qw_gpu_linear_static(h3_gpu *gpu, const qw_linear_desc *desc);

/* No counterpart in the reference (a measurement aid, like h3_gpu_timer_*):
 * spans time pieces of the work on the stream without synchronising it.
 * span_begin records an event tagged `tag`, span_end the matching end
 * event; spans do not nest. span_collect waits for the last span, writes
 * up to max (tag, device ms) pairs, forgets all spans and returns how many
 * it wrote, or -1 on error. At most 4096 spans between collects. */
int qw_gpu_span_begin(h3_gpu *gpu, int tag);
int qw_gpu_span_end(h3_gpu *gpu);
int qw_gpu_span_collect(h3_gpu *gpu, int *tags, double *ms, int max);

/* Fused per-head RMSNorm (single rounding, h3_shaders.metal:4309-4329) and
 * interleaved RoPE (h3_shaders.metal:4864-4896) over q and k in one
 * strided buffer [rows, ld]: q heads at column 0, k heads at k_offset.
 * Table row = row % rope_rows. norm_q/norm_k NULL skips the norm; rope NULL
 * skips the rotation. In place. */
int qw_gpu_qk_norm_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *qk, uint32_t rows,
                             uint32_t heads, uint32_t ld, uint32_t k_offset,
                             const h3_gpu_tensor *norm_q,
                             const h3_gpu_tensor *norm_k,
                             const h3_gpu_tensor *rope_cos,
                             const h3_gpu_tensor *rope_sin,
                             uint32_t rope_rows, float epsilon);

/* Batched block-causal flash attention over strided q/k/v views (e.g. the
 * fused [rows, 3H] projection): batch entries of q_rows queries / kv_rows
 * keys stacked along rows. kv_limit (u32 [q_rows], shared by the batch)
 * overrides the t2i closed form (text rows causal or full-prefix, image
 * rows all keys). */
typedef struct {
    h3_gpu_tensor *out;
    size_t out_offset;
    uint32_t ldo;
    const h3_gpu_tensor *q, *k, *v;
    size_t q_offset, k_offset, v_offset;
    uint32_t ldq, ldk, ldv;
    const h3_gpu_tensor *kv_limit;
    uint32_t batch, q_rows, kv_rows, heads;
    uint32_t text_rows;
    int text_causal;
    float scale;
} qw_attention_desc;
int qw_gpu_attention_bf16(h3_gpu *gpu, const qw_attention_desc *desc);

/* qwen_dit.m:1159-1186 on device: raw modulation [mod_rows, S*hidden] ->
 * slot layout with tanh'd gates stored by truncation. S = 4, or 6 when
 * shift_variant (then slots 4, 5 carry the shifts). */
int qw_gpu_modulation_reorder_bf16(h3_gpu *gpu, h3_gpu_tensor *slots_out,
                                   const h3_gpu_tensor *raw,
                                   uint32_t mod_rows, uint32_t hidden,
                                   int shift_variant);

/* Seeded synthetic values: bf16(std * z + offset), z from the counter-based
 * generator keyed by (seed, stream, index) — bit-identical to the host
 * restatement used by the tests. Fills [offset_elems, +count). */
int qw_gpu_fill_normal_bf16(h3_gpu *gpu, h3_gpu_tensor *tensor,
                            size_t offset_elems, size_t count, uint64_t seed,
                            uint64_t stream, float std, float offset);

/* Dequantised int8 weight q * scale as fp32 [rows, cols]. */
int qw_gpu_dequant_int8_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                            const h3_gpu_tensor *q,
                            const h3_gpu_tensor *scales, uint32_t rows,
                            uint32_t cols);

/* out[i] = bf16(q[i]) for count int8 values (count % 16 == 0): the exact,
 * unscaled widening used ahead of the bf16 GEMM. No counterpart in the
 * reference (whose int8 path is h3_shaders.metal:1320-1390 + in-kernel
 * dequant); exported so callers can keep widened weights resident. */
int qw_gpu_widen_int8_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                           const h3_gpu_tensor *q, size_t count);

/* One step of the denoise loop on device-resident fp32 latents x[count]:
 * v = neg ? n + cfg (p - n) : p with p = pos[pos_offset + i],
 * n = neg[neg_offset + i] (bf16 predictions of the image rows), then
 * x += dt v; fp32, same operations and rounding points as the host loop
 * (qwen_pipeline.m:421-429, qw_euler_velocity_step qwen_host.c:372-378).
 * neg may be NULL (no guidance). */
int qw_gpu_cfg_euler_f32(h3_gpu *gpu, h3_gpu_tensor *x, const h3_gpu_tensor *pos,
                         size_t pos_offset, const h3_gpu_tensor *neg,
                         size_t neg_offset, size_t count, float dt, float cfg);

#define QW_GPU_LORA_MAX_RANK 256
#define QW_GPU_LORA_MAX_TERMS 24
/* LoRA weight fusion (qwen_dit.m:535-1010):
 *   out = RNE_bf16(fp32(base) + sum_t scale_t * (B_t @ A_t))
 * base, out bf16 [rows, cols] (may not alias); term t adds to fused rows
 * [row0, row0 + rows) with A bf16 [rank, cols] and B bf16 [rows, rank],
 * rank <= 256, at most 24 terms, applied in order with one final rounding.
 * No counterpart in the reference (which fuses on the host). */
typedef struct {
    const h3_gpu_tensor *a, *b;
    uint32_t row0, rows, rank;
    float scale;
} qw_lora_term_desc;
int qw_gpu_lora_fuse_bf16(h3_gpu *gpu, h3_gpu_tensor *out,
                          const h3_gpu_tensor *base, uint32_t rows,
                          uint32_t cols, const qw_lora_term_desc *terms,
                          uint32_t nterms);

/* Strided row copy: rows x row_elems of dtype-size elements. */
int qw_gpu_copy_rows(h3_gpu *gpu, h3_gpu_tensor *dst, size_t dst_offset,
                     uint32_t dst_stride, const h3_gpu_tensor *src,
                     size_t src_offset, uint32_t src_stride, uint32_t rows,
                     uint32_t row_elems);

#ifdef __cplusplus
}
#endif
#endif

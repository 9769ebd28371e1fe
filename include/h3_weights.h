/* Component weight store over a directory of safetensors shards (reference
 * h3_weights.h:10-33): every *.safetensors header is read when the store
 * opens; payloads are read on demand straight into device tensors. */
#ifndef H3_WEIGHTS_H
#define H3_WEIGHTS_H

#include "h3_gpu.h"
#include "h3_safetensors.h"

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct h3_weight_store h3_weight_store;

/* reference h3_weights.h:14-15: shards in name order; fails on a directory
 * with none, on an unreadable shard and on a tensor name that appears in
 * two shards */
h3_weight_store *h3_weight_store_open(const char *directory, char *error,
                                      size_t error_size);
/* reference h3_weights.h:16-17 */
void h3_weight_store_free(h3_weight_store *store);
size_t h3_weight_store_shards(const h3_weight_store *store);
/* reference h3_weights.h:19-21: the tensor and (optionally) its shard */
const h3_st_tensor *h3_weight_find(const h3_weight_store *store,
                                   const char *name,
                                   const h3_st_header **header);
/* reference h3_weights.h:25-32: exact dtype and shape check, then the
 * payload is read in bounded host chunks into a new device tensor */
h3_gpu_tensor *h3_weight_load_bf16(const h3_weight_store *store, h3_gpu *gpu,
                                   const char *name, int ndim,
                                   const uint64_t *shape, char *error,
                                   size_t error_size);
h3_gpu_tensor *h3_weight_load_f32(const h3_weight_store *store, h3_gpu *gpu,
                                  const char *name, int ndim,
                                  const uint64_t *shape, char *error,
                                  size_t error_size);

/* The same checks, reading a BF16 tensor into elements
 * [offset, offset + elements) of an existing bf16 tensor (used to assemble
 * fused weights such as [q; k; v]). No counterpart in the reference. */
int h3_weight_read_bf16_into(const h3_weight_store *store, const char *name,
                             int ndim, const uint64_t *shape,
                             h3_gpu_tensor *dst, size_t offset, char *error,
                             size_t error_size);

#ifdef __cplusplus
}
#endif

#endif

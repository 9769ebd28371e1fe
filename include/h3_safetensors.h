/* Safetensors headers and payload reads, the subset of the reference's
 * h3_safetensors.h (h3_safetensors.h:9-53) that the DiT weight loader and
 * adapter tools use. Same type layouts and entry points; the directory
 * inventory (h3_st_inventory_dir) belongs to the reference's model-info
 * tool and is not part of this build. */
#ifndef H3_SAFETENSORS_H
#define H3_SAFETENSORS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference h3_safetensors.h:9-24 */
typedef enum {
    H3_DTYPE_UNKNOWN = 0,
    H3_DTYPE_BOOL,
    H3_DTYPE_I8,
    H3_DTYPE_U8,
    H3_DTYPE_I16,
    H3_DTYPE_U16,
    H3_DTYPE_F16,
    H3_DTYPE_BF16,
    H3_DTYPE_I32,
    H3_DTYPE_U32,
    H3_DTYPE_F32,
    H3_DTYPE_I64,
    H3_DTYPE_U64,
    H3_DTYPE_F64
} h3_dtype;

/* reference h3_safetensors.h:26-34. data_begin/data_end are the header's
 * data_offsets (relative to the payload); file_offset is absolute. */
typedef struct {
    char *name;
    h3_dtype dtype;
    int ndim;
    uint64_t shape[8];
    uint64_t data_begin;
    uint64_t data_end;
    uint64_t file_offset;
} h3_st_tensor;

/* reference h3_safetensors.h:36-42 */
typedef struct {
    char *path;
    uint64_t file_size;
    uint64_t header_size;
    h3_st_tensor *tensors;
    size_t tensor_count;
} h3_st_header;

/* reference h3_safetensors.h:44-45. Reads and validates the JSON header
 * only (no payload): 8-byte little-endian header length (<= 256 MiB), then
 * one object per tensor with dtype, shape (<= 8 dims) and data_offsets;
 * "__metadata__" is skipped. Rejects unknown dtypes, duplicate names,
 * offsets outside the payload and byte ranges that do not match the shape.
 * Returns 1, or 0 with the reason in error. */
int h3_st_read_header(const char *path, h3_st_header *header, char *error,
                      size_t error_size);
/* reference h3_safetensors.h:46 */
void h3_st_free_header(h3_st_header *header);
/* reference h3_safetensors.h:47: NULL when absent */
const h3_st_tensor *h3_st_find(const h3_st_header *header, const char *name);
/* reference h3_safetensors.h:48: product of the shape (1 for a scalar) */
uint64_t h3_st_tensor_elements(const h3_st_tensor *tensor);
/* reference h3_safetensors.h:49-50: reads exactly the tensor's bytes;
 * bytes must equal data_end - data_begin */
int h3_st_read_data(const h3_st_header *header, const h3_st_tensor *tensor,
                    void *data, size_t bytes, char *error, size_t error_size);
/* reference h3_safetensors.h:51-52 */
size_t h3_dtype_size(h3_dtype dtype);
const char *h3_dtype_name(h3_dtype dtype);

#ifdef __cplusplus
}
#endif

#endif

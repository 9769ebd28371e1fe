/* One fixed device workspace per GPU for the entry points that allocate
 * nothing (qw_gpu_linear_static): split-tile fp32 partials followed by the
 * split tiles' piece counters. Internal to the library. */
#pragma once
#include <stddef.h>

#include <hip/hip_runtime.h>

/* QW_STATIC_PARTS partials of one 256 x 256 fp32 tile (256 KiB each), then
 * QW_STATIC_FLAGS u32 counters: 32 MiB + 4 KiB per GPU, held until the
 * process ends. */
#define QW_STATIC_PARTS 128u
#define QW_STATIC_PART_BYTES (256u * 256u * 4u)
#define QW_STATIC_FLAGS 1024u
#define QW_STATIC_SCRATCH_BYTES \
    ((size_t)QW_STATIC_PARTS * QW_STATIC_PART_BYTES + (size_t)QW_STATIC_FLAGS * 4u)

#ifdef __cplusplus
extern "C" {
#endif
/* Device address of this GPU's copy of the static workspace: resolved with
 * hipGetSymbolAddress on the first call for `device` (which must be the
 * current device) and cached per device. 0 on success, else a HIP error
 * code with a message in err. */
int qw_static_scratch_address(int device, void **address, char *err, size_t err_size);
/* Ordering of the workspace's users on one device, whatever context or
 * stream they come from: acquire makes `stream` wait for the last call that
 * used the workspace (an event recorded by release) and holds a per-device
 * lock until release records this call's end on `stream`. Every call that
 * launches kernels on the workspace runs between the two. 0 on success,
 * else a HIP error code (acquire then holds nothing). */
int qw_static_scratch_acquire(int device, hipStream_t stream);
int qw_static_scratch_release(int device, hipStream_t stream);
#ifdef __cplusplus
}
#endif

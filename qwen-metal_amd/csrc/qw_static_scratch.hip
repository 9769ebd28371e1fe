/* The static device workspace of the no-allocation entry points. The
 * array lives in this library's own (registered) device code; each GPU the
 * library runs on holds its own copy at its own address, which is looked
 * up once per device. Host code uses only that address: the array's name
 * in host code is a host-side stand-in, never a device pointer. */
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdio.h>

#include "qw_static_scratch.h"

static __device__ __align__(256) unsigned char scratch[QW_STATIC_SCRATCH_BYTES];

#define QW_STATIC_MAX_DEVICES 64
static void *scratch_ptr[QW_STATIC_MAX_DEVICES];
static std::mutex scratch_lock;

extern "C" __attribute__((visibility("hidden"))) int qw_static_scratch_address(int device, void **address, char *err,
                                         size_t err_size) {
    if (device < 0 || device >= QW_STATIC_MAX_DEVICES) {
        snprintf(err, err_size, "static scratch: device %d out of range", device);
        return (int)hipErrorInvalidDevice;
    }
    std::lock_guard<std::mutex> hold(scratch_lock);
    if (!scratch_ptr[device]) {
        void *p = NULL;
        const hipError_t e = hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            snprintf(err, err_size, "static scratch: hipGetSymbolAddress on device %d: %s",
                     device, hipGetErrorString(e));
            return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
        }
        scratch_ptr[device] = p;
    }
    *address = scratch_ptr[device];
    return 0;
}

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
/* per device: the event recorded after the last call that used the
 * workspace, and the lock held from a call's wait on it to its new record */
static hipEvent_t scratch_done[QW_STATIC_MAX_DEVICES];
static std::mutex scratch_use[QW_STATIC_MAX_DEVICES];
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
        hipEvent_t ev = NULL;
        const hipError_t ee = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (ee != hipSuccess) {
            snprintf(err, err_size, "static scratch: event on device %d: %s", device,
                     hipGetErrorString(ee));
            return (int)ee;
        }
        scratch_done[device] = ev;
        scratch_ptr[device] = p;
    }
    *address = scratch_ptr[device];
    return 0;
}

extern "C" __attribute__((visibility("hidden"))) int qw_static_scratch_acquire(int device,
                                                                           hipStream_t stream) {
    if (device < 0 || device >= QW_STATIC_MAX_DEVICES || !scratch_done[device])
        return (int)hipErrorInvalidDevice;
    scratch_use[device].lock();
    /* a stream under graph capture cannot wait on an event recorded outside
     * it: its graph's order is the caller's to set */
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(stream, &cs);
    if (e == hipSuccess && cs == hipStreamCaptureStatusNone)
        e = hipStreamWaitEvent(stream, scratch_done[device], 0);
    if (e != hipSuccess) scratch_use[device].unlock();
    return (int)e;
}

extern "C" __attribute__((visibility("hidden"))) int qw_static_scratch_release(int device,
                                                                           hipStream_t stream) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(stream, &cs);
    if (e == hipSuccess && cs == hipStreamCaptureStatusNone)
        e = hipEventRecord(scratch_done[device], stream);
    scratch_use[device].unlock();
    return (int)e;
}

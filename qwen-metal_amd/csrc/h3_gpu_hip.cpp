/* h3_gpu over HIP: device, one stream, hipModule-loaded gfx950 kernels,
 * hipMalloc'd tensors, and the host-side launch/validation of every DiT
 * dispatch. The reference's Metal runtime is h3_gpu.m; the conventions
 * (int return, error string, begin/submit chain, stats) follow
 * h3_gpu.h:7-112 of the reference. Every launch checks operand sizes on the
 * host first, so a bad call fails with an error string instead of faulting
 * the device. */
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <string>

#include "../../include/h3_gpu.h"
#include "../../include/qwen_gpu_ext.h"
#include <algorithm>

#include "qw_kernel_args.h"
#include "qw_static_scratch.h"

enum {
    K_LN_MOD, K_RMS_ONE, K_QK_NORM_ROPE, K_GATE, K_ACT, K_SWIGLU, K_CAST,
    K_REORDER, K_FILL, K_QUANT, K_DEQUANT, K_COPY2D, K_ATTN,
    /* GEMM kernels in QW_LINEAR_* epilogue order (store, gelu, gate, qknorm) */
    K_GEMM_BF16_STORE_Q, K_GEMM_BF16_GELU_Q, K_GEMM_BF16_GATE_Q, K_GEMM_BF16_QKN_Q,
    K_WIDEN, K_LN_MOD_WIDE, K_EULER, K_LORA,
    K_GEMV_BF16_STORE, K_GEMV_BF16_GELU, K_GEMV_I8_STORE, K_GEMV_I8_GELU, K_ZERO,
    K_GEMM_W8_STORE_Q, K_GEMM_W8_GELU_Q, K_GEMM_W8_GATE_Q, K_GEMM_W8_QKN_Q,
    K_GEMM_BF16_STORE_T224, K_GEMM_BF16_GELU_T224, K_GEMM_BF16_GATE_T224, K_GEMM_BF16_QKN_T224,
    K_GEMM_BF16_STORE_H3, K_GEMM_BF16_GELU_H3, K_GEMM_BF16_GATE_H3, K_GEMM_BF16_QKN_H3,
    K_ATTN_W4,
    K_COUNT
};
static const char *k_names[K_COUNT] = {
    "qw_layer_norm_mod_bf16", "qw_rms_norm_one_bf16", "qw_qk_norm_rope_bf16",
    "qw_gate_bf16", "qw_act_bf16", "qw_swiglu_bf16", "qw_cast_f32_bf16",
    "qw_modulation_reorder_bf16", "qw_fill_normal_bf16", "qw_quantize_int8_rows",
    "qw_dequant_int8_f32", "qw_copy2d", "qw_attention_bf16",
    "qw_gemm_bf16_store_q", "qw_gemm_bf16_gelu_q", "qw_gemm_bf16_gate_q", "qw_gemm_bf16_qkn_q",
    "qw_widen_i8_bf16",
    "qw_layer_norm_mod_wide_bf16", "qw_cfg_euler_f32", "qw_lora_fuse_bf16",
    "qw_gemv_bf16_store", "qw_gemv_bf16_gelu", "qw_gemv_i8_store", "qw_gemv_i8_gelu",
    "qw_zero_u32",
    "qw_gemm_w8_store_q", "qw_gemm_w8_gelu_q", "qw_gemm_w8_gate_q", "qw_gemm_w8_qkn_q",
    "qw_gemm_bf16_store_t224", "qw_gemm_bf16_gelu_t224", "qw_gemm_bf16_gate_t224",
    "qw_gemm_bf16_qkn_t224",
    "qw_gemm_bf16_store_h3", "qw_gemm_bf16_gelu_h3", "qw_gemm_bf16_gate_h3",
    "qw_gemm_bf16_qkn_h3", "qw_attention_w4_bf16"};

/* How int8 linears run (QW_INT8_ROUTE, a measurement switch): AUTO (the
 * default) widens the weight to a bf16 copy and runs the bf16 kernels when
 * that measured faster -- 512+ rows and K < 8192 -- and otherwise runs the
 * int8 kernels that widen each W tile once per workgroup in LDS; WIDEN and
 * W8 force one route wherever it can run. */
enum { QW_INT8_AUTO = 0, QW_INT8_WIDEN = 1, QW_INT8_W8 = 2 };

#define QW_SPAN_MAX 4096

/* below this many rows an int8 linear widens inside its GEMM, unless the
 * launch is small enough for half tiles (linear_impl) */
#define QW_WIDEN_MIN_ROWS 512

struct h3_gpu {
    int device;
    hipStream_t stream;
    hipModule_t module;
    hipFunction_t fn[K_COUNT];
    char error[1024];
    h3_gpu_stats stats;
    hipEvent_t timer0, timer1;
    hipEvent_t chain0, chain1;
    int chain_open;
    std::string label;
    void *scratch;
    size_t scratch_bytes;
    uint32_t attn_threads;  /* attention workgroup size, 64 per 32-query wave */
    uint32_t attn4_threads; /* the same for the small launches' kernel */
    int attn_small; /* launches of fewer 256-query blocks than CUs on the 4-wave kernel (QW_ATTN_W4=0: off) */
    int int8_route; /* QW_INT8_* : how int8 linears of many rows run */
    int t224;       /* 224-row tiles allowed (QW_GEMM_T224=0 turns them off, for measurement) */
    uint32_t split_min_steps, split_force; /* measurement: QW_SPLIT_MIN_STEPS, QW_SPLIT_FORCE */
    uint32_t split_small_min; /* shortest piece of a small launch (QW_SPLIT_SMALL_MIN_STEPS) */
    int half3;      /* small launches' half tiles on the three-stage kernels (QW_GEMM_HALF3=0: two) */
    uint32_t widen_min_rows; /* int8: fewest rows for the widening route (QW_WIDEN_MIN_ROWS) */
    int t224_over_split; /* 224-row tiles preferred to split tiles (QW_T224_OVER_SPLIT=0: off) */
    int half_small; /* launches of at most cus / 2 tiles as half tiles (QW_GEMM_HALF_SMALL=0: off) */
    /* qw_gpu_span_*: event pairs recorded on the stream, read after a sync */
    hipEvent_t *span_ev;
    int *span_tag;
    int span_n, span_open;
    void *widen; /* bf16 copy of the int8 weight of the linear in flight */
    size_t widen_bytes;
    uint32_t cus;      /* compute units */
    float *sk_part;    /* split-tile partials: 256 x 256 fp32 each */
    uint32_t *sk_flag; /* split-tile piece counters, 0 between launches */
    /* this device's copy of the static workspace (qw_static_scratch.hip):
     * partials, then QW_STATIC_FLAGS counters */
    unsigned char *static_scratch;
};

struct h3_gpu_tensor {
    h3_gpu *gpu;
    unsigned char *ptr;
    size_t elements;
    h3_gpu_dtype dtype;
    int owns;
};

static size_t dtype_size(h3_gpu_dtype d) {
    return d == H3_GPU_BF16 ? 2 : d == H3_GPU_I8 ? 1 : 4;
}

static int fail(h3_gpu *g, const char *fmt, ...) {
    if (g) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(g->error, sizeof(g->error), fmt, ap);
        va_end(ap);
    }
    return 0;
}

static void set_err(char *error, size_t n, const char *fmt, ...) {
    if (!error || !n) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(error, n, fmt, ap);
    va_end(ap);
}

static double now_s() {
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

/* ---------------------------------------------------------------------- */
/* context                                                                */

extern "C" h3_gpu *h3_gpu_create(const char *code_object_path, char *error,
                                 size_t error_size) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        set_err(error, error_size, "no HIP device available");
        return NULL;
    }
    const char *dev_env = getenv("QW_HIP_DEVICE");
    int device = dev_env && *dev_env ? atoi(dev_env) : 0;
    if (device < 0 || device >= count) {
        set_err(error, error_size, "QW_HIP_DEVICE=%d out of range (%d devices)", device, count);
        return NULL;
    }
    if (hipSetDevice(device) != hipSuccess) {
        set_err(error, error_size, "hipSetDevice(%d) failed", device);
        return NULL;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        set_err(error, error_size, "hipGetDeviceProperties failed");
        return NULL;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_err(error, error_size, "device %d is %s; this code object is gfx950 only",
                device, prop.gcnArchName);
        return NULL;
    }
    std::string path;
    if (code_object_path && *code_object_path) {
        path = code_object_path;
    } else {
        Dl_info info;
        if (!dladdr((void *)&h3_gpu_create, &info) || !info.dli_fname) {
            set_err(error, error_size, "cannot locate libqwen_dit_hip.so");
            return NULL;
        }
        path = info.dli_fname;
        size_t slash = path.rfind('/');
        path = (slash == std::string::npos ? std::string(".") : path.substr(0, slash)) +
               "/qwen_kernels.hsaco";
    }
    h3_gpu *g = new h3_gpu();
    memset(g->error, 0, sizeof(g->error));
    memset(&g->stats, 0, sizeof(g->stats));
    g->device = device;
    g->chain_open = 0;
    g->scratch = NULL;
    g->scratch_bytes = 0;
    g->widen = NULL;
    g->widen_bytes = 0;
    g->span_ev = NULL;
    g->span_tag = NULL;
    g->span_n = 0;
    g->span_open = 0;
    g->int8_route = QW_INT8_AUTO;
    if (const char *r = getenv("QW_INT8_ROUTE")) {
        if (!strcmp(r, "w8")) g->int8_route = QW_INT8_W8;
        else if (!strcmp(r, "widen")) g->int8_route = QW_INT8_WIDEN;
    }
    g->t224 = 1;
    if (const char *r = getenv("QW_GEMM_T224")) g->t224 = atoi(r) != 0;
    g->split_min_steps = 32;
    if (const char *r = getenv("QW_SPLIT_MIN_STEPS")) g->split_min_steps = (uint32_t)atoi(r);
    g->split_small_min = 16;
    if (const char *r = getenv("QW_SPLIT_SMALL_MIN_STEPS")) g->split_small_min = (uint32_t)atoi(r);
    g->split_force = 0;
    if (const char *r = getenv("QW_SPLIT_FORCE")) g->split_force = (uint32_t)atoi(r);
    g->half3 = 1;
    if (const char *r = getenv("QW_GEMM_HALF3")) g->half3 = atoi(r) != 0;
    g->widen_min_rows = QW_WIDEN_MIN_ROWS;
    if (const char *r = getenv("QW_WIDEN_MIN_ROWS")) g->widen_min_rows = (uint32_t)atoi(r);
    g->t224_over_split = 1;
    if (const char *r = getenv("QW_T224_OVER_SPLIT")) g->t224_over_split = atoi(r) != 0;
    g->half_small = 1;
    if (const char *r = getenv("QW_GEMM_HALF_SMALL")) g->half_small = atoi(r) != 0;
    g->cus = 0;
    g->sk_part = NULL;
    g->sk_flag = NULL;
    g->static_scratch = NULL;
    hipError_t e = hipModuleLoad(&g->module, path.c_str());
    if (e != hipSuccess) {
        set_err(error, error_size, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e));
        delete g;
        return NULL;
    }
    for (int k = 0; k < K_COUNT; k++) {
        e = hipModuleGetFunction(&g->fn[k], g->module, k_names[k]);
        if (e != hipSuccess) {
            set_err(error, error_size, "kernel %s missing from %s", k_names[k], path.c_str());
            hipModuleUnload(g->module);
            delete g;
            return NULL;
        }
    }
    /* The attention kernels' workgroups (their launch bounds) set the query
     * blocks: one 64-lane wave per 32 queries. */
    for (int w = 0; w < 2; w++) {
        const int kid = w ? K_ATTN_W4 : K_ATTN;
        int attn_threads = 0;
        e = hipFuncGetAttribute(&attn_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, g->fn[kid]);
        if (e != hipSuccess || attn_threads < 64 || attn_threads > 1024 || attn_threads % 64) {
            set_err(error, error_size, "%s: bad workgroup bound %d", k_names[kid], attn_threads);
            hipModuleUnload(g->module);
            delete g;
            return NULL;
        }
        (w ? g->attn4_threads : g->attn_threads) = (uint32_t)attn_threads;
    }
    g->attn_small = 1;
    if (const char *r = getenv("QW_ATTN_W4")) g->attn_small = atoi(r) != 0;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, g->device) != hipSuccess ||
        cus <= 0) {
        set_err(error, error_size, "compute unit count unavailable");
        hipModuleUnload(g->module);
        delete g;
        return NULL;
    }
    g->cus = (uint32_t)cus;
    {
        /* once per device, with the device current: the address of its
         * copy of the no-allocation entry points' static workspace */
        void *ss = NULL;
        char se[256] = {0};
        if (qw_static_scratch_address(device, &ss, se, sizeof(se)) != 0) {
            set_err(error, error_size, "%s", se);
            hipModuleUnload(g->module);
            delete g;
            return NULL;
        }
        g->static_scratch = (unsigned char *)ss;
    }
    if (hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&g->timer0) != hipSuccess || hipEventCreate(&g->timer1) != hipSuccess ||
        hipEventCreate(&g->chain0) != hipSuccess || hipEventCreate(&g->chain1) != hipSuccess) {
        set_err(error, error_size, "stream/event creation failed");
        hipModuleUnload(g->module);
        delete g;
        return NULL;
    }
    return g;
}

extern "C" void h3_gpu_free(h3_gpu *g) {
    if (!g) return;
    hipSetDevice(g->device);
    hipStreamSynchronize(g->stream);
    if (g->scratch) hipFree(g->scratch);
    if (g->widen) hipFree(g->widen);
    if (g->sk_part) hipFree(g->sk_part);
    if (g->sk_flag) hipFree(g->sk_flag);
    if (g->span_ev) {
        for (int i = 0; i < 2 * QW_SPAN_MAX; i++) hipEventDestroy(g->span_ev[i]);
        free(g->span_ev);
        free(g->span_tag);
    }
    hipEventDestroy(g->timer0);
    hipEventDestroy(g->timer1);
    hipEventDestroy(g->chain0);
    hipEventDestroy(g->chain1);
    hipStreamDestroy(g->stream);
    hipModuleUnload(g->module);
    delete g;
}

extern "C" const char *h3_gpu_error(const h3_gpu *g) { return g ? g->error : "no gpu"; }

extern "C" int h3_gpu_get_stats(const h3_gpu *g, h3_gpu_stats *s) {
    if (!g || !s) return 0;
    *s = g->stats;
    return 1;
}

extern "C" void h3_gpu_profile_set_label(h3_gpu *g, const char *label) {
    if (g) g->label = label ? label : "";
}

extern "C" void h3_gpu_profile_mark(h3_gpu *g, const char *phase) {
    if (!g || !getenv("H3_PROFILE")) return;
    hipStreamSynchronize(g->stream);
    fprintf(stderr, "[h3-profile] %s %s: dispatches=%llu submissions=%llu live=%.1f MB\n",
            g->label.c_str(), phase ? phase : "", (unsigned long long)g->stats.direct_dispatches,
            (unsigned long long)g->stats.submissions, g->stats.live_bytes / 1e6);
}

extern "C" int h3_gpu_begin(h3_gpu *g) {
    if (!g) return 0;
    if (!g->chain_open) {
        hipEventRecord(g->chain0, g->stream);
        g->chain_open = 1;
    }
    return 1;
}

extern "C" int h3_gpu_continue(h3_gpu *g) {
    /* HIP streams are already asynchronous and ordered: nothing to commit. */
    return g ? 1 : 0;
}

extern "C" int h3_gpu_submit(h3_gpu *g) {
    if (!g) return 0;
    double t0 = now_s();
    if (g->chain_open) hipEventRecord(g->chain1, g->stream);
    hipError_t e = hipStreamSynchronize(g->stream);
    g->stats.command_wait_seconds += now_s() - t0;
    g->stats.submissions++;
    if (e == hipSuccess) e = hipGetLastError();
    if (g->chain_open) {
        float ms = 0;
        if (hipEventElapsedTime(&ms, g->chain0, g->chain1) == hipSuccess)
            g->stats.gpu_seconds += ms * 1e-3;
        g->chain_open = 0;
    }
    if (e != hipSuccess) return fail(g, "submit: %s", hipGetErrorString(e));
    return 1;
}

extern "C" int h3_gpu_timer_begin(h3_gpu *g) {
    if (!g) return 0;
    return hipEventRecord(g->timer0, g->stream) == hipSuccess ? 1
                                                            : fail(g, "timer_begin failed");
}

extern "C" double h3_gpu_timer_end(h3_gpu *g) {
    if (!g) return -1.0;
    if (hipEventRecord(g->timer1, g->stream) != hipSuccess) return -1.0;
    if (hipEventSynchronize(g->timer1) != hipSuccess) return -1.0;
    float ms = 0;
    if (hipEventElapsedTime(&ms, g->timer0, g->timer1) != hipSuccess) return -1.0;
    return ms;
}

/* Spans: a begin and an end event recorded on the stream around a piece of
 * work, no synchronisation; qw_gpu_span_collect waits for the last one and
 * returns every span's device time. Up to QW_SPAN_MAX spans between
 * collects; events are created on the first span. */
extern "C" int qw_gpu_span_begin(h3_gpu *g, int tag) {
    if (!g) return 0;
    if (g->span_open) return fail(g, "span_begin: a span is already open");
    if (!g->span_ev) {
        g->span_ev = (hipEvent_t *)calloc(2 * QW_SPAN_MAX, sizeof(hipEvent_t));
        g->span_tag = (int *)calloc(QW_SPAN_MAX, sizeof(int));
        if (!g->span_ev || !g->span_tag) return fail(g, "span_begin: out of host memory");
        for (int i = 0; i < 2 * QW_SPAN_MAX; i++)
            if (hipEventCreate(&g->span_ev[i]) != hipSuccess) {
                for (int j = 0; j < i; j++) hipEventDestroy(g->span_ev[j]);
                free(g->span_ev);
                free(g->span_tag);
                g->span_ev = NULL;
                g->span_tag = NULL;
                return fail(g, "span_begin: event creation failed");
            }
    }
    if (g->span_n >= QW_SPAN_MAX) return fail(g, "span_begin: more than %d spans", QW_SPAN_MAX);
    g->span_tag[g->span_n] = tag;
    if (hipEventRecord(g->span_ev[2 * g->span_n], g->stream) != hipSuccess)
        return fail(g, "span_begin: event record failed");
    g->span_open = 1;
    return 1;
}

extern "C" int qw_gpu_span_end(h3_gpu *g) {
    if (!g) return 0;
    if (!g->span_open) return fail(g, "span_end: no open span");
    if (hipEventRecord(g->span_ev[2 * g->span_n + 1], g->stream) != hipSuccess)
        return fail(g, "span_end: event record failed");
    g->span_open = 0;
    g->span_n++;
    return 1;
}

extern "C" int qw_gpu_span_collect(h3_gpu *g, int *tags, double *ms, int max) {
    if (!g) return -1;
    if (g->span_open) {
        fail(g, "span_collect: a span is still open");
        return -1;
    }
    const int n = g->span_n < max ? g->span_n : max;
    if (g->span_n && hipEventSynchronize(g->span_ev[2 * g->span_n - 1]) != hipSuccess) {
        fail(g, "span_collect: event wait failed");
        return -1;
    }
    for (int i = 0; i < n; i++) {
        float t = 0;
        if (hipEventElapsedTime(&t, g->span_ev[2 * i], g->span_ev[2 * i + 1]) != hipSuccess) {
            fail(g, "span_collect: elapsed time unavailable");
            return -1;
        }
        if (tags) tags[i] = g->span_tag[i];
        if (ms) ms[i] = t;
    }
    g->span_n = 0;
    return n;
}

/* ---------------------------------------------------------------------- */
/* tensors                                                                */

static h3_gpu_tensor *tensor_new(h3_gpu *g, size_t elements, h3_gpu_dtype d) {
    if (!g) return NULL;
    size_t bytes = elements * dtype_size(d);
    if (bytes == 0) bytes = 16;
    bytes = (bytes + 255) & ~(size_t)255;
    void *p = NULL;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        fail(g, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return NULL;
    }
    if (hipMemsetAsync(p, 0, bytes, g->stream) != hipSuccess ||
        hipStreamSynchronize(g->stream) != hipSuccess) {
        hipFree(p);
        fail(g, "tensor zero-fill failed");
        return NULL;
    }
    h3_gpu_tensor *t = new h3_gpu_tensor{g, (unsigned char *)p, elements, d, 1};
    g->stats.allocated_bytes += bytes;
    g->stats.live_bytes += bytes;
    g->stats.tensor_allocations++;
    if (g->stats.live_bytes > g->stats.peak_live_bytes) g->stats.peak_live_bytes = g->stats.live_bytes;
    return t;
}

extern "C" h3_gpu_tensor *h3_gpu_tensor_new_f32(h3_gpu *g, size_t n) { return tensor_new(g, n, H3_GPU_F32); }
extern "C" h3_gpu_tensor *h3_gpu_tensor_new_bf16(h3_gpu *g, size_t n) { return tensor_new(g, n, H3_GPU_BF16); }
extern "C" h3_gpu_tensor *h3_gpu_tensor_new_i8(h3_gpu *g, size_t n) { return tensor_new(g, n, H3_GPU_I8); }
extern "C" h3_gpu_tensor *h3_gpu_tensor_new_u32(h3_gpu *g, size_t n) { return tensor_new(g, n, H3_GPU_U32); }

static int copy_in(h3_gpu_tensor *t, size_t off_bytes, const void *src, size_t bytes) {
    h3_gpu *g = t->gpu;
    if (off_bytes + bytes > t->elements * dtype_size(t->dtype))
        return fail(g, "tensor write out of range (%zu + %zu > %zu bytes)", off_bytes, bytes,
                    t->elements * dtype_size(t->dtype));
    if (!bytes) return 1;
    hipError_t e = hipMemcpyAsync(t->ptr + off_bytes, src, bytes, hipMemcpyHostToDevice, g->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g->stream);
    return e == hipSuccess ? 1 : fail(g, "tensor write: %s", hipGetErrorString(e));
}

static int copy_out(const h3_gpu_tensor *t, size_t off_bytes, void *dst, size_t bytes) {
    h3_gpu *g = t->gpu;
    if (off_bytes + bytes > t->elements * dtype_size(t->dtype))
        return fail(g, "tensor read out of range");
    if (!bytes) return 1;
    hipError_t e = hipMemcpyAsync(dst, t->ptr + off_bytes, bytes, hipMemcpyDeviceToHost, g->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g->stream);
    return e == hipSuccess ? 1 : fail(g, "tensor read: %s", hipGetErrorString(e));
}

static h3_gpu_tensor *tensor_from(h3_gpu *g, const void *v, size_t n, h3_gpu_dtype d) {
    h3_gpu_tensor *t = tensor_new(g, n, d);
    if (t && v && !copy_in(t, 0, v, n * dtype_size(d))) {
        h3_gpu_tensor_free(t);
        return NULL;
    }
    return t;
}

extern "C" h3_gpu_tensor *h3_gpu_tensor_from_f32(h3_gpu *g, const float *v, size_t n) {
    return tensor_from(g, v, n, H3_GPU_F32);
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_from_bf16(h3_gpu *g, const uint16_t *v, size_t n) {
    return tensor_from(g, v, n, H3_GPU_BF16);
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_from_u32(h3_gpu *g, const uint32_t *v, size_t n) {
    return tensor_from(g, v, n, H3_GPU_U32);
}

extern "C" h3_gpu_tensor *h3_gpu_tensor_view(const h3_gpu_tensor *base, size_t offset,
                                             size_t elements) {
    if (!base) return NULL;
    if (offset + elements > base->elements) {
        fail(base->gpu, "view [%zu, +%zu) outside tensor of %zu", offset, elements,
             base->elements);
        return NULL;
    }
    return new h3_gpu_tensor{base->gpu, base->ptr + offset * dtype_size(base->dtype), elements,
                             base->dtype, 0};
}

extern "C" void h3_gpu_tensor_free(h3_gpu_tensor *t) {
    if (!t) return;
    if (t->owns) {
        h3_gpu *g = t->gpu;
        /* the stream may still reference the buffer */
        hipStreamSynchronize(g->stream);
        size_t bytes = (t->elements * dtype_size(t->dtype) + 255) & ~(size_t)255;
        if (!bytes) bytes = 256;
        g->stats.live_bytes -= bytes < g->stats.live_bytes ? bytes : g->stats.live_bytes;
        hipFree(t->ptr);
    }
    delete t;
}

extern "C" size_t h3_gpu_tensor_elements(const h3_gpu_tensor *t) { return t ? t->elements : 0; }
extern "C" h3_gpu_dtype h3_gpu_tensor_dtype(const h3_gpu_tensor *t) { return t ? t->dtype : H3_GPU_F32; }
extern "C" void *h3_gpu_tensor_device_ptr(const h3_gpu_tensor *t) { return t ? t->ptr : NULL; }

#define REQ_DT(t, d, what)                                                           \
    do {                                                                             \
        if (!(t)) return fail(g, "%s: missing tensor", what);                        \
        if ((t)->dtype != (d)) return fail(g, "%s: wrong dtype", what);              \
    } while (0)

extern "C" int h3_gpu_tensor_read_f32(const h3_gpu_tensor *t, float *v, size_t n) {
    if (!t || t->dtype != H3_GPU_F32) return t ? fail(t->gpu, "read_f32: dtype") : 0;
    return copy_out(t, 0, v, n * 4);
}
extern "C" int h3_gpu_tensor_read_f32_range(const h3_gpu_tensor *t, size_t off, float *v, size_t n) {
    if (!t || t->dtype != H3_GPU_F32) return t ? fail(t->gpu, "read_f32: dtype") : 0;
    return copy_out(t, off * 4, v, n * 4);
}
extern "C" int h3_gpu_tensor_read_bf16(const h3_gpu_tensor *t, uint16_t *v, size_t n) {
    if (!t || t->dtype != H3_GPU_BF16) return t ? fail(t->gpu, "read_bf16: dtype") : 0;
    return copy_out(t, 0, v, n * 2);
}
extern "C" int h3_gpu_tensor_write_f32(h3_gpu_tensor *t, const float *v, size_t n) {
    if (!t || t->dtype != H3_GPU_F32) return t ? fail(t->gpu, "write_f32: dtype") : 0;
    return copy_in(t, 0, v, n * 4);
}
extern "C" int h3_gpu_tensor_write_f32_range(h3_gpu_tensor *t, size_t off, const float *v, size_t n) {
    if (!t || t->dtype != H3_GPU_F32) return t ? fail(t->gpu, "write_f32: dtype") : 0;
    return copy_in(t, off * 4, v, n * 4);
}
extern "C" int h3_gpu_tensor_write_bf16(h3_gpu_tensor *t, const uint16_t *v, size_t n) {
    if (!t || t->dtype != H3_GPU_BF16) return t ? fail(t->gpu, "write_bf16: dtype") : 0;
    return copy_in(t, 0, v, n * 2);
}
extern "C" int h3_gpu_tensor_write_bf16_range(h3_gpu_tensor *t, size_t off, const uint16_t *v,
                                              size_t n) {
    if (!t || t->dtype != H3_GPU_BF16) return t ? fail(t->gpu, "write_bf16: dtype") : 0;
    return copy_in(t, off * 2, v, n * 2);
}
extern "C" int h3_gpu_tensor_read_bytes(const h3_gpu_tensor *t, void *b, size_t n) {
    return t ? copy_out(t, 0, b, n) : 0;
}
extern "C" int h3_gpu_tensor_write_bytes(h3_gpu_tensor *t, const void *b, size_t n) {
    return t ? copy_in(t, 0, b, n) : 0;
}

/* ---------------------------------------------------------------------- */
/* launches                                                               */

template <class T>
static int launch(h3_gpu *g, int kid, dim3 grid, dim3 block, const T &args) {
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) return 1; /* empty problem */
    void *params[] = {(void *)&args};
    hipError_t e = hipModuleLaunchKernel(g->fn[kid], grid.x, grid.y, grid.z, block.x, block.y,
                                         block.z, 0, g->stream, params, NULL);
    if (e != hipSuccess) return fail(g, "launch %s: %s", k_names[kid], hipGetErrorString(e));
    g->stats.direct_dispatches++;
    return 1;
}

static bool fits(const h3_gpu_tensor *t, size_t offset, size_t elements) {
    return t && offset + elements <= t->elements;
}

static uint32_t blocks_for(uint64_t n, uint32_t per) { return (uint32_t)((n + per - 1) / per); }

static int ln_mod(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in,
                  const h3_gpu_tensor *mod, const h3_gpu_tensor *row_map, uint32_t rows,
                  uint32_t width, uint32_t slots, uint32_t scale_slot, int32_t shift_slot,
                  float eps) {
    REQ_DT(out, H3_GPU_BF16, "layer_norm_mod out");
    REQ_DT(in, H3_GPU_BF16, "layer_norm_mod in");
    REQ_DT(mod, H3_GPU_BF16, "layer_norm_mod modulation");
    REQ_DT(row_map, H3_GPU_U32, "layer_norm_mod row_map");
    if (width % 8 || width / 8 > 1024 || width == 0)
        return fail(g, "layer_norm_mod: width %u must be a multiple of 8, <= 8192", width);
    if (scale_slot >= slots || (shift_slot >= 0 && (uint32_t)shift_slot >= slots))
        return fail(g, "layer_norm_mod: slot out of range");
    if (!fits(out, 0, (size_t)rows * width) || !fits(in, 0, (size_t)rows * width) ||
        !fits(row_map, 0, rows))
        return fail(g, "layer_norm_mod: tensor too small");
    /* every row_map entry must address a modulation row: checked on host */
    uint32_t mod_rows = (uint32_t)(mod->elements / ((size_t)slots * width));
    if (mod_rows == 0) return fail(g, "layer_norm_mod: modulation too small");
    qw_ln_mod_args a = {(uint16_t *)out->ptr, (const uint16_t *)in->ptr,
                        (const uint16_t *)mod->ptr, (const uint32_t *)row_map->ptr,
                        rows, width, slots, scale_slot, shift_slot, eps};
    if (width <= 4096) return launch(g, K_LN_MOD, dim3((rows + 3) / 4), dim3(256), a);
    return launch(g, K_LN_MOD_WIDE, dim3(rows), dim3((width / 8 + 63) / 64 * 64), a);
}

extern "C" int qw_gpu_layer_norm_mod_bf16(h3_gpu *g, h3_gpu_tensor *out,
                                          const h3_gpu_tensor *in,
                                          const h3_gpu_tensor *mod,
                                          const h3_gpu_tensor *row_map, uint32_t rows,
                                          uint32_t width, uint32_t slots, uint32_t scale_slot,
                                          float eps) {
    return ln_mod(g, out, in, mod, row_map, rows, width, slots, scale_slot, -1, eps);
}

extern "C" int qw_gpu_layer_norm_mod_shift_bf16(h3_gpu *g, h3_gpu_tensor *out,
                                                const h3_gpu_tensor *in,
                                                const h3_gpu_tensor *mod,
                                                const h3_gpu_tensor *row_map, uint32_t rows,
                                                uint32_t width, uint32_t slots,
                                                uint32_t scale_slot, int32_t shift_slot,
                                                float eps) {
    return ln_mod(g, out, in, mod, row_map, rows, width, slots, scale_slot, shift_slot, eps);
}

extern "C" int qw_gpu_rms_norm_one_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in,
                                        const h3_gpu_tensor *w, uint32_t rows, uint32_t width,
                                        float eps) {
    REQ_DT(out, H3_GPU_BF16, "rms_norm_one out");
    REQ_DT(in, H3_GPU_BF16, "rms_norm_one in");
    REQ_DT(w, H3_GPU_BF16, "rms_norm_one weight");
    if (width % 8 || width / 8 > 1024 || width == 0)
        return fail(g, "rms_norm_one: width %u must be a multiple of 8, <= 8192", width);
    if (!fits(out, 0, (size_t)rows * width) || !fits(in, 0, (size_t)rows * width) ||
        !fits(w, 0, width))
        return fail(g, "rms_norm_one: tensor too small");
    qw_rms_one_args a = {(uint16_t *)out->ptr, (const uint16_t *)in->ptr,
                         (const uint16_t *)w->ptr, rows, width, eps};
    return launch(g, K_RMS_ONE, dim3(rows), dim3((width / 8 + 63) / 64 * 64), a);
}

static int act(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, uint64_t n, int kind) {
    REQ_DT(out, H3_GPU_BF16, "activation out");
    REQ_DT(in, H3_GPU_BF16, "activation in");
    if (!fits(out, 0, n) || !fits(in, 0, n)) return fail(g, "activation: tensor too small");
    qw_act_args a = {(uint16_t *)out->ptr, (const uint16_t *)in->ptr, n, kind};
    return launch(g, K_ACT, dim3(blocks_for(n, 256)), dim3(256), a);
}

extern "C" int h3_gpu_silu_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in,
                                uint32_t n) {
    return act(g, out, in, n, QW_ACT_SILU);
}
extern "C" int h3_gpu_gelu_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in,
                                uint32_t n, int approximate) {
    if (!approximate) return fail(g, "gelu: only the tanh approximation is on the DiT path");
    return act(g, out, in, n, QW_ACT_GELU_TANH);
}
extern "C" int qw_gpu_tanh_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in,
                                uint32_t n) {
    return act(g, out, in, n, QW_ACT_TANH);
}

extern "C" int qw_gpu_swiglu_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *fc1,
                                  uint32_t rows, uint32_t width) {
    REQ_DT(out, H3_GPU_BF16, "swiglu out");
    REQ_DT(fc1, H3_GPU_BF16, "swiglu fc1");
    if (!fits(out, 0, (size_t)rows * width) || !fits(fc1, 0, (size_t)rows * width * 2))
        return fail(g, "swiglu: tensor too small");
    qw_swiglu_args a = {(uint16_t *)out->ptr, (const uint16_t *)fc1->ptr, rows, width};
    return launch(g, K_SWIGLU, dim3(blocks_for((uint64_t)rows * width, 256)), dim3(256), a);
}

extern "C" int h3_gpu_cast_f32_to_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in,
                                       uint32_t n) {
    REQ_DT(out, H3_GPU_BF16, "cast out");
    REQ_DT(in, H3_GPU_F32, "cast in");
    if (!fits(out, 0, n) || !fits(in, 0, n)) return fail(g, "cast: tensor too small");
    qw_cast_args a = {(uint16_t *)out->ptr, (const float *)in->ptr, n};
    return launch(g, K_CAST, dim3(blocks_for(n, 256)), dim3(256), a);
}

extern "C" int qw_gpu_cfg_euler_f32(h3_gpu *g, h3_gpu_tensor *x, const h3_gpu_tensor *pos,
                                    size_t pos_offset, const h3_gpu_tensor *neg,
                                    size_t neg_offset, size_t count, float dt, float cfg) {
    if (!g) return 0;
    REQ_DT(x, H3_GPU_F32, "euler sample");
    REQ_DT(pos, H3_GPU_BF16, "euler prediction");
    if (neg) REQ_DT(neg, H3_GPU_BF16, "euler unconditional prediction");
    if (!fits(x, 0, count) || !fits(pos, pos_offset, count) ||
        (neg && !fits(neg, neg_offset, count)))
        return fail(g, "euler: tensor too small");
    qw_euler_args a = {(float *)x->ptr, (const uint16_t *)pos->ptr + pos_offset,
                       neg ? (const uint16_t *)neg->ptr + neg_offset : NULL, count, dt, cfg};
    return launch(g, K_EULER, dim3(blocks_for(count, 256)), dim3(256), a);
}

extern "C" int qw_gpu_lora_fuse_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *base,
                                     uint32_t rows, uint32_t cols, const qw_lora_term_desc *terms,
                                     uint32_t nterms) {
    if (!g) return 0;
    REQ_DT(out, H3_GPU_BF16, "lora out");
    REQ_DT(base, H3_GPU_BF16, "lora base");
    if (!fits(out, 0, (size_t)rows * cols) || !fits(base, 0, (size_t)rows * cols))
        return fail(g, "lora: tensors smaller than %u x %u", rows, cols);
    if (nterms > QW_LORA_MAX_TERMS) return fail(g, "lora: %u terms (max %d)", nterms, QW_LORA_MAX_TERMS);
    qw_lora_args a;
    memset(&a, 0, sizeof(a));
    a.out = (uint16_t *)out->ptr;
    a.base = (const uint16_t *)base->ptr;
    a.rows = rows;
    a.cols = cols;
    a.nterms = nterms;
    for (uint32_t t = 0; t < nterms; t++) {
        const qw_lora_term_desc *d = &terms[t];
        REQ_DT(d->a, H3_GPU_BF16, "lora A");
        REQ_DT(d->b, H3_GPU_BF16, "lora B");
        if (!d->rank || d->rank > QW_LORA_MAX_RANK)
            return fail(g, "lora: rank %u outside [1, %d]", d->rank, QW_LORA_MAX_RANK);
        if ((uint64_t)d->row0 + d->rows > rows) return fail(g, "lora: term rows outside the weight");
        if (!fits(d->a, 0, (size_t)d->rank * cols) || !fits(d->b, 0, (size_t)d->rows * d->rank))
            return fail(g, "lora: A or B smaller than its shape");
        a.terms[t] = qw_lora_term{(const uint16_t *)d->a->ptr, (const uint16_t *)d->b->ptr, d->row0,
                                  d->rows, d->rank, d->scale};
    }
    return launch(g, K_LORA, dim3((cols + 63) / 64, (rows + 63) / 64), dim3(256), a);
}

extern "C" int h3_gpu_gate_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *res,
                                const h3_gpu_tensor *branch, const h3_gpu_tensor *mod,
                                const h3_gpu_tensor *row_map, uint32_t rows, uint32_t width,
                                uint32_t slots, uint32_t gate_slot) {
    REQ_DT(out, H3_GPU_BF16, "gate out");
    REQ_DT(res, H3_GPU_BF16, "gate residual");
    REQ_DT(branch, H3_GPU_BF16, "gate branch");
    REQ_DT(mod, H3_GPU_BF16, "gate modulation");
    REQ_DT(row_map, H3_GPU_U32, "gate row_map");
    size_t n = (size_t)rows * width;
    if (width % 8) return fail(g, "gate: width must be a multiple of 8");
    if (gate_slot >= slots) return fail(g, "gate: slot out of range");
    if (!fits(out, 0, n) || !fits(res, 0, n) || !fits(branch, 0, n) || !fits(row_map, 0, rows) ||
        mod->elements < (size_t)slots * width)
        return fail(g, "gate: tensor too small");
    qw_gate_args a = {(uint16_t *)out->ptr, (const uint16_t *)res->ptr,
                      (const uint16_t *)branch->ptr, (const uint16_t *)mod->ptr,
                      (const uint32_t *)row_map->ptr, rows, width, slots, gate_slot};
    return launch(g, K_GATE, dim3(blocks_for(n / 8, 256)), dim3(256), a);
}

extern "C" int qw_gpu_qk_norm_rope_bf16(h3_gpu *g, h3_gpu_tensor *qk, uint32_t rows,
                                        uint32_t heads, uint32_t ld, uint32_t k_offset,
                                        const h3_gpu_tensor *norm_q, const h3_gpu_tensor *norm_k,
                                        const h3_gpu_tensor *rope_cos,
                                        const h3_gpu_tensor *rope_sin, uint32_t rope_rows,
                                        float eps) {
    REQ_DT(qk, H3_GPU_BF16, "qk_norm_rope qk");
    int do_norm = norm_q || norm_k;
    int do_rope = rope_cos || rope_sin;
    if (do_norm) {
        REQ_DT(norm_q, H3_GPU_BF16, "qk_norm_rope norm_q");
        REQ_DT(norm_k, H3_GPU_BF16, "qk_norm_rope norm_k");
        if (norm_q->elements < 128 || norm_k->elements < 128)
            return fail(g, "qk_norm_rope: norm weights need 128 elements");
    }
    if (do_rope) {
        REQ_DT(rope_cos, H3_GPU_F32, "qk_norm_rope cos");
        REQ_DT(rope_sin, H3_GPU_F32, "qk_norm_rope sin");
        if (!rope_rows || !fits(rope_cos, 0, (size_t)rope_rows * 64) ||
            !fits(rope_sin, 0, (size_t)rope_rows * 64))
            return fail(g, "qk_norm_rope: rope tables too small");
    }
    if (((uintptr_t)qk->ptr | (do_rope ? (uintptr_t)rope_cos->ptr | (uintptr_t)rope_sin->ptr : 0) |
         (do_norm ? (uintptr_t)norm_q->ptr | (uintptr_t)norm_k->ptr : 0)) % 16)
        return fail(g, "qk_norm_rope: tensors must be 16-byte aligned");
    if (ld % 8 || k_offset % 8 || k_offset + (size_t)heads * 128 > ld ||
        (size_t)heads * 128 > ld || (rows && !fits(qk, 0, (size_t)(rows - 1) * ld + k_offset + heads * 128)))
        return fail(g, "qk_norm_rope: bad geometry");
    qw_qk_norm_rope_args a = {(uint16_t *)qk->ptr,
                              do_norm ? (const uint16_t *)norm_q->ptr : NULL,
                              do_norm ? (const uint16_t *)norm_k->ptr : NULL,
                              do_rope ? (const float *)rope_cos->ptr : NULL,
                              do_rope ? (const float *)rope_sin->ptr : NULL,
                              rows, heads, ld, k_offset, do_rope ? rope_rows : 1,
                              do_norm, do_rope, eps};
    uint64_t items = (uint64_t)rows * heads * 2;
    return launch(g, K_QK_NORM_ROPE, dim3(blocks_for(items, 16)), dim3(256), a);
}

extern "C" int h3_gpu_head_rms_norm_bf16(h3_gpu *g, h3_gpu_tensor *t, const h3_gpu_tensor *w,
                                         uint32_t seq, uint32_t heads, uint32_t head_dim,
                                         float eps) {
    if (head_dim != 128) return fail(g, "head_rms_norm: head_dim must be 128");
    REQ_DT(t, H3_GPU_BF16, "head_rms_norm tensor");
    REQ_DT(w, H3_GPU_BF16, "head_rms_norm weight");
    if (heads % 2) return fail(g, "head_rms_norm: heads must be even");
    /* The fused kernel's "q" half covers heads [0, heads/2) and its "k" half
     * heads [heads/2, heads) of the same row, both with this weight. */
    return qw_gpu_qk_norm_rope_bf16(g, t, seq, heads / 2, heads * 128, (heads / 2) * 128, w, w,
                                    NULL, NULL, 0, eps);
}

extern "C" int qw_gpu_qk_rope_bf16(h3_gpu *g, h3_gpu_tensor *qo, h3_gpu_tensor *ko,
                                   const h3_gpu_tensor *qi, const h3_gpu_tensor *ki,
                                   const h3_gpu_tensor *cos_t, const h3_gpu_tensor *sin_t,
                                   uint32_t seq, uint32_t heads, uint32_t head_dim) {
    if (head_dim != 128) return fail(g, "qk_rope: head_dim must be 128");
    if (qo != qi || ko != ki) return fail(g, "qk_rope: only in-place operation is supported");
    REQ_DT(qo, H3_GPU_BF16, "qk_rope q");
    REQ_DT(ko, H3_GPU_BF16, "qk_rope k");
    size_t n = (size_t)seq * heads * 128;
    if (!fits(qo, 0, n) || !fits(ko, 0, n)) return fail(g, "qk_rope: tensor too small");
    if (heads % 2) return fail(g, "qk_rope: heads must be even");
    /* one rotation-only pass per tensor (head halves as in head_rms_norm) */
    for (int pass = 0; pass < 2; pass++) {
        h3_gpu_tensor *t = pass ? ko : qo;
        if (!qw_gpu_qk_norm_rope_bf16(g, t, seq, heads / 2, heads * 128, (heads / 2) * 128, NULL,
                                      NULL, cos_t, sin_t, seq, 0.0f))
            return 0;
    }
    return 1;
}

extern "C" int qw_gpu_modulation_reorder_bf16(h3_gpu *g, h3_gpu_tensor *out,
                                              const h3_gpu_tensor *raw, uint32_t mod_rows,
                                              uint32_t hidden, int shift_variant) {
    REQ_DT(out, H3_GPU_BF16, "reorder out");
    REQ_DT(raw, H3_GPU_BF16, "reorder raw");
    size_t n = (size_t)mod_rows * hidden * (shift_variant ? 6 : 4);
    if (!fits(out, 0, n) || !fits(raw, 0, n)) return fail(g, "reorder: tensor too small");
    if (out->ptr == raw->ptr) return fail(g, "reorder: output must not alias the input");
    qw_reorder_args a = {(uint16_t *)out->ptr, (const uint16_t *)raw->ptr, mod_rows, hidden,
                         shift_variant};
    return launch(g, K_REORDER, dim3(blocks_for((uint64_t)mod_rows * hidden, 256)), dim3(256), a);
}

extern "C" int qw_gpu_fill_normal_bf16(h3_gpu *g, h3_gpu_tensor *t, size_t off, size_t count,
                                       uint64_t seed, uint64_t stream, float std, float offset) {
    REQ_DT(t, H3_GPU_BF16, "fill tensor");
    if (!fits(t, off, count)) return fail(g, "fill: range outside tensor");
    qw_fill_args a = {(uint16_t *)t->ptr + off, count, seed, stream, std, offset};
    return launch(g, K_FILL, dim3(blocks_for(count, 256)), dim3(256), a);
}

extern "C" int h3_gpu_quantize_weight_int8(h3_gpu *g, h3_gpu_tensor *out, h3_gpu_tensor *scales,
                                           const h3_gpu_tensor *in, uint32_t rows,
                                           uint32_t cols) {
    REQ_DT(out, H3_GPU_I8, "quantize out");
    REQ_DT(scales, H3_GPU_F32, "quantize scales");
    REQ_DT(in, H3_GPU_BF16, "quantize in");
    size_t n = (size_t)rows * cols;
    if (!fits(out, 0, n) || !fits(in, 0, n) || !fits(scales, 0, rows))
        return fail(g, "quantize: tensor too small");
    qw_quant_args a = {(int8_t *)out->ptr, (float *)scales->ptr, (const uint16_t *)in->ptr, rows,
                       cols};
    return launch(g, K_QUANT, dim3(rows), dim3(256), a);
}

extern "C" int qw_gpu_dequant_int8_f32(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q,
                                       const h3_gpu_tensor *scales, uint32_t rows,
                                       uint32_t cols) {
    REQ_DT(out, H3_GPU_F32, "dequant out");
    REQ_DT(q, H3_GPU_I8, "dequant q");
    REQ_DT(scales, H3_GPU_F32, "dequant scales");
    size_t n = (size_t)rows * cols;
    if (!fits(out, 0, n) || !fits(q, 0, n) || !fits(scales, 0, rows))
        return fail(g, "dequant: tensor too small");
    qw_dequant_args a = {(float *)out->ptr, (const int8_t *)q->ptr, (const float *)scales->ptr,
                         rows, cols};
    return launch(g, K_DEQUANT, dim3(blocks_for(n, 256)), dim3(256), a);
}

extern "C" int qw_gpu_copy_rows(h3_gpu *g, h3_gpu_tensor *dst, size_t doff, uint32_t dstride,
                                const h3_gpu_tensor *src, size_t soff, uint32_t sstride,
                                uint32_t rows, uint32_t row_elems) {
    if (!dst || !src || dst->dtype != src->dtype) return fail(g, "copy_rows: dtype mismatch");
    size_t es = dtype_size(dst->dtype);
    if (!rows || !row_elems) return 1;
    if ((row_elems * es) % 4 || (doff * es) % 4 || (soff * es) % 4 || (dstride * es) % 4 ||
        (sstride * es) % 4)
        return fail(g, "copy_rows: rows must be 4-byte aligned");
    if (!fits(dst, doff, (size_t)(rows - 1) * dstride + row_elems) ||
        !fits(src, soff, (size_t)(rows - 1) * sstride + row_elems))
        return fail(g, "copy_rows: range outside tensor");
    qw_copy2d_args a = {dst->ptr + doff * es, src->ptr + soff * es, rows, row_elems * es,
                        dstride * es, sstride * es};
    uint64_t words = (uint64_t)rows * row_elems * es / 4;
    g->stats.blit_copies++;
    return launch(g, K_COPY2D, dim3(blocks_for(words, 256)), dim3(256), a);
}

extern "C" int h3_gpu_copy_bf16(h3_gpu *g, h3_gpu_tensor *dst, size_t doff,
                                const h3_gpu_tensor *src, size_t soff, size_t n) {
    REQ_DT(dst, H3_GPU_BF16, "copy dst");
    REQ_DT(src, H3_GPU_BF16, "copy src");
    if (!fits(dst, doff, n) || !fits(src, soff, n)) return fail(g, "copy: range outside tensor");
    if (!n) return 1;
    hipError_t e = hipMemcpyAsync(dst->ptr + doff * 2, src->ptr + soff * 2, n * 2,
                                  hipMemcpyDeviceToDevice, g->stream);
    g->stats.blit_copies++;
    return e == hipSuccess ? 1 : fail(g, "copy: %s", hipGetErrorString(e));
}

/* ---- GEMM ---------------------------------------------------------------- */

static int widen_launch(h3_gpu *g, uint16_t *out, const int8_t *in, size_t n) {
    qw_widen_args wa;
    wa.out = out;
    wa.in = in;
    wa.count = n;
    unsigned blocks = (unsigned)std::min<size_t>((n / 8 + 255) / 256, 65536);
    return launch(g, K_WIDEN, dim3(blocks ? blocks : 1), dim3(256), wa);
}

extern "C" int qw_gpu_widen_int8_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q,
                                      size_t count) {
    if (!g) return 0;
    REQ_DT(out, H3_GPU_BF16, "widen out");
    REQ_DT(q, H3_GPU_I8, "widen in");
    if (count % 16) return fail(g, "widen: count %zu is not a multiple of 16", count);
    if (!fits(out, 0, count) || !fits(q, 0, count)) return fail(g, "widen: tensor too small");
    if (!count) return 1;
    return widen_launch(g, (uint16_t *)out->ptr, (const int8_t *)q->ptr, count);
}


/* Split tiles. A grid of one workgroup per 256 x 256 tile runs in waves of
 * `cus` tiles; when the last wave is partly filled (R = tiles % cus tiles,
 * all of them when there is no full wave), each of its tiles can instead be
 * cut into s k-ranges: R s pieces taking ceil(R s / cus) waves of 1/s the
 * length. s minimises that tail time plus 0.02 (s - 1) for writing and
 * re-reading the fp32 partials, and is used only when that beats 0.9 of the
 * whole-tile tail (M = 8704, K = 12288, N = 3072, residual-gate epilogue:
 * 152 tail tiles in 3 pieces 557-588 us against 573-644 us for the
 * whole-tile walk, same boxes; 2, 4 or 5 pieces 595-660 us). Pieces stay at least 32 k-steps (2048 k) long: shorter
 * pieces lost more to their partials than they gained (K = 3072 linears
 * measured slower when split, K = 12288 ones faster); the half tiles of a
 * launch of at most cus / 2 tiles, whose pieces all run in one wave, go
 * down to 16. And
 * R s <= QW_SPLIT_MAX_PIECES * cus bounds the partial workspace. */
#define QW_SPLIT_MAX_PIECES 2
static uint32_t split_choice(h3_gpu *g, uint32_t tiles, uint32_t ksteps,
                             uint64_t max_pieces = (uint64_t)QW_SPLIT_MAX_PIECES * 1024u,
                             uint32_t min_steps = 0) {
    if (!min_steps) min_steps = g->split_min_steps;
    const uint32_t G = g->cus, R = tiles % G;
    if (R == 0) return 1; /* every wave is full: nothing to split */
    if (g->split_force > 1 && (uint64_t)R * g->split_force <= (uint64_t)QW_SPLIT_MAX_PIECES * G &&
        (uint64_t)R * g->split_force <= max_pieces && ksteps >= g->split_force)
        return g->split_force;
    uint32_t best = 1;
    double best_t = 0.9;
    for (uint32_t s = 2; s <= 8; s++) {
        if ((uint64_t)R * s > (uint64_t)QW_SPLIT_MAX_PIECES * G || (uint64_t)R * s > max_pieces ||
            ksteps < min_steps * s)
            break;
        const double t = (double)((R * s + G - 1) / G) / s + 0.02 * (s - 1);
        if (t < best_t) {
            best_t = t;
            best = s;
        }
    }
    return best;
}

/* Pieces for the half tiles of a small launch (at most cus / 2 tiles), all
 * in one round of CUs: the s that minimises 0.72 ksteps / s + 12 + 0.04
 * units s microseconds -- a half tile's slice, then each piece's prologue,
 * partial sums and last-piece reduction, which grow with the pieces in
 * flight. Fitted to the three-stage kernels at K = 3072 (M = 320: 24, 48,
 * 64, 96, 128 half tiles in 3, 3, 3, 2, 2 pieces 26.0, 29.3, 32.4, 35.8,
 * 40.6 us against 34.7-35.6 unsplit; M = 1152: 120 in 2 pieces 38.8
 * against 35.5), within 1.2 us of each. */
static uint32_t small_split_choice(h3_gpu *g, uint32_t units, uint32_t ksteps) {
    if (g->split_force > 1 && (uint64_t)units * g->split_force <= g->cus &&
        ksteps >= g->split_force)
        return g->split_force;
    uint32_t best = 1;
    double best_t = 0.72 * ksteps;
    for (uint32_t s = 2; s <= 8; s++) {
        if ((uint64_t)units * s > g->cus || ksteps < g->split_small_min * s) break;
        const double t = 0.72 * ksteps / s + 12.0 + 0.04 * units * s;
        if (t < best_t) {
            best_t = t;
            best = s;
        }
    }
    return best;
}

/* no_alloc: the workspace-free form behind qw_gpu_linear_static (int8
 * weights always widen inside the GEMM; split-tile partials and counters live
 * in the static workspace, as far as it holds them) */
static int linear_impl(h3_gpu *g, const qw_linear_desc *d, int no_alloc) {
    if (!g || !d) return 0;
    REQ_DT(d->out, H3_GPU_BF16, "linear out");
    REQ_DT(d->in, H3_GPU_BF16, "linear in");
    if (!d->weight) return fail(g, "linear: missing weight");
    const int int8 = d->weight->dtype == H3_GPU_I8;
    if (!int8 && d->weight->dtype != H3_GPU_BF16) return fail(g, "linear: weight dtype");
    if (d->rows == 0 || d->cols == 0) return 1;
    if (d->k == 0 || d->k % 64) return fail(g, "linear: k=%u must be a positive multiple of 64", d->k);
    if (d->lda % 8 || d->in_offset % 8 || d->lda < d->k)
        return fail(g, "linear: input rows must be 16-byte aligned (lda %u, offset %zu)", d->lda,
                    d->in_offset);
    if (d->ldc < d->cols) return fail(g, "linear: ldc < cols");
    if (d->cols % 8 || d->ldc % 4 || d->out_offset % 4)
        return fail(g, "linear: cols (%u) must be a multiple of 8 and output rows 8-byte aligned",
                    d->cols);
    if (!fits(d->in, d->in_offset, (size_t)(d->rows - 1) * d->lda + d->k))
        return fail(g, "linear: input too small");
    if (!fits(d->out, d->out_offset, (size_t)(d->rows - 1) * d->ldc + d->cols))
        return fail(g, "linear: output too small");
    if (!fits(d->weight, 0, (size_t)d->cols * d->k)) return fail(g, "linear: weight too small");
    if ((uint64_t)d->cols * d->k >= (1ull << 32) || (uint64_t)d->rows * d->lda >= (1ull << 32))
        return fail(g, "linear: operand exceeds 32-bit element offsets");
    if (int8 || d->wscale) {
        REQ_DT(d->wscale, H3_GPU_F32, "linear scales");
        if (!fits(d->wscale, 0, d->cols)) return fail(g, "linear: scales too small");
    }
    if (d->bias) {
        REQ_DT(d->bias, H3_GPU_BF16, "linear bias");
        if (!fits(d->bias, 0, d->cols)) return fail(g, "linear: bias too small");
    }
    const uint16_t *gate = NULL;
    const uint32_t *row_map = NULL;
    uint32_t gate_stride = 0;
    if (d->epilogue == QW_LINEAR_GATE) {
        REQ_DT(d->modulation, H3_GPU_BF16, "linear gate modulation");
        REQ_DT(d->row_map, H3_GPU_U32, "linear gate row_map");
        if (d->gate_slot >= d->slots) return fail(g, "linear: gate slot out of range");
        if (!fits(d->row_map, 0, d->rows)) return fail(g, "linear: row_map too small");
        gate_stride = d->slots * d->cols;
        if (d->modulation->elements < gate_stride) return fail(g, "linear: modulation too small");
        gate = (const uint16_t *)d->modulation->ptr + (size_t)d->gate_slot * d->cols;
        row_map = (const uint32_t *)d->row_map->ptr;
    } else if (d->epilogue == QW_LINEAR_QKNORM) {
        REQ_DT(d->norm_q, H3_GPU_BF16, "linear qk norm_q");
        REQ_DT(d->norm_k, H3_GPU_BF16, "linear qk norm_k");
        REQ_DT(d->rope_cos, H3_GPU_F32, "linear qk rope cos");
        REQ_DT(d->rope_sin, H3_GPU_F32, "linear qk rope sin");
        if (d->cols % 384 || d->out_offset || d->ldc % 8)
            return fail(g, "linear qk: cols must be q|k|v heads of 128, output at offset 0");
        if (d->norm_q->elements < 128 || d->norm_k->elements < 128 || !d->rope_rows ||
            !fits(d->rope_cos, 0, (size_t)d->rope_rows * 64) ||
            !fits(d->rope_sin, 0, (size_t)d->rope_rows * 64))
            return fail(g, "linear qk: norm weights or rope tables too small");
        if (((uintptr_t)d->norm_q->ptr | (uintptr_t)d->norm_k->ptr | (uintptr_t)d->rope_cos->ptr |
             (uintptr_t)d->rope_sin->ptr | (uintptr_t)d->out->ptr) % 16)
            return fail(g, "linear qk: tensors must be 16-byte aligned");
    } else if (d->epilogue != QW_LINEAR_STORE && d->epilogue != QW_LINEAR_GELU) {
        return fail(g, "linear: unknown epilogue %d", d->epilogue);
    }
    if (d->epilogue == QW_LINEAR_QKNORM && d->rope_rows < 128) {
        /* the fused epilogue wraps a 128-row block's RoPE table rows with one
         * subtraction, which needs a table of at least 128 rows; a shorter
         * one runs the plain linear, then the standalone norm + RoPE
         * (bit-identical to the fused epilogue) */
        qw_linear_desc plain = *d;
        plain.epilogue = QW_LINEAR_STORE;
        if (!linear_impl(g, &plain, no_alloc)) return 0;
        return qw_gpu_qk_norm_rope_bf16(g, d->out, d->rows, d->cols / 384, d->ldc, d->cols / 3,
                                        d->norm_q, d->norm_k, d->rope_cos, d->rope_sin,
                                        d->rope_rows, d->eps);
    }
    /* at most 8 rows, plain or GELU epilogue: one wave per 2 output columns
     * streams the weight once */
    if (d->rows <= 8 &&
        (d->epilogue == QW_LINEAR_STORE || d->epilogue == QW_LINEAR_GELU)) {
        qw_gemm_args a;
        memset(&a, 0, sizeof(a));
        a.a = (const uint16_t *)d->in->ptr + d->in_offset;
        a.w = d->weight->ptr;
        a.wscale = d->wscale ? (const float *)d->wscale->ptr : NULL;
        a.bias = d->bias ? (const uint16_t *)d->bias->ptr : NULL;
        a.out = (uint16_t *)d->out->ptr + d->out_offset;
        a.m = d->rows;
        a.n = d->cols;
        a.k = d->k;
        a.lda = d->lda;
        a.ldc = d->ldc;
        const int kid = (int8 ? K_GEMV_I8_STORE : K_GEMV_BF16_STORE) +
                        (d->epilogue == QW_LINEAR_GELU ? 1 : 0);
        const uint32_t waves = (d->cols + 1) / 2; /* 2 columns per wave */
        return launch(g, kid, dim3((waves + 3) / 4), dim3(256), a);
    }
    /* int8 weights: the "_w8" kernels widen each int8 W tile once per
     * workgroup into the bf16 W stage in LDS (no copy through HBM, half
     * the weight bytes). Where it measured faster -- 512+ rows and K <
     * 8192 -- the weight is instead widened to a bf16 copy by one
     * bandwidth-bound pass and the bf16 kernels run; both routes give the
     * same bits (the per-row scale multiplies the finished fp32 sums). Same
     * box, alternating, M = 8704, us (widening pass + bf16 kernel / w8):
     * QKV 378-387 / 391-406, out 140-145 / 145-151, up 485-504 / 530-565,
     * down 558-571 / 558-573; steps 66.30-66.49 ms with every int8 linear
     * widened, 68.11-68.24 with every one on w8, 66.32-66.47 with w8 on the
     * down projection only. The w8 kernels' extra cost is the widening's
     * VALU work (1.5 instructions per weight per workgroup): the same
     * kernel with the conversion left out runs as fast as the widening
     * pass plus the bf16 kernel. */
    /* the 224-row tile rule on this shape (whole tiles, bf16 kernels) */
    const uint32_t tn_w = (d->cols + 255) / 256, tiles_w = ((d->rows + 255) / 256) * tn_w;
    const uint32_t t224_w = ((d->rows + 223) / 224) * tn_w;
    int rule224 = 0;
    if (g->t224 && g->cus % 8 == 0) {
        const uint32_t C = g->cus, R = tiles_w % C;
        const double w256 = (double)(tiles_w / C) + (R ? (2 * R <= C ? 0.5 : 1.0) : 0.0);
        rule224 = 0.875 * (double)((t224_w + C - 1) / C) < 0.97 * w256;
    }
    /* K >= 8192 keeps the in-LDS widening, unless the widened weight's bf16
     * kernel takes 224-row tiles (the down projection at M = 8704: whole
     * steps 64.07 against 65.39 ms with the pass and 224-row tiles, medians
     * of 8, same box, alternating) */
    int route = g->int8_route;
    if (route == QW_INT8_AUTO)
        route = d->k >= 8192 && !(rule224 && g->t224_over_split) ? QW_INT8_W8 : QW_INT8_WIDEN;
    /* A launch of at most cus / 2 tiles widens by a pass at any row count
     * and K: the bf16 kernels' half tiles beat the whole "_w8" tiles by more
     * than the pass costs (M = 64-448, us, w8 / pass + half tiles: QKV
     * 64-66 / 48-55, out 63 / 35-38, up 65-67 / 56-59, down 74-84 / 66-76). */
    const int small_w = g->int8_route == QW_INT8_AUTO && g->half_small && 2 * tiles_w <= g->cus;
    if (small_w) route = QW_INT8_WIDEN;
    const int widen = int8 && !no_alloc && (d->rows >= g->widen_min_rows || small_w) &&
                      route == QW_INT8_WIDEN;
    const void *wptr = d->weight->ptr;
    if (widen) {
        const size_t n = (size_t)d->cols * d->k, bytes = n * 2;
        if (g->widen_bytes < bytes) {
            hipStreamSynchronize(g->stream);
            if (g->widen) hipFree(g->widen);
            g->widen = NULL;
            g->widen_bytes = 0;
            if (hipMalloc(&g->widen, bytes) != hipSuccess)
                return fail(g, "linear: widen buffer allocation (%zu bytes) failed", bytes);
            g->widen_bytes = bytes;
            g->stats.allocated_bytes += bytes; /* runtime workspaces count too */
        }
        if (!widen_launch(g, (uint16_t *)g->widen, (const int8_t *)d->weight->ptr, n)) return 0;
        wptr = g->widen;
    }
    qw_gemm_args a;
    a.a = (const uint16_t *)d->in->ptr + d->in_offset;
    a.w = wptr;
    a.wscale = d->wscale ? (const float *)d->wscale->ptr : NULL;
    a.bias = d->bias ? (const uint16_t *)d->bias->ptr : NULL;
    a.out = (uint16_t *)d->out->ptr + d->out_offset;
    a.gate = gate;
    a.row_map = row_map;
    a.m = d->rows;
    a.n = d->cols;
    a.k = d->k;
    a.lda = d->lda;
    a.ldc = d->ldc;
    a.gate_row_stride = gate_stride;
    {
        const uint64_t ab = ((uint64_t)(d->rows - 1) * d->lda + d->k) * 2;
        const uint64_t wb = (uint64_t)d->cols * d->k * (int8 && !widen ? 1 : 2);
        const uint64_t ob = ((uint64_t)(d->rows - 1) * d->ldc + d->cols) * 2;
        if (ab >= (1ull << 31) || wb >= (1ull << 31) || ob >= (1ull << 31))
            return fail(g, "linear: operand exceeds 2 GiB buffer range");
        a.a_bytes = (uint32_t)ab;
        a.w_bytes = (uint32_t)wb;
        a.out_bytes = (uint32_t)ob;
    }
    const int qkn = d->epilogue == QW_LINEAR_QKNORM;
    /* the 4-wave kernels (one wave per SIMD, 128 x 128 per wave). Same box,
     * alternating, M = 8704, us, against the 8-wave 16x16x32 kernels they
     * replaced (two waves per SIMD, 64 x 128 per wave): QKV 447 / 458, out
     * 149 / 155, up (GELU) 537 / 554, down 598 / 623. */
    const int kid = (int8 && !widen ? K_GEMM_W8_STORE_Q : K_GEMM_BF16_STORE_Q) + d->epilogue;
    const unsigned threads = 256, bm = 256, bn = 256;
    a.norm_q = qkn ? (const uint16_t *)d->norm_q->ptr : NULL;
    a.norm_k = qkn ? (const uint16_t *)d->norm_k->ptr : NULL;
    a.rope_cos = qkn ? (const float *)d->rope_cos->ptr : NULL;
    a.rope_sin = qkn ? (const float *)d->rope_sin->ptr : NULL;
    a.rope_rows = qkn ? d->rope_rows : 1;
    a.qk_cols = qkn ? d->cols / 3 * 2 : 0;
    a.eps = qkn ? d->eps : 0.0f;
    a.tiles_m = (d->rows + bm - 1) / bm;
    a.tiles_n = (d->cols + bn - 1) / bn;
    const uint32_t tiles = a.tiles_m * a.tiles_n;
    a.dp_tiles = tiles;
    a.split = 1;
    a.sk_part = NULL;
    a.sk_flag = NULL;
    uint32_t grid = tiles;
    int small = 0;
    /* 224-row tiles where they leave fewer (work-weighted) waves than
     * 256-row tiles with their half-tile tail: a wave of 224-row tiles is
     * 0.875 of one of 256-row tiles. Out projection, M = 8704: 2 waves of
     * 0.875 (468 tiles) against 2 waves (408 tiles). */
    const uint32_t t224 = ((d->rows + 223) / 224) * a.tiles_n;
    int use224 = 0;
    if (!(int8 && !widen) && g->t224 && g->cus % 8 == 0) {
        const uint32_t C = g->cus, R = tiles % C;
        const double w256 = (double)(tiles / C) + (R ? (2 * R <= C ? 0.5 : 1.0) : 0.0);
        const double w224 = 0.875 * (double)((t224 + C - 1) / C);
        use224 = w224 < 0.97 * w256;
    }
    if (no_alloc) {
        const uint32_t s = split_choice(g, tiles, d->k / 64, QW_STATIC_PARTS);
        if (s > 1) {
            const uint32_t R = tiles % g->cus;
            const size_t need = (size_t)R * s * QW_STATIC_PART_BYTES;
            /* split_choice caps R s at QW_STATIC_PARTS and R < cus: an
             * internal invariant, checked so a change to either fails loudly */
            if (need > (size_t)QW_STATIC_PARTS * QW_STATIC_PART_BYTES || R > QW_STATIC_FLAGS)
                return fail(g, "linear_static: internal error: %u split pieces over the static "
                               "workspace's %u", R * s, QW_STATIC_PARTS);
            uint32_t *flags = (uint32_t *)(g->static_scratch +
                                           (size_t)QW_STATIC_PARTS * QW_STATIC_PART_BYTES);
            /* the counters must start at zero: a previous call leaves them
             * zero, but one that did not complete might not */
            qw_zero_args za;
            za.p = flags;
            za.count = R;
            if (!launch(g, K_ZERO, dim3(blocks_for(R, 256)), dim3(256), za)) return 0;
            a.dp_tiles = tiles - R;
            a.split = s;
            a.sk_part = (float *)g->static_scratch;
            a.sk_flag = flags;
            grid = a.dp_tiles + R * s;
        }
    } else {
        /* a launch of at most half as many tiles as CUs (bf16-W kernels)
         * runs as twice as many 128 x 256 half tiles, split in k-ranges
         * where that pays (a half tile's split pieces also re-read half the
         * partial bytes) */
        small = !(int8 && !widen) && 2 * tiles <= g->cus && g->cus % 8 == 0 && g->half_small;
        const uint32_t units = small ? 2 * tiles : tiles;
        /* half tiles of a small launch: pieces of at least 16 k-steps, all
         * in one round of CUs (a second round of short pieces costs more
         * than it saves: M = 320, K = 3072, N = 10752, 168 half tiles in 3
         * pieces 62.8 us against 37 unsplit) */
        /* where 224-row tiles fill the waves better they also beat split
         * tiles (down projection shape, bf16 W, M = 8704: 500 us unsplit on
         * 224-row tiles against 568 with 256-row tiles and a 3-piece tail) */
        const uint32_t s = small ? small_split_choice(g, units, d->k / 64)
                         : use224 && g->t224_over_split ? 1u
                                                        : split_choice(g, units, d->k / 64);
        if (s > 1) {
            if (!g->sk_part) {
                hipStreamSynchronize(g->stream);
                const size_t n = (size_t)QW_SPLIT_MAX_PIECES * g->cus;
                g->stats.allocated_bytes += n * 256 * 256 * 4 + (size_t)g->cus * 4;
                if (hipMalloc((void **)&g->sk_part, n * 256 * 256 * 4) != hipSuccess) {
                    g->sk_part = NULL;
                    return fail(g, "linear: split-tile workspace allocation failed");
                }
                if (hipMalloc((void **)&g->sk_flag, (size_t)g->cus * 4) != hipSuccess ||
                    hipMemset(g->sk_flag, 0, (size_t)g->cus * 4) != hipSuccess) {
                    hipFree(g->sk_part);
                    g->sk_part = NULL;
                    g->sk_flag = NULL;
                    return fail(g, "linear: split-tile flag allocation failed");
                }
            }
            const uint32_t R = units % g->cus;
            /* the workspace holds QW_SPLIT_MAX_PIECES * cus partials and
             * cus counters; split_choice keeps within both */
            if ((uint64_t)R * s > (uint64_t)QW_SPLIT_MAX_PIECES * g->cus || R > g->cus)
                return fail(g, "linear: %u x %u split pieces exceed the partial workspace", R, s);
            a.dp_tiles = small ? 0 : tiles - R;
            a.split = s;
            a.sk_part = g->sk_part;
            a.sk_flag = g->sk_flag;
            grid = a.dp_tiles + R * s;
        }
    }
    /* bf16-weight kernels without split tiles: one workgroup per CU walks
     * the tiles, so a tile's output stores drain under the next tile's first
     * loads (up 521 -> 514 us, QKV 365 -> 359 us against one workgroup per
     * tile) */
    a.half_from = 0;
    a.half_count = 0;
    a.half3 = g->half3;
    if (small) {
        if (g->half3) /* one half tile (or piece of one) per workgroup, three stages */
            return launch(g, K_GEMM_BF16_STORE_H3 + d->epilogue,
                          dim3(2 * tiles * (a.split > 1 ? a.split : 1)), dim3(threads), a);
        if (a.split > 1) {
            a.half_count = 1; /* the split tiles run as half tiles */
        } else {
            a.half_count = 2 * tiles;
            grid = 2 * tiles;
        }
        return launch(g, kid, dim3(grid), dim3(threads), a);
    }
    if (a.split == 1 && use224) {
        a.tiles_m = (d->rows + 223) / 224;
        return launch(g, K_GEMM_BF16_STORE_T224 + d->epilogue,
                      dim3(t224 < g->cus ? t224 : g->cus), dim3(threads), a);
    }
    if (a.split == 1 && grid > g->cus && g->cus % 8 == 0) {
        grid = g->cus;
        /* a last wave of at most half the CUs' tiles runs as twice as many
         * half tiles (bf16 W kernels): up projection at M = 8704, 96 tail
         * tiles of 1632, 577-580 us against 511 us for the 1536 tiles of
         * M = 8192 */
        const uint32_t R = tiles % g->cus;
        if (R && 2 * R <= g->cus && !(int8 && !widen)) {
            a.half_from = tiles - R;
            a.half_count = 2 * R;
        }
    }
    return launch(g, kid, dim3(grid), dim3(threads), a);
}

extern "C" int qw_gpu_linear(h3_gpu *g, const qw_linear_desc *d) { return linear_impl(g, d, 0); }

extern "C" int qw_gpu_linear_static(h3_gpu *g, const qw_linear_desc *d) {
    if (!g) return 0;
    if (!g->static_scratch) return fail(g, "linear_static: no static workspace");
    /* every context on this device shares the workspace: this call's
     * kernels wait for the last call that used it, from any stream */
    hipError_t e = (hipError_t)qw_static_scratch_acquire(g->device, g->stream);
    if (e != hipSuccess) return fail(g, "linear_static: ordering: %s", hipGetErrorString(e));
    const int ok = linear_impl(g, d, 1);
    e = (hipError_t)qw_static_scratch_release(g->device, g->stream);
    if (e != hipSuccess) return fail(g, "linear_static: ordering: %s", hipGetErrorString(e));
    return ok;
}

static qw_linear_desc plain_linear(h3_gpu_tensor *out, const h3_gpu_tensor *in,
                                   const h3_gpu_tensor *w, const h3_gpu_tensor *bias,
                                   uint32_t rows, uint32_t k, uint32_t n) {
    qw_linear_desc d;
    memset(&d, 0, sizeof(d));
    d.out = out;
    d.ldc = n;
    d.in = in;
    d.lda = k;
    d.weight = w;
    d.bias = bias;
    d.rows = rows;
    d.k = k;
    d.cols = n;
    d.epilogue = QW_LINEAR_STORE;
    return d;
}

extern "C" int h3_gpu_linear_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in,
                                  const h3_gpu_tensor *w, const h3_gpu_tensor *bias,
                                  uint32_t rows, uint32_t k, uint32_t n) {
    if (!w || w->dtype != H3_GPU_BF16) return fail(g, "linear_bf16: weight must be bf16");
    qw_linear_desc d = plain_linear(out, in, w, bias, rows, k, n);
    return qw_gpu_linear(g, &d);
}

extern "C" int qw_gpu_qkv_bf16(h3_gpu *g, h3_gpu_tensor *qo, h3_gpu_tensor *ko,
                               h3_gpu_tensor *vo, const h3_gpu_tensor *in,
                               const h3_gpu_tensor *wq, const h3_gpu_tensor *wk,
                               const h3_gpu_tensor *wv, uint32_t rows, uint32_t dim) {
    return h3_gpu_linear_bf16(g, qo, in, wq, NULL, rows, dim, dim) &&
           h3_gpu_linear_bf16(g, ko, in, wk, NULL, rows, dim, dim) &&
           h3_gpu_linear_bf16(g, vo, in, wv, NULL, rows, dim, dim);
}

static void *scratch(h3_gpu *g, size_t bytes) {
    if (g->scratch_bytes >= bytes) return g->scratch;
    hipStreamSynchronize(g->stream);
    if (g->scratch) hipFree(g->scratch);
    g->scratch = NULL;
    g->scratch_bytes = 0;
    if (hipMalloc(&g->scratch, bytes) != hipSuccess) return NULL;
    g->scratch_bytes = bytes;
    g->stats.allocated_bytes += bytes;
    return g->scratch;
}

extern "C" int h3_gpu_mlp_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in,
                               const h3_gpu_tensor *fc1, const h3_gpu_tensor *fc2,
                               uint32_t rows, uint32_t in_dim, uint32_t hidden,
                               uint32_t out_dim) {
    size_t wide = (size_t)rows * hidden * 2, act_n = (size_t)rows * hidden;
    unsigned char *s = (unsigned char *)scratch(g, (wide + act_n) * 2 + 512);
    if (!s) return fail(g, "mlp: scratch allocation failed");
    h3_gpu_tensor tw = {g, s, wide, H3_GPU_BF16, 0};
    h3_gpu_tensor ta = {g, s + ((wide * 2 + 255) & ~(size_t)255), act_n, H3_GPU_BF16, 0};
    return h3_gpu_linear_bf16(g, &tw, in, fc1, NULL, rows, in_dim, 2 * hidden) &&
           qw_gpu_swiglu_bf16(g, &ta, &tw, rows, hidden) &&
           h3_gpu_linear_bf16(g, out, &ta, fc2, NULL, rows, hidden, out_dim);
}

/* ---- attention ----------------------------------------------------------- */

extern "C" int qw_gpu_attention_bf16(h3_gpu *g, const qw_attention_desc *d) {
    if (!g || !d) return 0;
    REQ_DT(d->out, H3_GPU_BF16, "attention out");
    REQ_DT(d->q, H3_GPU_BF16, "attention q");
    REQ_DT(d->k, H3_GPU_BF16, "attention k");
    REQ_DT(d->v, H3_GPU_BF16, "attention v");
    if (!d->batch || !d->q_rows || !d->heads) return 1;
    if (!d->kv_rows) return fail(g, "attention: no keys");
    const uint32_t hd = d->heads * 128;
    if (d->ldq < hd || d->ldk < hd || d->ldv < hd || d->ldo < hd)
        return fail(g, "attention: row strides smaller than heads * 128");
    if (d->ldq % 8 || d->ldk % 8 || d->ldv % 8 || d->ldo % 4 || d->q_offset % 8 ||
        d->k_offset % 8 || d->v_offset % 8 || d->out_offset % 4)
        return fail(g, "attention: rows must be 16-byte aligned");
    size_t qr = (size_t)d->batch * d->q_rows, kr = (size_t)d->batch * d->kv_rows;
    if (!fits(d->q, d->q_offset, (qr - 1) * d->ldq + hd) ||
        !fits(d->k, d->k_offset, (kr - 1) * d->ldk + hd) ||
        !fits(d->v, d->v_offset, (kr - 1) * d->ldv + hd) ||
        !fits(d->out, d->out_offset, (qr - 1) * d->ldo + hd))
        return fail(g, "attention: tensor too small");
    if (d->kv_limit) {
        REQ_DT(d->kv_limit, H3_GPU_U32, "attention kv_limit");
        if (!fits(d->kv_limit, 0, d->q_rows)) return fail(g, "attention: kv_limit too small");
    }
    if (!d->kv_limit && d->text_rows > d->q_rows)
        return fail(g, "attention: text_rows > q_rows");
    qw_attn_args a;
    a.out = (uint16_t *)d->out->ptr + d->out_offset;
    a.q = (const uint16_t *)d->q->ptr + d->q_offset;
    a.k = (const uint16_t *)d->k->ptr + d->k_offset;
    a.v = (const uint16_t *)d->v->ptr + d->v_offset;
    a.kv_limit = d->kv_limit ? (const uint32_t *)d->kv_limit->ptr : NULL;
    a.q_rows = d->q_rows;
    a.kv_rows = d->kv_rows;
    a.heads = d->heads;
    a.batch = d->batch;
    a.ldq = d->ldq;
    a.ldk = d->ldk;
    a.ldv = d->ldv;
    a.ldo = d->ldo;
    a.text_rows = d->text_rows;
    a.text_causal = d->text_causal;
    a.scale = d->scale;
    a.scale_log2 = d->scale * 1.4426950408889634f;
    g->stats.mps_sdpa_dispatches += 0;
    if (((uint64_t)(d->kv_rows - 1) * std::max(d->ldk, d->ldv) + hd) * 2 >= (1ull << 31))
        return fail(g, "attention: one batch entry's K/V exceed 2 GiB");
    /* Fewer 256-query blocks than CUs: 128-query workgroups, two per CU,
     * bring the idle CUs in (the same bits; 1 x 24 heads x 1152 rows 28.7
     * against 44.3 us, 320 rows 13.4 against 18.8; at 2 x 24 x 4352 rows the
     * 256-query kernel stays ahead, 391.5 against 398.9 us). */
    const uint32_t aqb = g->attn_threads / 2; /* 32 query rows per 64-lane wave */
    const uint64_t nwg = (uint64_t)((d->q_rows + aqb - 1) / aqb) * d->heads * d->batch;
    if (nwg >= (1ull << 31)) return fail(g, "attention: grid too large");
    if (g->attn_small && nwg < g->cus) {
        const uint32_t aqb4 = g->attn4_threads / 2;
        const uint64_t nwg4 = (uint64_t)((d->q_rows + aqb4 - 1) / aqb4) * d->heads * d->batch;
        return launch(g, K_ATTN_W4, dim3((uint32_t)nwg4), dim3(g->attn4_threads), a);
    }
    return launch(g, K_ATTN, dim3((uint32_t)nwg), dim3(g->attn_threads), a);
}

static int sdpa_contig(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q,
                       const h3_gpu_tensor *k, const h3_gpu_tensor *v,
                       const h3_gpu_tensor *limit, uint32_t q_rows, uint32_t kv_rows,
                       uint32_t heads, uint32_t head_dim, float scale, uint32_t text_rows,
                       int causal) {
    if (head_dim != 128) return fail(g, "sdpa: head_dim must be 128");
    qw_attention_desc d;
    memset(&d, 0, sizeof(d));
    d.out = out;
    d.q = q;
    d.k = k;
    d.v = v;
    d.ldo = d.ldq = d.ldk = d.ldv = heads * 128;
    d.kv_limit = limit;
    d.batch = 1;
    d.q_rows = q_rows;
    d.kv_rows = kv_rows;
    d.heads = heads;
    d.text_rows = text_rows;
    d.text_causal = causal;
    d.scale = scale;
    return qw_gpu_attention_bf16(g, &d);
}

extern "C" int qw_gpu_flash_sdpa_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q,
                                      const h3_gpu_tensor *k, const h3_gpu_tensor *v,
                                      uint32_t q_rows, uint32_t kv_rows, uint32_t heads,
                                      uint32_t head_dim, float scale) {
    return sdpa_contig(g, out, q, k, v, NULL, q_rows, kv_rows, heads, head_dim, scale, 0, 0);
}

extern "C" int qw_gpu_sdpa_rect_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q,
                                     const h3_gpu_tensor *k, const h3_gpu_tensor *v,
                                     uint32_t q_rows, uint32_t kv_rows, uint32_t heads,
                                     uint32_t head_dim, float scale) {
    return sdpa_contig(g, out, q, k, v, NULL, q_rows, kv_rows, heads, head_dim, scale, 0, 0);
}

extern "C" int qw_gpu_flash_sdpa_prefix_bf16(h3_gpu *g, h3_gpu_tensor *out,
                                             const h3_gpu_tensor *q, const h3_gpu_tensor *k,
                                             const h3_gpu_tensor *v,
                                             const h3_gpu_tensor *kv_limit, uint32_t q_rows,
                                             uint32_t kv_rows, uint32_t heads, uint32_t kv_heads,
                                             uint32_t head_dim, float scale) {
    if (kv_heads != heads) return fail(g, "sdpa_prefix: grouped K/V heads not supported");
    if (!kv_limit) return fail(g, "sdpa_prefix: kv_limit required");
    return sdpa_contig(g, out, q, k, v, kv_limit, q_rows, kv_rows, heads, head_dim, scale, 0, 0);
}

extern "C" int h3_gpu_gqa_causal_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q,
                                      const h3_gpu_tensor *k, const h3_gpu_tensor *v,
                                      uint32_t seq, uint32_t qh, uint32_t kvh, uint32_t head_dim,
                                      float scale) {
    if (kvh != qh) return fail(g, "gqa_causal: grouped K/V heads not supported");
    return sdpa_contig(g, out, q, k, v, NULL, seq, seq, qh, head_dim, scale, seq, 1);
}

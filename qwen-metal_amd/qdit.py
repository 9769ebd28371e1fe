"""ctypes binding of libqwen_dit_hip.so (the C-ABI in include/*.h).

Thin plumbing for tests, smoke() and bench.py: numpy arrays in, device
tensors through the h3_gpu runtime, results back. Every call raises on a
0 return with the runtime's error string. No compute happens here.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libqwen_dit_hip.so")
HSACO_PATH = os.path.join(LIB_DIR, "qwen_kernels.hsaco")

F32, BF16, I8, U32 = 0, 1, 2, 3
_NP = {F32: np.float32, BF16: np.uint16, I8: np.int8, U32: np.uint32}
MLP_SWIGLU, MLP_GELU_TANH = 0, 1
LINEAR_STORE, LINEAR_GELU, LINEAR_GATE, LINEAR_QKNORM = 0, 1, 2, 3

vp = C.c_void_p
u32 = C.c_uint32
sz = C.c_size_t


class Stats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "allocated_bytes", "live_bytes", "peak_live_bytes", "tensor_allocations",
        "direct_dispatches", "mps_linear_dispatches", "mps_conv_dispatches",
        "mps_sdpa_dispatches", "blit_copies", "submissions")] + [
        ("command_encode_seconds", C.c_double), ("command_wait_seconds", C.c_double),
        ("gpu_seconds", C.c_double)]


class StTensor(C.Structure):
    """h3_st_tensor (include/h3_safetensors.h)"""
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_int), ("ndim", C.c_int),
                ("shape", C.c_uint64 * 8), ("data_begin", C.c_uint64),
                ("data_end", C.c_uint64), ("file_offset", C.c_uint64)]


class StHeader(C.Structure):
    """h3_st_header (include/h3_safetensors.h)"""
    _fields_ = [("path", C.c_char_p), ("file_size", C.c_uint64), ("header_size", C.c_uint64),
                ("tensors", C.POINTER(StTensor)), ("tensor_count", C.c_size_t)]


class DitConfig(C.Structure):
    _fields_ = [("hidden", u32), ("heads", u32), ("mlp_width", u32), ("text_dim", u32),
                ("z_dim", u32), ("layers", u32), ("mlp_act", C.c_int),
                ("adaln_shift", C.c_int), ("has_bias", C.c_int),
                ("text_causal", C.c_int), ("int8_weights", C.c_int)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class LinearDesc(C.Structure):
    _fields_ = [("out", vp), ("out_offset", sz), ("ldc", u32), ("in_", vp),
                ("in_offset", sz), ("lda", u32), ("weight", vp), ("wscale", vp),
                ("bias", vp), ("rows", u32), ("k", u32), ("cols", u32),
                ("epilogue", C.c_int), ("modulation", vp), ("row_map", vp),
                ("slots", u32), ("gate_slot", u32), ("norm_q", vp), ("norm_k", vp),
                ("rope_cos", vp), ("rope_sin", vp), ("rope_rows", u32), ("eps", C.c_float)]


class AttentionDesc(C.Structure):
    _fields_ = [("out", vp), ("out_offset", sz), ("ldo", u32), ("q", vp), ("k", vp),
                ("v", vp), ("q_offset", sz), ("k_offset", sz), ("v_offset", sz),
                ("ldq", u32), ("ldk", u32), ("ldv", u32), ("kv_limit", vp),
                ("batch", u32), ("q_rows", u32), ("kv_rows", u32), ("heads", u32),
                ("text_rows", u32), ("text_causal", C.c_int), ("scale", C.c_float)]


# Every exported entry point with its (restype, argtypes). The CPU test
# checks the library exports each name declared in include/*.h.
SIGNATURES = {
    "h3_gpu_create": (vp, [C.c_char_p, C.c_char_p, sz]),
    "h3_gpu_free": (None, [vp]),
    "h3_gpu_tensor_new_f32": (vp, [vp, sz]),
    "h3_gpu_tensor_new_bf16": (vp, [vp, sz]),
    "h3_gpu_tensor_new_i8": (vp, [vp, sz]),
    "h3_gpu_tensor_new_u32": (vp, [vp, sz]),
    "h3_gpu_tensor_from_f32": (vp, [vp, vp, sz]),
    "h3_gpu_tensor_from_bf16": (vp, [vp, vp, sz]),
    "h3_gpu_tensor_from_u32": (vp, [vp, vp, sz]),
    "h3_gpu_tensor_view": (vp, [vp, sz, sz]),
    "h3_gpu_tensor_free": (None, [vp]),
    "h3_gpu_tensor_elements": (sz, [vp]),
    "h3_gpu_tensor_dtype": (C.c_int, [vp]),
    "h3_gpu_tensor_read_f32": (C.c_int, [vp, vp, sz]),
    "h3_gpu_tensor_read_f32_range": (C.c_int, [vp, sz, vp, sz]),
    "h3_gpu_tensor_read_bf16": (C.c_int, [vp, vp, sz]),
    "h3_gpu_tensor_write_f32": (C.c_int, [vp, vp, sz]),
    "h3_gpu_tensor_write_f32_range": (C.c_int, [vp, sz, vp, sz]),
    "h3_gpu_tensor_write_bf16": (C.c_int, [vp, vp, sz]),
    "h3_gpu_tensor_write_bf16_range": (C.c_int, [vp, sz, vp, sz]),
    "h3_gpu_tensor_read_bytes": (C.c_int, [vp, vp, sz]),
    "h3_gpu_tensor_write_bytes": (C.c_int, [vp, vp, sz]),
    "h3_gpu_tensor_device_ptr": (vp, [vp]),
    "h3_gpu_begin": (C.c_int, [vp]),
    "h3_gpu_continue": (C.c_int, [vp]),
    "h3_gpu_submit": (C.c_int, [vp]),
    "h3_gpu_error": (C.c_char_p, [vp]),
    "h3_gpu_get_stats": (C.c_int, [vp, C.POINTER(Stats)]),
    "h3_gpu_profile_set_label": (None, [vp, C.c_char_p]),
    "h3_gpu_profile_mark": (None, [vp, C.c_char_p]),
    "h3_gpu_timer_begin": (C.c_int, [vp]),
    "h3_gpu_timer_end": (C.c_double, [vp]),
    "h3_gpu_linear_bf16": (C.c_int, [vp, vp, vp, vp, vp, u32, u32, u32]),
    "h3_gpu_mlp_bf16": (C.c_int, [vp, vp, vp, vp, vp, u32, u32, u32, u32]),
    "h3_gpu_quantize_weight_int8": (C.c_int, [vp, vp, vp, vp, u32, u32]),
    "h3_gpu_silu_bf16": (C.c_int, [vp, vp, vp, u32]),
    "h3_gpu_gelu_bf16": (C.c_int, [vp, vp, vp, u32, C.c_int]),
    "h3_gpu_gate_bf16": (C.c_int, [vp, vp, vp, vp, vp, vp, u32, u32, u32, u32]),
    "h3_gpu_head_rms_norm_bf16": (C.c_int, [vp, vp, vp, u32, u32, u32, C.c_float]),
    "h3_gpu_gqa_causal_bf16": (C.c_int, [vp, vp, vp, vp, vp, u32, u32, u32, u32, C.c_float]),
    "h3_gpu_cast_f32_to_bf16": (C.c_int, [vp, vp, vp, u32]),
    "h3_gpu_copy_bf16": (C.c_int, [vp, vp, sz, vp, sz, sz]),
    "qw_gpu_layer_norm_mod_bf16": (C.c_int, [vp, vp, vp, vp, vp, u32, u32, u32, u32, C.c_float]),
    "qw_gpu_rms_norm_one_bf16": (C.c_int, [vp, vp, vp, vp, u32, u32, C.c_float]),
    "qw_gpu_tanh_bf16": (C.c_int, [vp, vp, vp, u32]),
    "qw_gpu_qk_rope_bf16": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, u32, u32, u32]),
    "qw_gpu_swiglu_bf16": (C.c_int, [vp, vp, vp, u32, u32]),
    "qw_gpu_flash_sdpa_bf16": (C.c_int, [vp, vp, vp, vp, vp, u32, u32, u32, u32, C.c_float]),
    "qw_gpu_flash_sdpa_prefix_bf16": (C.c_int, [vp, vp, vp, vp, vp, vp, u32, u32, u32, u32,
                                                u32, C.c_float]),
    "qw_gpu_qkv_bf16": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, u32, u32]),
    "qw_gpu_sdpa_rect_bf16": (C.c_int, [vp, vp, vp, vp, vp, u32, u32, u32, u32, C.c_float]),
    "qw_gpu_layer_norm_mod_shift_bf16": (C.c_int, [vp, vp, vp, vp, vp, u32, u32, u32, u32,
                                                   C.c_int32, C.c_float]),
    "qw_gpu_linear": (C.c_int, [vp, C.POINTER(LinearDesc)]),
    "qw_gpu_linear_static": (C.c_int, [vp, C.POINTER(LinearDesc)]),
    "qw_gpu_qk_norm_rope_bf16": (C.c_int, [vp, vp, u32, u32, u32, u32, vp, vp, vp, vp, u32,
                                           C.c_float]),
    "qw_gpu_attention_bf16": (C.c_int, [vp, C.POINTER(AttentionDesc)]),
    "qw_gpu_modulation_reorder_bf16": (C.c_int, [vp, vp, vp, u32, u32, C.c_int]),
    "qw_gpu_fill_normal_bf16": (C.c_int, [vp, vp, sz, sz, C.c_uint64, C.c_uint64, C.c_float,
                                          C.c_float]),
    "qw_gpu_dequant_int8_f32": (C.c_int, [vp, vp, vp, vp, u32, u32]),
    "qw_gpu_widen_int8_bf16": (C.c_int, [vp, vp, vp, sz]),
    "qw_gpu_cfg_euler_f32": (C.c_int, [vp, vp, vp, sz, vp, sz, sz, C.c_float, C.c_float]),
    "qw_gpu_copy_rows": (C.c_int, [vp, vp, sz, u32, vp, sz, u32, u32, u32]),
    "qw_dit_config_reference": (None, [C.POINTER(DitConfig)]),
    "qw_dit_config_baseline": (None, [C.POINTER(DitConfig)]),
    "qw_dit_create": (vp, [vp, C.c_char_p, C.c_int, C.c_char_p, sz]),
    "qw_dit_create_random": (vp, [vp, C.POINTER(DitConfig), C.c_uint64, C.c_char_p, sz]),
    "qw_dit_free": (None, [vp]),
    "qw_dit_get_config": (C.POINTER(DitConfig), [vp]),
    "qw_dit_block_tensor": (vp, [vp, C.c_int, C.c_int]),
    "qw_dit_block_scales": (vp, [vp, C.c_int, C.c_int]),
    "qw_dit_embed": (C.c_int, [vp, vp, u32, vp, u32, vp, C.c_char_p, sz]),
    "qw_dit_timestep_features": (None, [vp, sz, vp]),
    "qw_dit_conditioning": (C.c_int, [vp, vp, u32, vp, vp, vp, C.c_char_p, sz]),
    "qw_dit_block": (C.c_int, [vp, C.c_int, vp, vp, vp, vp, vp, u32, u32, vp, vp, u32, vp, vp,
                               vp, C.c_char_p, sz]),
    "qw_dit_prefix_limits": (None, [vp, u32, vp]),
    "qw_dit_final": (C.c_int, [vp, vp, vp, vp, u32, vp, C.c_char_p, sz]),
    "qw_dit_forward": (C.c_int, [vp, vp, u32, vp, u32, C.c_float, vp, vp, vp, C.c_char_p, sz]),
    "qw_dit_forward_batch": (C.c_int, [vp, vp, u32, vp, u32, u32, C.c_float, vp, vp, vp,
                                       C.c_char_p, sz]),
    "qw_dit_forward_batch_features": (C.c_int, [vp, vp, u32, vp, u32, u32, vp, sz, vp, vp, vp,
                                                C.c_char_p, sz]),
    "qw_dit_block_profile": (C.c_int, [vp, vp, C.c_int]),
    "qw_dit_set_trace": (C.c_int, [vp, vp, vp]),
    "qw_dit_apply_lora": (C.c_int, [vp, C.c_char_p, C.c_float, C.c_char_p, sz]),
    "qw_dit_remove_lora": (C.c_int, [vp, C.c_char_p, C.c_char_p, sz]),
    "qw_dit_switch_lora": (C.c_int, [vp, C.c_char_p, C.c_float, C.c_char_p, sz]),
    "qw_dit_clear_lora": (C.c_int, [vp, C.c_char_p, sz]),
    "qw_dit_lora_count": (C.c_int, [vp]),
    "qw_dit_lora_path_at": (C.c_char_p, [vp, C.c_int]),
    "qw_dit_lora_scale_at": (C.c_float, [vp, C.c_int]),
    "qw_gpu_lora_fuse_bf16": (C.c_int, [vp, vp, vp, u32, u32, vp, u32]),
    "qw_dit_embed_segments": (C.c_int, [vp, vp, vp, vp, u32, vp, C.c_char_p, sz]),
    "qw_dit_forward_ti2i": (C.c_int, [vp, vp, vp, vp, u32, u32, vp, vp, C.c_float, vp,
                                      C.c_char_p, sz]),
    "qw_dit_ti2i_cache_clear": (None, [vp]),
    "qw_latent_grid": (C.c_int, [C.c_int, C.c_int, vp, vp]),
    "qw_calculate_shift": (C.c_double, [C.c_int]),
    "qw_schedule_build": (C.c_int, [C.c_int, C.c_int, vp]),
    "qw_schedule_from_sigmas": (C.c_int, [vp, C.c_int, vp]),
    "qw_euler_velocity_step": (None, [vp, vp, sz, C.c_float, C.c_float]),
    "qw_rope_build": (C.c_int, [vp, C.c_int, vp]),
    "qw_rope_free": (None, [vp]),
    "qw_rope_row": (C.c_int, [C.c_int]),
    "qw_rng_seed": (None, [vp, C.c_uint64]),
    "qw_rng_u32": (C.c_uint32, [vp]),
    "qw_rng_normal": (C.c_float, [vp]),
    "qw_rng_fill_normal": (None, [vp, vp, sz]),
    "qw_sched_cfg_default": (None, [vp]),
    "qw_pipe_schedule": (C.c_int, [u32, u32, vp, u32, vp, vp, C.c_char_p, sz]),
    "qw_pipe_rope_tables": (C.c_int, [vp, u32, u32, u32, vp, vp, C.c_char_p, sz]),
    "qw_pipe_rope_tables_host": (None, [u32, u32, u32, vp, vp]),
    "qw_pipe_rope_tables_blocks": (C.c_int, [vp, vp, vp, vp, u32, vp, vp, C.c_char_p, sz]),
    "qw_gpu_span_begin": (C.c_int, [vp, C.c_int]),
    "qw_gpu_span_end": (C.c_int, [vp]),
    "qw_gpu_span_collect": (C.c_int, [vp, vp, vp, C.c_int]),
    "qw_dit_set_spans": (C.c_int, [vp, C.c_int]),
    "qw_pipe_rope_tables_blocks_host": (sz, [vp, vp, vp, u32, vp, vp]),
    "h3_st_read_header": (C.c_int, [C.c_char_p, vp, C.c_char_p, sz]),
    "h3_st_free_header": (None, [vp]),
    "h3_st_find": (vp, [vp, C.c_char_p]),
    "h3_st_tensor_elements": (C.c_uint64, [vp]),
    "h3_st_read_data": (C.c_int, [vp, vp, vp, sz, C.c_char_p, sz]),
    "h3_dtype_size": (sz, [C.c_int]),
    "h3_dtype_name": (C.c_char_p, [C.c_int]),
    "h3_weight_store_open": (vp, [C.c_char_p, C.c_char_p, sz]),
    "h3_weight_store_free": (None, [vp]),
    "h3_weight_store_shards": (sz, [vp]),
    "h3_weight_find": (vp, [vp, C.c_char_p, vp]),
    "h3_weight_load_bf16": (vp, [vp, vp, C.c_char_p, C.c_int, vp, C.c_char_p, sz]),
    "h3_weight_load_f32": (vp, [vp, vp, C.c_char_p, C.c_int, vp, C.c_char_p, sz]),
    "h3_weight_read_bf16_into": (C.c_int, [vp, C.c_char_p, C.c_int, vp, vp, sz, C.c_char_p,
                                           sz]),
    "qw_dit_load": (vp, [vp, C.c_char_p, C.POINTER(DitConfig), C.c_char_p, sz]),
    "qw_pipe_denoise": (C.c_int, [vp, vp, vp, u32, vp, u32, vp, u32, u32, u32, C.c_float, vp,
                                  u32, vp, C.c_char_p, sz]),
}

_LIB = None


def lib():
    """Load the product library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C qwen-metal_amd`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _p(a):
    return a.ctypes.data_as(vp)


class Tensor:
    def __init__(self, gpu, handle, n, dtype, owner=None):
        self.gpu, self.h, self.n, self.dtype, self._owner = gpu, handle, n, dtype, owner

    def read(self, n=None):
        n = self.n if n is None else n
        out = np.empty(n, _NP[self.dtype])
        self.gpu.check(lib().h3_gpu_tensor_read_bytes(self.h, _p(out), out.nbytes), "read")
        return out

    def write(self, arr):
        arr = np.ascontiguousarray(arr, dtype=_NP[self.dtype]).ravel()
        assert arr.size <= self.n
        self.gpu.check(lib().h3_gpu_tensor_write_bytes(self.h, _p(arr), arr.nbytes), "write")

    def view(self, offset, n):
        h = lib().h3_gpu_tensor_view(self.h, offset, n)
        if not h:
            raise RuntimeError(self.gpu.error())
        return Tensor(self.gpu, h, n, self.dtype, owner=self)

    def free(self):
        # a tensor outliving its context is left to process exit
        if self.h and self.gpu.h:
            lib().h3_gpu_tensor_free(self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Gpu:
    def __init__(self, hsaco=None):
        err = C.create_string_buffer(1024)
        self.h = lib().h3_gpu_create((hsaco or HSACO_PATH).encode(), err, 1024)
        if not self.h:
            raise RuntimeError("h3_gpu_create: " + err.value.decode())
        self._keep = []

    def error(self):
        return lib().h3_gpu_error(self.h).decode()

    def check(self, ok, what=""):
        if not ok:
            raise RuntimeError(f"{what}: {self.error()}")

    def new(self, n, dtype):
        fn = {F32: "h3_gpu_tensor_new_f32", BF16: "h3_gpu_tensor_new_bf16",
              I8: "h3_gpu_tensor_new_i8", U32: "h3_gpu_tensor_new_u32"}[dtype]
        h = getattr(lib(), fn)(self.h, n)
        if not h:
            raise RuntimeError(self.error())
        return Tensor(self, h, n, dtype)

    def put(self, arr, dtype=None):
        """Upload arr into a new device tensor. The context keeps the tensor
        alive until release(), so an inline `gpu.put(x).h` handed to a
        kernel cannot be freed (and its memory reused) before the kernel
        runs."""
        arr = np.ascontiguousarray(arr)
        if dtype is None:
            dtype = {np.dtype(np.float32): F32, np.dtype(np.uint16): BF16,
                     np.dtype(np.int8): I8, np.dtype(np.uint32): U32}[arr.dtype]
        t = self.new(arr.size, dtype)
        if arr.size:
            t.write(arr)
        self._keep.append(t)
        return t

    def release(self):
        """Drop the keep-alive references of put() (after a submit)."""
        lib().h3_gpu_submit(self.h)
        self._keep = []

    def submit(self):
        self.check(lib().h3_gpu_submit(self.h), "submit")
        lib().h3_gpu_begin(self.h)

    def stats(self):
        s = Stats()
        lib().h3_gpu_get_stats(self.h, C.byref(s))
        return s

    def timer_begin(self):
        self.check(lib().h3_gpu_timer_begin(self.h), "timer")

    def timer_end(self):
        ms = lib().h3_gpu_timer_end(self.h)
        if ms < 0:
            raise RuntimeError("timer_end failed")
        return ms

    def close(self):
        if self.h:
            self.release()
            lib().h3_gpu_free(self.h)
            self.h = None

    # ---- dispatch helpers (enqueue only) ----
    def linear(self, out, inp, weight, rows, k, cols, bias=None, wscale=None,
               epilogue=LINEAR_STORE, ldc=None, lda=None, out_offset=0, in_offset=0,
               modulation=None, row_map=None, slots=0, gate_slot=0, qknorm=None,
               no_alloc=False):
        """qknorm = (norm_q, norm_k, rope_cos, rope_sin, rope_rows, eps) with
        epilogue LINEAR_QKNORM; no_alloc: qw_gpu_linear_static"""
        nq, nk, rc, rs, rr, eps = qknorm if qknorm else (None, None, None, None, 0, 0.0)
        h = lambda t: t.h if t is not None else None  # noqa: E731
        d = LinearDesc(out.h, out_offset, ldc or cols, inp.h, in_offset, lda or k, weight.h,
                       h(wscale), h(bias), rows, k, cols, epilogue, h(modulation), h(row_map),
                       slots, gate_slot, h(nq), h(nk), h(rc), h(rs), rr, eps)
        fn = lib().qw_gpu_linear_static if no_alloc else lib().qw_gpu_linear
        self.check(fn(self.h, C.byref(d)), "linear")

    def attention(self, out, q, k, v, batch, q_rows, kv_rows, heads, ldq, ldk, ldv, ldo,
                  q_offset=0, k_offset=0, v_offset=0, kv_limit=None, text_rows=0,
                  text_causal=0, scale=None):
        scale = 1.0 / np.sqrt(128.0) if scale is None else scale
        d = AttentionDesc(out.h, 0, ldo, q.h, k.h, v.h, q_offset, k_offset, v_offset, ldq, ldk,
                          ldv, kv_limit.h if kv_limit else None, batch, q_rows, kv_rows, heads,
                          text_rows, text_causal, scale)
        self.check(lib().qw_gpu_attention_bf16(self.h, C.byref(d)), "attention")


class Dit:
    def __init__(self, gpu, cfg: dict, seed: int = 0, model_dir=None):
        """Seeded random weights (qw_dit_create_random), or with model_dir
        the safetensors checkpoint under model_dir/transformer (qw_dit_load)."""
        self.gpu = gpu
        c = DitConfig(**cfg)
        err = C.create_string_buffer(1024)
        if model_dir is not None:
            self.h = lib().qw_dit_load(gpu.h, str(model_dir).encode(), C.byref(c), err, 1024)
            if not self.h:
                raise RuntimeError("qw_dit_load: " + err.value.decode())
        else:
            self.h = lib().qw_dit_create_random(gpu.h, C.byref(c), seed, err, 1024)
            if not self.h:
                raise RuntimeError("qw_dit_create_random: " + err.value.decode())
        self.cfg = lib().qw_dit_get_config(self.h).contents

    def forward_batch(self, text_in, text_rows, latents, image_rows, batch, sigma, rope_cos,
                      rope_sin, output):
        err = C.create_string_buffer(1024)
        ok = lib().qw_dit_forward_batch(self.h, text_in.h if text_in else None, text_rows,
                                        latents.h, image_rows, batch, sigma, rope_cos.h,
                                        rope_sin.h, output.h, err, 1024)
        if not ok:
            raise RuntimeError("forward_batch: " + err.value.decode())

    def block(self, layer, hidden, modulation, rope_cos, rope_sin, row_map, rows, text_rows,
              kv_limit=None, k_out=None, v_out=None, debug_attn=None):
        err = C.create_string_buffer(1024)
        h = lambda t: t.h if t is not None else None  # noqa: E731
        ok = lib().qw_dit_block(self.h, layer, hidden.h, modulation.h, rope_cos.h, rope_sin.h,
                                row_map.h, rows, text_rows, h(kv_limit), None, 0, h(k_out),
                                h(v_out), h(debug_attn), err, 1024)
        if not ok:
            raise RuntimeError("block: " + err.value.decode())

    def block_tensor(self, block, field):
        return lib().qw_dit_block_tensor(self.h, block, field)

    def close(self):
        if self.h:
            lib().qw_dit_free(self.h)
            self.h = None

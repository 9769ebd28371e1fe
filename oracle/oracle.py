"""ctypes view of the CPU oracle (liboracle.so) — TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
as the checker; the product library never loads it. bf16 arrays are numpy
uint16 bit patterns.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
SZ = C.c_size_t


class QoRng(C.Structure):
    _fields_ = [("state", C.c_uint64), ("increment", C.c_uint64),
                ("spare", C.c_float), ("has_spare", C.c_int)]


class QoConfig(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("heads", C.c_uint32),
                ("mlp_width", C.c_uint32), ("text_dim", C.c_uint32),
                ("z_dim", C.c_uint32), ("layers", C.c_uint32),
                ("mlp_act", C.c_int), ("adaln_shift", C.c_int),
                ("has_bias", C.c_int), ("text_causal", C.c_int),
                ("int8_weights", C.c_int)]


class QoLin(C.Structure):
    _fields_ = [("w", C.POINTER(C.c_uint16)), ("q", C.POINTER(C.c_int8)),
                ("scales", C.POINTER(C.c_float)),
                ("bias", C.POINTER(C.c_uint16)), ("n", C.c_uint32),
                ("k", C.c_uint32), ("int8", C.c_int)]


class QoLayer(C.Structure):
    _fields_ = [("qkv", QoLin), ("out", QoLin), ("fc1", QoLin), ("fc2", QoLin),
                ("norm_q", C.POINTER(C.c_uint16)),
                ("norm_k", C.POINTER(C.c_uint16))]


class QoModel(C.Structure):
    _fields_ = [("cfg", QoConfig), ("layer", C.POINTER(QoLayer)),
                ("img_in", QoLin), ("txt_in1", QoLin), ("txt_in2", QoLin),
                ("time_l1", QoLin), ("time_l2", QoLin), ("mod", QoLin),
                ("norm_out", QoLin), ("proj_out", QoLin),
                ("txt_norm", C.POINTER(C.c_uint16))]


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = C.CDLL(path)
        L.qo_f32_to_bf16.restype = C.c_uint16
        L.qo_f32_to_bf16.argtypes = [C.c_float]
        L.qo_f32_to_bf16_trunc.restype = C.c_uint16
        L.qo_f32_to_bf16_trunc.argtypes = [C.c_float]
        L.qo_bf16_to_f32.restype = C.c_float
        L.qo_bf16_to_f32.argtypes = [C.c_uint16]
        L.qo_rng_seed.argtypes = [C.POINTER(QoRng), C.c_uint64]
        L.qo_rng_u32.restype = C.c_uint32
        L.qo_rng_u32.argtypes = [C.POINTER(QoRng)]
        L.qo_rng_normal.restype = C.c_float
        L.qo_rng_normal.argtypes = [C.POINTER(QoRng)]
        L.qo_rng_fill_normal.argtypes = [C.POINTER(QoRng), f32p, SZ]
        L.qo_calculate_shift.restype = C.c_double
        L.qo_calculate_shift.argtypes = [C.c_int]
        L.qo_schedule_build.restype = C.c_int
        L.qo_schedule_build.argtypes = [C.c_int, C.c_int, f32p]
        L.qo_schedule_exp_mu.restype = C.c_int
        L.qo_schedule_exp_mu.argtypes = [C.c_int, C.c_double, C.c_double, f32p]
        L.qo_euler_step.argtypes = [f32p, f32p, SZ, C.c_float, C.c_float]
        L.qo_rope_table_entry.argtypes = [C.c_int, C.c_int, C.c_int,
                                          C.POINTER(C.c_float),
                                          C.POINTER(C.c_float)]
        L.qo_rope_tables.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, f32p,
                                     f32p]
        L.qo_rope_tables_blocks.restype = SZ
        L.qo_rope_tables_blocks.argtypes = [u32p, u32p, u32p, C.c_uint32, f32p, f32p]
        L.qo_timestep_features.argtypes = [f32p, SZ, f32p]
        L.qo_synth_normal.restype = C.c_float
        L.qo_synth_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.qo_fill_normal_bf16.argtypes = [u16p, SZ, C.c_uint64, C.c_uint64,
                                          C.c_float, C.c_float]
        L.qo_gemm_nt_f32.argtypes = [f32p, SZ, f32p, SZ, f32p, SZ, SZ, SZ, SZ]
        L.qo_linear.argtypes = [u16p, SZ, u16p, SZ, u16p, C.c_void_p, SZ, SZ,
                                SZ]
        L.qo_linear_i8.argtypes = [u16p, SZ, u16p, SZ, i8p, f32p, C.c_void_p,
                                   SZ, SZ, SZ]
        L.qo_quantize_int8_rows.argtypes = [i8p, f32p, u16p, SZ, SZ]
        L.qo_dequant_int8_rows.argtypes = [f32p, i8p, f32p, SZ, SZ]
        L.qo_layer_norm_mod.argtypes = [u16p, u16p, u16p, u32p, SZ, SZ,
                                        C.c_uint32, C.c_uint32, C.c_int,
                                        C.c_float]
        L.qo_layer_norm_mod_r.argtypes = L.qo_layer_norm_mod.argtypes + [C.c_int]
        L.qo_gate_r.argtypes = [u16p, u16p, u16p, u16p, u32p, SZ, SZ,
                                C.c_uint32, C.c_uint32, C.c_int]
        L.qo_rms_norm_one.argtypes = [u16p, u16p, u16p, SZ, SZ, C.c_float]
        L.qo_head_rms_norm.argtypes = [u16p, SZ, u16p, SZ, SZ, SZ, C.c_float]
        L.qo_qk_rope.argtypes = [u16p, SZ, f32p, f32p, SZ, SZ, SZ]
        L.qo_gate.argtypes = [u16p, u16p, u16p, u16p, u32p, SZ, SZ,
                              C.c_uint32, C.c_uint32]
        L.qo_gelu_tanh.argtypes = [u16p, u16p, SZ]
        L.qo_silu.argtypes = [u16p, u16p, SZ]
        L.qo_swiglu.argtypes = [u16p, u16p, SZ, SZ]
        L.qo_attention.argtypes = [u16p, SZ, u16p, SZ, u16p, SZ, u16p, SZ,
                                   u32p, SZ, SZ, SZ, SZ, C.c_float]
        L.qo_attention_ex.argtypes = L.qo_attention.argtypes + [SZ]
        L.qo_set_attention_p_mode.argtypes = [C.c_int]
        L.qo_t2i_limits.argtypes = [u32p, C.c_uint32, C.c_uint32, C.c_int]
        L.qo_modulation_reorder.argtypes = [u16p, u16p, SZ, SZ, C.c_int]
        L.qo_model_init_random.restype = C.c_int
        L.qo_model_init_random.argtypes = [C.POINTER(QoModel),
                                           C.POINTER(QoConfig), C.c_uint64,
                                           C.c_uint32]
        L.qo_model_free.argtypes = [C.POINTER(QoModel)]
        L.qo_embed.argtypes = [C.POINTER(QoModel), u16p, C.c_uint32, u16p,
                               C.c_uint32, u16p]
        L.qo_conditioning.argtypes = [C.POINTER(QoModel), f32p, C.c_uint32,
                                      u16p, u16p, u16p]
        L.qo_block.argtypes = [C.POINTER(QoModel), C.c_int, u16p, u16p, f32p,
                               f32p, u32p, C.c_uint32, C.c_uint32,
                               C.c_void_p, C.c_void_p]
        L.qo_block_rows.argtypes = [C.POINTER(QoModel), C.c_int, u16p, u16p, f32p, f32p,
                                    u32p, C.c_uint32, C.c_uint32, u32p, C.c_uint32, u16p]
        L.qo_final.argtypes = [C.POINTER(QoModel), u16p, u16p, u32p,
                               C.c_uint32, u16p]
        L.qo_forward.restype = C.c_int
        L.qo_forward.argtypes = [C.POINTER(QoModel), C.c_void_p, C.c_uint32,
                                 u16p, C.c_uint32, C.c_float, f32p, f32p,
                                 C.c_uint32, u16p]
        L.qo_num_threads.restype = C.c_int
        L.qo_forward_ti2i.restype = C.c_int
        L.qo_forward_ti2i.argtypes = [C.POINTER(QoModel), C.c_void_p, C.c_uint32, C.c_void_p,
                                      C.c_uint32, C.c_void_p, C.c_uint32, C.c_float, f32p,
                                      f32p, C.c_uint32, u16p]
        L.qo_prefix_limits.restype = None
        L.qo_prefix_limits.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p]
        _LIB = L
    return _LIB


# ---- numpy helpers ---------------------------------------------------------

def bf16_to_f32(a):
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a):
    """RNE, matching h3_shaders.metal:16-20 (finite inputs)."""
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    b = b + np.uint32(0x7FFF) + ((b >> 16) & np.uint32(1))
    return (b >> 16).astype(np.uint16)


def fill_normal_bf16(n, seed, stream, std=1.0, offset=0.0):
    out = np.empty(n, np.uint16)
    lib().qo_fill_normal_bf16(out, n, seed, stream, std, offset)
    return out


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def linear(x, w, bias, rows, k, n):
    y = np.empty((rows, n), np.uint16)
    lib().qo_linear(y, n, np.ascontiguousarray(x), k, np.ascontiguousarray(w),
                    ptr(bias), rows, k, n)
    return y


def linear_i8(x, q, scales, bias, rows, k, n):
    y = np.empty((rows, n), np.uint16)
    lib().qo_linear_i8(y, n, np.ascontiguousarray(x), k,
                       np.ascontiguousarray(q), np.ascontiguousarray(scales),
                       ptr(bias), rows, k, n)
    return y


def quantize_int8_rows(w, rows, cols):
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    lib().qo_quantize_int8_rows(q, s, np.ascontiguousarray(w), rows, cols)
    return q, s


def attention(q, k, v, limits, q_rows, kv_rows, heads, head_dim=128,
              scale=None, ldq=None, ldk=None, ldv=None, prescale_rows=0):
    """prescale_rows: leading rows under the t2i text-row rule (q scaled and
    re-rounded to bf16 before QK, h3_shaders.metal:4397-4401)"""
    hd = heads * head_dim
    scale = 1.0 / np.sqrt(head_dim) if scale is None else scale
    out = np.zeros((q_rows, hd), np.uint16)
    lib().qo_attention_ex(out, hd, q, ldq or hd, k, ldk or hd, v, ldv or hd,
                          np.ascontiguousarray(limits, dtype=np.uint32), q_rows,
                          kv_rows, heads, head_dim, float(scale), prescale_rows)
    return out


def set_attention_p_mode(mode):
    """1: the oracle rounds each softmax probability to bf16 (as the flash
    kernel's P operand), 0: fp32 probabilities"""
    lib().qo_set_attention_p_mode(int(mode))


def t2i_limits(rows, text_rows, text_causal):
    lim = np.empty(rows, np.uint32)
    lib().qo_t2i_limits(lim, rows, text_rows, int(text_causal))
    return lim


def rope_tables(text_rows, gh, gw):
    rows = text_rows + gh * gw
    c = np.empty((rows, 64), np.float32)
    s = np.empty((rows, 64), np.float32)
    lib().qo_rope_tables(text_rows, gh, gw, c, s)
    return c, s


def rope_tables_blocks(block_h, block_w, text_before):
    """ti2i multi-block tables: [rows, 64] cos and sin"""
    bh, bw, tb = (np.ascontiguousarray(x, np.uint32) for x in (block_h, block_w, text_before))
    rows = int(tb.sum() + (bh.astype(np.int64) * bw).sum())
    c = np.empty((rows, 64), np.float32)
    s = np.empty((rows, 64), np.float32)
    assert lib().qo_rope_tables_blocks(bh, bw, tb, len(bh), c, s) == rows
    return c, s


def timestep_features(sigmas):
    sig = np.ascontiguousarray(sigmas, dtype=np.float32)
    out = np.empty((len(sig), 256), np.float32)
    lib().qo_timestep_features(sig, len(sig), out)
    return out


class Segment(C.Structure):
    """qo_segment / qw_dit_segment: rows, is_image, src_offset"""
    _fields_ = [("rows", C.c_uint32), ("is_image", C.c_int), ("src_offset", C.c_uint32)]


def segment_array(segs):
    return (Segment * len(segs))(*[Segment(r, int(i), o) for r, i, o in segs])


def prefix_limits(segs):
    rows = sum(r for r, _, _ in segs)
    out = np.empty(rows, np.uint32)
    lib().qo_prefix_limits(segment_array(segs), len(segs), out.ctypes.data)
    return out


class Model:
    """Seeded random DiT (same weight streams as the GPU library)."""

    def __init__(self, cfg: dict, seed: int, layers: int):
        self.cfg = QoConfig(**cfg)
        self.m = QoModel()
        lib().qo_model_init_random(C.byref(self.m), C.byref(self.cfg), seed,
                                   layers)

    def close(self):
        if self.m is not None:
            lib().qo_model_free(C.byref(self.m))
            self.m = None

    def __del__(self):
        self.close()

    def forward(self, text_in, text_rows, latents, image_rows, sigma,
                rope_cos, rope_sin, layers):
        rows = text_rows + image_rows
        out = np.empty((rows, self.cfg.z_dim), np.uint16)
        ok = lib().qo_forward(C.byref(self.m),
                              ptr(text_in) if text_rows else None, text_rows,
                              np.ascontiguousarray(latents), image_rows,
                              float(sigma), np.ascontiguousarray(rope_cos),
                              np.ascontiguousarray(rope_sin), layers, out)
        if not ok:
            raise RuntimeError("qo_forward failed")
        return out

    def forward_ti2i(self, text_in, text_total, latents, image_total, segs, sigma,
                     rope_cos, rope_sin, layers):
        """segs: [(rows, is_image, src_offset), ...]; output [rows, z_dim]."""
        seg = segment_array(segs)
        rows = sum(r for r, _, _ in segs)
        out = np.empty((rows, self.cfg.z_dim), np.uint16)
        ok = lib().qo_forward_ti2i(C.byref(self.m), ptr(text_in) if text_total else None,
                                   text_total, ptr(np.ascontiguousarray(latents)), image_total,
                                   seg, len(segs), float(sigma), np.ascontiguousarray(rope_cos),
                                   np.ascontiguousarray(rope_sin), layers, out)
        if not ok:
            raise RuntimeError("qo_forward_ti2i failed")
        return out

    def block_rows(self, layer, hidden, modulation, rope_cos, rope_sin, row_map, rows,
                   text_rows, sample):
        """qo_block's output for the listed rows only: [len(sample), H]"""
        sample = np.ascontiguousarray(sample, np.uint32)
        out = np.empty((len(sample), self.cfg.hidden), np.uint16)
        lib().qo_block_rows(C.byref(self.m), layer, np.ascontiguousarray(hidden),
                            np.ascontiguousarray(modulation), np.ascontiguousarray(rope_cos),
                            np.ascontiguousarray(rope_sin), np.ascontiguousarray(row_map),
                            rows, text_rows, sample, len(sample), out)
        return out

    def block(self, layer, hidden, modulation, rope_cos, rope_sin, row_map,
              rows, text_rows, limits=None, want_attn=False):
        dbg = np.empty((rows, self.cfg.hidden), np.uint16) if want_attn else None
        lib().qo_block(C.byref(self.m), layer, hidden, modulation, rope_cos,
                       rope_sin, row_map, rows, text_rows, ptr(limits),
                       ptr(dbg))
        return dbg

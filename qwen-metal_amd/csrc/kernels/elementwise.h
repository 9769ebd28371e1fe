/* Bandwidth-bound kernels of the DiT block: LayerNorm-modulation, RMSNorm,
 * fused per-head QK RMSNorm + interleaved RoPE, residual gate, activations,
 * casts, the conditioning reorder, the seeded generator and the int8
 * weight quantizer. 128-bit loads where rows allow, wave-shuffle
 * reductions, fp32 math with one bf16 rounding per reference kernel output
 * (fp contraction off so the rounding points are the written ones). */
#pragma once
#include "common.h"

/* ---- LayerNorm + (1 + scale) [+ shift] --------------------------------- */
/* h3_shaders.metal:4767-4815. One wave per row (width <= 4096), four rows
 * per block: lane l owns the 16-byte chunks l, l + 64, ... of the row,
 * held in registers for both passes, and both reductions are wave
 * shuffles (no LDS, no barrier). */
#define LN_CH 8 /* chunks of 8 per lane: width <= 64 * 8 * 8 = 4096 */
QW_KERNEL void __launch_bounds__(256) qw_layer_norm_mod_bf16(qw_ln_mod_args a) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return; /* whole waves */
    const u16 *in = a.in + (size_t)row * a.width;
    float x[LN_CH][8];
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < LN_CH; c++) {
        const uint32_t c8 = (c * 64 + lane) * 8;
        u32x4 raw = {0, 0, 0, 0};
        if (c8 < a.width) raw = *(const u32x4 *)(in + c8);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[c][2 * i] = lo_bf(raw[i]);
            x[c][2 * i + 1] = hi_bf(raw[i]);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) s += x[c][i];
    }
    const float mean = wave_sum(s) / (float)a.width;
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < LN_CH; c++) {
        if ((c * 64 + lane) * 8 >= a.width) continue;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float d = x[c][i] - mean;
            q = fmaf(d, d, q);
        }
    }
    const float var = wave_sum(q) / (float)a.width;
    const float inv = 1.0f / sqrtf(var + a.eps);
    const u16 *mod = a.modulation + (size_t)a.row_map[row] * a.slots * a.width;
#pragma unroll
    for (int c = 0; c < LN_CH; c++) {
        const uint32_t c8 = (c * 64 + lane) * 8;
        if (c8 >= a.width) continue;
        const u32x4 sc = *(const u32x4 *)(mod + (size_t)a.scale_slot * a.width + c8);
        u32x4 sh = {0, 0, 0, 0};
        if (a.shift_slot >= 0) sh = *(const u32x4 *)(mod + (size_t)a.shift_slot * a.width + c8);
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v0 = ((x[c][2 * i] - mean) * inv) * (1.0f + lo_bf(sc[i]));
            float v1 = ((x[c][2 * i + 1] - mean) * inv) * (1.0f + hi_bf(sc[i]));
            if (a.shift_slot >= 0) {
                v0 += lo_bf(sh[i]);
                v1 += hi_bf(sh[i]);
            }
            o[i] = pack_bf(v0, v1);
        }
        *(u32x4 *)(a.out + (size_t)row * a.width + c8) = o;
    }
}

/* The same for rows wider than 4096: one block per row, width / 8 threads
 * rounded up to whole waves, each owning one 16-byte chunk (idle tail
 * lanes contribute zeros to the reductions). */
QW_KERNEL void __launch_bounds__(1024)
qw_layer_norm_mod_wide_bf16(qw_ln_mod_args a) {
#pragma clang fp contract(off)
    __shared__ float red[16];
    const uint32_t row = blockIdx.x;
    const uint32_t c8 = threadIdx.x * 8;
    const bool active = c8 < a.width; /* blockDim is rounded up to whole waves */
    u32x4 raw = {0, 0, 0, 0};
    if (active) raw = *(const u32x4 *)(a.in + (size_t)row * a.width + c8);
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        x[2 * i] = lo_bf(raw[i]);
        x[2 * i + 1] = hi_bf(raw[i]);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) s += x[i];
    const float mean = block_sum(s, red) / (float)a.width;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float d = x[i] - mean;
        q = fmaf(d, d, q);
    }
    const float var = block_sum(active ? q : 0.0f, red) / (float)a.width;
    const float inv = 1.0f / sqrtf(var + a.eps);
    if (!active) return;
    const u16 *mod = a.modulation + (size_t)a.row_map[row] * a.slots * a.width;
    const u32x4 sc = *(const u32x4 *)(mod + (size_t)a.scale_slot * a.width + c8);
    u32x4 sh = {0, 0, 0, 0};
    if (a.shift_slot >= 0) sh = *(const u32x4 *)(mod + (size_t)a.shift_slot * a.width + c8);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float v0 = ((x[2 * i] - mean) * inv) * (1.0f + lo_bf(sc[i]));
        float v1 = ((x[2 * i + 1] - mean) * inv) * (1.0f + hi_bf(sc[i]));
        if (a.shift_slot >= 0) {
            v0 += lo_bf(sh[i]);
            v1 += hi_bf(sh[i]);
        }
        o[i] = pack_bf(v0, v1);
    }
    *(u32x4 *)(a.out + (size_t)row * a.width + c8) = o;
}

/* ---- RMSNorm with (w + 1) ----------------------------------------------- */
/* h3_shaders.metal:4817-4850; same block shape as the LayerNorm. */
QW_KERNEL void __launch_bounds__(1024) qw_rms_norm_one_bf16(qw_rms_one_args a) {
#pragma clang fp contract(off)
    __shared__ float red[16];
    const uint32_t row = blockIdx.x;
    const uint32_t c8 = threadIdx.x * 8;
    const bool active = c8 < a.width;
    u32x4 raw = {0, 0, 0, 0};
    if (active) raw = *(const u32x4 *)(a.in + (size_t)row * a.width + c8);
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        x[2 * i] = lo_bf(raw[i]);
        x[2 * i + 1] = hi_bf(raw[i]);
    }
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) q = fmaf(x[i], x[i], q);
    const float inv = 1.0f / sqrtf(block_sum(q, red) / (float)a.width + a.eps);
    if (!active) return;
    const u32x4 w = *(const u32x4 *)(a.weight + c8);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++)
        o[i] = pack_bf(x[2 * i] * inv * (lo_bf(w[i]) + 1.0f),
                       x[2 * i + 1] * inv * (hi_bf(w[i]) + 1.0f));
    *(u32x4 *)(a.out + (size_t)row * a.width + c8) = o;
}

/* ---- per-head RMSNorm (single rounding) then interleaved RoPE ----------- */
/* h3_shaders.metal:4309-4329 followed by 4864-4896, fused. 16 lanes per
 * (row, head, q|k) item, 16 items per 256-thread block; lane l owns the 8
 * elements 8l..8l+7 (one 16-byte load), i.e. the RoPE pairs 4l..4l+3, and
 * the sum of squares is reduced across the 16 lanes of its item. The norm
 * output is rounded to bf16 before the rotation, as the two reference
 * kernels do. In place on a strided [rows, ld] buffer (the fused q|k|v
 * projection output). */
QW_KERNEL void __launch_bounds__(256) qw_qk_norm_rope_bf16(qw_qk_norm_rope_args a) {
#pragma clang fp contract(off)
    const uint32_t l = threadIdx.x & 15;
    const uint64_t item = (uint64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const uint64_t per_row = 2ull * a.heads;
    const bool active = item < (uint64_t)a.rows * per_row;
    const uint64_t it = active ? item : 0; /* inactive lanes still join the shuffles */
    const uint32_t row = (uint32_t)(it / per_row);
    const uint32_t rem = (uint32_t)(it % per_row);
    const uint32_t is_k = rem >= a.heads;
    const uint32_t head = is_k ? rem - a.heads : rem;
    u16 *p = a.qk + (size_t)row * a.ld + (is_k ? a.k_offset : 0) + head * QW_HEAD_DIM + 8 * l;
    const u32x4 w = *(const u32x4 *)p;
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        x[2 * i] = lo_bf(w[i]);
        x[2 * i + 1] = hi_bf(w[i]);
    }
    if (a.do_norm) {
        const u32x4 wn = *(const u32x4 *)((is_k ? a.norm_k : a.norm_q) + 8 * l);
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) ss = fmaf(x[i], x[i], ss);
        ss = row16_sum(ss);
        const float inv = head_rms_inv(ss, a.eps);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[2 * i] = bf2f(f2bf(x[2 * i] * inv * lo_bf(wn[i])));
            x[2 * i + 1] = bf2f(f2bf(x[2 * i + 1] * inv * hi_bf(wn[i])));
        }
    }
    if (a.do_rope) {
        const size_t t = (size_t)(row % a.rope_rows) * 64 + 4 * l;
        const floatx4 c = *(const floatx4 *)(a.rope_cos + t);
        const floatx4 sn = *(const floatx4 *)(a.rope_sin + t);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float y0 = x[2 * i] * c[i] - x[2 * i + 1] * sn[i];
            const float y1 = x[2 * i] * sn[i] + x[2 * i + 1] * c[i];
            x[2 * i] = y0;
            x[2 * i + 1] = y1;
        }
    }
    if (active)
        *(u32x4 *)p = u32x4{pack_bf(x[0], x[1]), pack_bf(x[2], x[3]), pack_bf(x[4], x[5]),
                            pack_bf(x[6], x[7])};
}

/* ---- residual gate: out = res + branch * gate[row_map[r]] ---------------- */
/* h3_shaders.metal:3583-3599, 8 elements per thread. */
QW_KERNEL void __launch_bounds__(256) qw_gate_bf16(qw_gate_args a) {
#pragma clang fp contract(off)
    const uint64_t i8 = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i8 >= (uint64_t)a.rows * a.width) return;
    const uint32_t row = (uint32_t)(i8 / a.width), col = (uint32_t)(i8 % a.width);
    const u32x4 r = *(const u32x4 *)(a.residual + i8);
    const u32x4 b = *(const u32x4 *)(a.branch + i8);
    const u32x4 g = *(const u32x4 *)(a.modulation +
                                     ((size_t)a.row_map[row] * a.slots + a.gate_slot) * a.width + col);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++)
        o[i] = pack_bf(lo_bf(r[i]) + lo_bf(b[i]) * lo_bf(g[i]),
                       hi_bf(r[i]) + hi_bf(b[i]) * hi_bf(g[i]));
    *(u32x4 *)(a.out + i8) = o;
}

/* ---- activations --------------------------------------------------------- */
/* h3_shaders.metal:3385-3408 (gelu), 3284-3291 (silu), qwen tanh pre-pass. */
QW_KERNEL void __launch_bounds__(256) qw_act_bf16(qw_act_args a) {
#pragma clang fp contract(off)
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.count) return;
    float v = bf2f(a.in[i]);
    float y = a.act == QW_ACT_GELU_TANH ? gelu_tanh_f(v)
              : a.act == QW_ACT_SILU    ? silu_f(v)
                                        : tanhf(v);
    a.out[i] = f2bf(y);
}

/* h3_shaders.metal:5078-5095: silu(gate) rounded to bf16, times up. */
QW_KERNEL void __launch_bounds__(256) qw_swiglu_bf16(qw_swiglu_args a) {
#pragma clang fp contract(off)
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)a.rows * a.width) return;
    const uint64_t row = i / a.width, col = i % a.width;
    float g = bf2f(a.fc1[row * 2 * a.width + col]);
    float u = bf2f(a.fc1[row * 2 * a.width + a.width + col]);
    a.out[i] = f2bf(bf2f(f2bf(silu_f(g))) * u);
}

/* h3_shaders.metal:188-193 */
QW_KERNEL void __launch_bounds__(256) qw_cast_f32_bf16(qw_cast_args a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < a.count) a.out[i] = f2bf(a.in[i]);
}

/* ---- denoise loop: CFG combine + Euler step, on the resident fp32 latents */
QW_KERNEL void __launch_bounds__(256) qw_cfg_euler_f32(qw_euler_args a) {
#pragma clang fp contract(off)
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.count) return;
    float v = bf2f(a.pos[i]);
    if (a.neg) {
        const float n = bf2f(a.neg[i]);
        v = n + a.cfg * (v - n);
    }
    a.x[i] += a.dt * v;
}

/* ---- conditioning reorder (device replacement of a host round trip) ------ */
/* qwen_dit.m:1159-1186: scales copied, gates tanh'd in fp32 and stored by
 * truncation (qw_f32_to_bits). Shift variant keeps the shifts in slots 4, 5. */
QW_KERNEL void __launch_bounds__(256) qw_modulation_reorder_bf16(qw_reorder_args a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)a.mod_rows * a.hidden) return;
    const uint32_t r = (uint32_t)(i / a.hidden), c = (uint32_t)(i % a.hidden);
    const uint32_t H = a.hidden, S = a.shift_variant ? 6 : 4;
    const u16 *src = a.raw + (size_t)r * S * H;
    u16 *dst = a.slots_out + (size_t)r * S * H;
    const uint32_t sc1 = a.shift_variant ? 1 : 0, g1 = a.shift_variant ? 2 : 1;
    const uint32_t sc2 = a.shift_variant ? 4 : 2, g2 = a.shift_variant ? 5 : 3;
    dst[c] = src[sc1 * H + c];
    dst[H + c] = src[sc2 * H + c];
    dst[2 * H + c] = f2bf_trunc(tanhf(bf2f(src[g1 * H + c])));
    dst[3 * H + c] = f2bf_trunc(tanhf(bf2f(src[g2 * H + c])));
    if (a.shift_variant) {
        dst[4 * H + c] = src[c];
        dst[5 * H + c] = src[3 * H + c];
    }
}

/* ---- seeded synthetic N(0, 1)-like values -------------------------------- */
/* Counter-based (splitmix64 finaliser), integer sum of twelve 16-bit
 * uniforms; bit-identical to the host generator by construction. */
__device__ __forceinline__ uint64_t qw_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

QW_KERNEL void __launch_bounds__(256) qw_fill_normal_bf16(qw_fill_args a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.count) return;
    const uint64_t key = qw_mix64(a.seed ^ qw_mix64(a.stream + 0x9e3779b97f4a7c15ull));
    int32_t sum = 0;
#pragma unroll
    for (uint64_t j = 0; j < 3; j++) {
        uint64_t h = qw_mix64(key + (i * 3u + j) * 0x9e3779b97f4a7c15ull);
        sum += (int32_t)(h & 0xffffu) + (int32_t)((h >> 16) & 0xffffu) +
               (int32_t)((h >> 32) & 0xffffu) + (int32_t)(h >> 48);
    }
    const float z = (float)(2 * sum - 12 * 65535) * (1.0f / 131072.0f);
    a.out[i] = f2bf(__builtin_fmaf(a.std, z, a.offset));
}

/* ---- int8 weight quantizer ------------------------------------------------ */
/* h3_shaders.metal:1320-1390 with clip 1.0: per output row, m = max|w|,
 * scale = m / 127, q = clamp(rint(w * (127 / m)), -127, 127). One block of
 * 256 threads per row. */
QW_KERNEL void __launch_bounds__(256) qw_quantize_int8_rows(qw_quant_args a) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    const uint32_t row = blockIdx.x;
    const u16 *w = a.w + (size_t)row * a.cols;
    float mx = 0.0f;
    for (uint32_t c = threadIdx.x; c < a.cols; c += 256) mx = fmaxf(mx, fabsf(bf2f(w[c])));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float scale = mx > 0.0f ? mx / 127.0f : 1.0f / 127.0f;
    const float inverse = mx > 0.0f ? 127.0f / mx : 127.0f;
    if (threadIdx.x == 0) a.scales[row] = scale;
    for (uint32_t c = threadIdx.x; c < a.cols; c += 256) {
        int v = (int)rintf(bf2f(w[c]) * inverse);
        v = v > 127 ? 127 : (v < -127 ? -127 : v);
        a.q[(size_t)row * a.cols + c] = (int8_t)v;
    }
}

/* Dequantised weight q * scale in fp32 (the bit-exactness probe). */
QW_KERNEL void __launch_bounds__(256) qw_dequant_int8_f32(qw_dequant_args a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)a.rows * a.cols) return;
    a.out[i] = (float)a.q[i] * a.scales[i / a.cols];
}

/* ---- strided 2D byte copy (row slices, K/V export) ------------------------ */
QW_KERNEL void __launch_bounds__(256) qw_copy2d(qw_copy2d_args a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t words = a.row_bytes / 4;
    if (i >= a.rows * words) return;
    const uint64_t r = i / words, c = i % words;
    ((uint32_t *)((char *)a.dst + r * a.dst_stride))[c] =
        ((const uint32_t *)((const char *)a.src + r * a.src_stride))[c];
}

/* n u32 words set to zero (counters that must start at zero; a kernel, not
 * hipMemsetAsync, so the clear can sit inside a captured graph) */
QW_KERNEL void __launch_bounds__(256) qw_zero_u32(qw_zero_args a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < a.count) a.p[i] = 0u;
}

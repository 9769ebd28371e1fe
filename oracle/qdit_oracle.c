/* qdit_oracle.c — CPU restatement of the qwen-metal DiT forward.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library, never part of
 * it. Compiled with -ffp-contract=off so every multiply-add rounds exactly
 * where the source says (explicit fmaf() where the reference fuses).
 * Reference citations are file:line into wangyancz/qwen-metal.
 */
#include "qdit_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------- */
/* bf16                                                                   */

uint16_t qo_f32_to_bf16(float value) {
    /* h3_shaders.metal:16-20: add 0x7fff + lsb, keep the high half. */
    uint32_t bits;
    memcpy(&bits, &value, 4);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

uint16_t qo_f32_to_bf16_trunc(float value) {
    /* qwen_dit.m:229-233 (qw_f32_to_bits): plain truncation. */
    uint32_t bits;
    memcpy(&bits, &value, 4);
    return (uint16_t)(bits >> 16);
}

float qo_bf16_to_f32(uint16_t bits) {
    uint32_t wide = (uint32_t)bits << 16;
    float value;
    memcpy(&value, &wide, 4);
    return value;
}

static inline float bf(uint16_t b) { return qo_bf16_to_f32(b); }
static inline uint16_t rne(float f) { return qo_f32_to_bf16(f); }
static inline float round_bf(float f) { return bf(rne(f)); }

void qo_bf16_to_f32_array(const uint16_t *in, float *out, size_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++) out[i] = bf(in[i]);
}

void qo_f32_to_bf16_array(const float *in, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++) out[i] = rne(in[i]);
}

/* Attention probability rounding ahead of P.V: 0 = fp32 P (exact
 * softmax), 1 = P rounded to bf16 after the row sum is taken (the
 * reference's flash kernel, h3_shaders.metal:2882-3040, multiplies bf16 P
 * by V). */
static int g_attn_p_mode = 0;
void qo_set_attention_p_mode(int mode) { g_attn_p_mode = mode; }

int qo_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------------- */
/* host math                                                              */

uint32_t qo_rng_u32(qo_rng *rng) {
    /* PCG32 XSH-RR step, qwen_host.c:440-446. */
    uint64_t old = rng->state;
    rng->state = old * UINT64_C(6364136223846793005) + rng->increment;
    uint32_t xorshifted = (uint32_t)(((old >> 18u) ^ old) >> 27u);
    uint32_t rot = (uint32_t)(old >> 59u);
    return (xorshifted >> rot) | (xorshifted << ((32u - rot) & 31u));
}

void qo_rng_seed(qo_rng *rng, uint64_t seed) {
    /* qwen_host.c:452-458: stream from the seed, golden-ratio state kick. */
    memset(rng, 0, sizeof(*rng));
    rng->increment = (seed << 1u) | 1u;
    (void)qo_rng_u32(rng);
    rng->state += seed ^ UINT64_C(0x9e3779b97f4a7c15);
    (void)qo_rng_u32(rng);
}

float qo_rng_normal(qo_rng *rng) {
    /* Box-Muller pair in double, qwen_host.c:460-471: cos first, sin kept. */
    if (rng->has_spare) {
        rng->has_spare = 0;
        return rng->spare;
    }
    double u1 = ((double)qo_rng_u32(rng) + 1.0) / 4294967297.0;
    double u2 = ((double)qo_rng_u32(rng) + 0.5) / 4294967296.0;
    double r = sqrt(-2.0 * log(u1));
    double a = 6.283185307179586476925286766559 * u2;
    rng->spare = (float)(r * sin(a));
    rng->has_spare = 1;
    return (float)(r * cos(a));
}

void qo_rng_fill_normal(qo_rng *rng, float *v, size_t n) {
    for (size_t i = 0; i < n; i++) v[i] = qo_rng_normal(rng);
}

double qo_calculate_shift(int image_seq_len) {
    /* qwen_host.c:18-26: line through (256, 0.5) and (8192, 0.9). */
    double slope = (0.9 - 0.5) / (8192.0 - 256.0);
    double intercept = 0.5 - slope * 256.0;
    return (double)image_seq_len * slope + intercept;
}

int qo_schedule_exp_mu(int steps, double exp_mu, double terminal,
                       float *sigma) {
    /* qwen_pipeline.m:130-205 (dynamic shifting branch): every
     * intermediate is a float32 value; exp_mu enters as a double. */
    if (steps < 1 || !sigma) return 0; /* no upper bound, as the reference */
    for (int i = 0; i < steps; i++) {
        double raw = steps == 1 ? 1.0
                                : 1.0 + (double)i * ((1.0 / steps) - 1.0) /
                                            (double)(steps - 1);
        float t = (float)raw;
        float inv = (float)(1.0 / t);
        float base = (float)(inv - 1.0f);
        sigma[i] = (float)(exp_mu / (exp_mu + (double)base));
    }
    if (terminal > 0.0 && terminal < 1.0) {
        float tail = (float)(1.0 - (double)sigma[steps - 1]);
        float scale = (float)((double)tail / (1.0 - terminal));
        if (scale != 0.0f)
            for (int i = 0; i < steps; i++) {
                float om = (float)(1.0 - (double)sigma[i]);
                sigma[i] = (float)(1.0 - (double)om / (double)scale);
            }
    }
    sigma[steps] = 0.0f;
    return 1;
}

int qo_schedule_build(int steps, int image_seq_len, float *sigma) {
    /* qwen_host.c:335-370: float32 numpy semantics of set_timesteps. The
     * linspace is formed in double, each element cast to float32. */
    if (steps < 1 || steps > 1000 || image_seq_len < 1 || !sigma) return 0;
    float exp_mu = (float)exp(qo_calculate_shift(image_seq_len));
    double stop = 1.0 / (double)steps;
    double delta = steps > 1 ? (stop - 1.0) / (double)(steps - 1) : 0.0;
    for (int i = 0; i < steps; i++) {
        double v = 1.0 + (double)i * delta;
        if (i == steps - 1) v = stop;
        float base = (float)v;
        float inv = 1.0f / base;
        float denom = exp_mu + (inv - 1.0f);
        sigma[i] = exp_mu / denom;
    }
    float om_last = 1.0f - sigma[steps - 1];
    float scale = om_last / (1.0f - 0.02f);
    for (int i = 0; i < steps; i++) {
        float om = 1.0f - sigma[i];
        sigma[i] = 1.0f - om / scale;
    }
    sigma[steps] = 0.0f;
    return 1;
}

void qo_euler_step(float *sample, const float *velocity, size_t n,
                   float sigma, float sigma_next) {
    /* qwen_host.c:372-378. */
    float dt = sigma - sigma_next;
    for (size_t i = 0; i < n; i++) sample[i] += dt * velocity[i];
}

void qo_rope_table_entry(int axis_dim, int table_row, int pair,
                         float *cos_out, float *sin_out) {
    /* qwen_host.c:388-430: rows 0..8191 -> coordinate = row, rows
     * 8192..9215 -> -1024..-1; float32 frequency and angle. */
    int coordinate = table_row < 8192 ? table_row : (table_row - 8192) - 1024;
    float freq = (float)pow(10000.0, -2.0 * (double)pair / (double)axis_dim);
    float angle = (float)coordinate * freq;
    *cos_out = cosf(angle);
    *sin_out = sinf(angle);
}

void qo_rope_tables(uint32_t text_rows, uint32_t gh, uint32_t gw,
                    float *cos_out, float *sin_out) {
    /* qwen_pipeline.m:212-273: text row t at (t, t, t); image row (h, w) at
     * (text_rows, h - ceil(gh/2), w - ceil(gw/2)); angle in double. */
    static const int dims[3] = {16, 56, 56};
    uint32_t rows = text_rows + gh * gw;
    long half_h = (long)(gh - gh / 2), half_w = (long)(gw - gw / 2);
    for (uint32_t t = 0; t < rows; t++) {
        double pos[3];
        if (t < text_rows) {
            pos[0] = pos[1] = pos[2] = (double)t;
        } else {
            uint32_t idx = t - text_rows;
            pos[0] = (double)text_rows;
            pos[1] = (double)((long)(idx / gw) - half_h);
            pos[2] = (double)((long)(idx % gw) - half_w);
        }
        size_t col = 0;
        for (int a = 0; a < 3; a++)
            for (int p = 0; p < dims[a] / 2; p++, col++) {
                double f = pow(10000.0, -2.0 * (double)p / (double)dims[a]);
                double ang = pos[a] * f;
                cos_out[(size_t)t * 64 + col] = (float)cos(ang);
                sin_out[(size_t)t * 64 + col] = (float)sin(ang);
            }
    }
}

size_t qo_rope_tables_blocks(const uint32_t *block_h, const uint32_t *block_w,
                             const uint32_t *text_before, uint32_t n_blocks,
                             float *cos_out, float *sin_out) {
    /* qwen_pipeline.m:611-680 (ti2i): text rows at (p, p, p) with p
     * advancing by one per row; an image block of gh x gw at (frame, h -
     * ceil(gh/2), w - ceil(gw/2)) with the frame frozen at the position the
     * block starts at, after which the position advances by max(gh, gw).
     * Angles in double, as qo_rope_tables. */
    static const int dims[3] = {16, 56, 56};
    double position = 0.0;
    size_t r = 0;
    for (uint32_t b = 0; b < n_blocks; b++) {
        uint32_t rows_b = text_before[b] + block_h[b] * block_w[b];
        long half_h = (long)(block_h[b] - block_h[b] / 2);
        long half_w = (long)(block_w[b] - block_w[b] / 2);
        double frame = position + (double)text_before[b];
        for (uint32_t i = 0; i < rows_b; i++, r++) {
            double pos[3];
            if (i < text_before[b]) {
                pos[0] = pos[1] = pos[2] = position + (double)i;
            } else {
                uint32_t idx = i - text_before[b];
                pos[0] = frame;
                pos[1] = (double)((long)(idx / block_w[b]) - half_h);
                pos[2] = (double)((long)(idx % block_w[b]) - half_w);
            }
            size_t col = 0;
            for (int a = 0; a < 3; a++)
                for (int p = 0; p < dims[a] / 2; p++, col++) {
                    double f = pow(10000.0, -2.0 * (double)p / (double)dims[a]);
                    double ang = pos[a] * f;
                    cos_out[r * 64 + col] = (float)cos(ang);
                    sin_out[r * 64 + col] = (float)sin(ang);
                }
        }
        position = frame + (double)(block_h[b] > block_w[b] ? block_h[b] : block_w[b]);
    }
    return r;
}

void qo_timestep_features(const float *sigmas, size_t count,
                          float *features) {
    /* qwen_dit.m:1085-1096: [cos(1000 s f_i) | sin(1000 s f_i)],
     * f_i = 10000^(-i/128), double precision, stored float. */
    for (size_t r = 0; r < count; r++) {
        double raw = (double)sigmas[r] * 1000.0;
        for (int i = 0; i < 128; i++) {
            double arg = raw * pow(10000.0, -(double)i / 128.0);
            features[r * 256 + i] = (float)cos(arg);
            features[r * 256 + 128 + i] = (float)sin(arg);
        }
    }
}

/* ---------------------------------------------------------------------- */
/* synthetic generator (shared bit-for-bit with the GPU fill kernel)       */

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * UINT64_C(0xbf58476d1ce4e5b9);
    z = (z ^ (z >> 27)) * UINT64_C(0x94d049bb133111eb);
    return z ^ (z >> 31);
}

float qo_synth_normal(uint64_t seed, uint64_t stream, uint64_t index) {
    uint64_t key = mix64(seed ^ mix64(stream + UINT64_C(0x9e3779b97f4a7c15)));
    int32_t sum = 0;
    for (uint64_t j = 0; j < 3; j++) {
        uint64_t h = mix64(key + (index * 3u + j) * UINT64_C(0x9e3779b97f4a7c15));
        sum += (int32_t)(h & 0xffffu) + (int32_t)((h >> 16) & 0xffffu) +
               (int32_t)((h >> 32) & 0xffffu) + (int32_t)(h >> 48);
    }
    int32_t centered = 2 * sum - 12 * 65535;
    return (float)centered * (1.0f / 131072.0f);
}

void qo_fill_normal_bf16(uint16_t *out, size_t n, uint64_t seed,
                         uint64_t stream, float std, float offset) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++)
        out[i] = rne(fmaf(std, qo_synth_normal(seed, stream, i), offset));
}

/* ---------------------------------------------------------------------- */
/* GEMM (fp32, C = A B^T)                                                  */

typedef float v8f __attribute__((vector_size(32)));

static inline v8f ld8(const float *p) {
    v8f v;
    memcpy(&v, p, 32);
    return v;
}

static inline float hsum8(v8f v) {
    return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
}

/* c[i][j] (+)= sum_k a[i][k] b[j][k] over one K chunk. */
static void gemm_chunk(const float *a, size_t lda, const float *b, size_t ldb,
                       float *c, size_t ldc, size_t m, size_t n, size_t k,
                       int accumulate) {
    size_t k8 = k & ~(size_t)7;
    size_t i = 0;
    for (; i + 3 <= m; i += 3) {
        const float *a0 = a + i * lda, *a1 = a0 + lda, *a2 = a1 + lda;
        size_t j = 0;
        for (; j + 4 <= n; j += 4) {
            const float *b0 = b + j * ldb, *b1 = b0 + ldb, *b2 = b1 + ldb,
                        *b3 = b2 + ldb;
            v8f c00 = {0}, c01 = {0}, c02 = {0}, c03 = {0};
            v8f c10 = {0}, c11 = {0}, c12 = {0}, c13 = {0};
            v8f c20 = {0}, c21 = {0}, c22 = {0}, c23 = {0};
            for (size_t kk = 0; kk < k8; kk += 8) {
                v8f x0 = ld8(a0 + kk), x1 = ld8(a1 + kk), x2 = ld8(a2 + kk);
                /* fused multiply-adds: the contraction's fp32 summation
                 * order is free (any order is an fp32-accumulating linear);
                 * only the elementwise code keeps -ffp-contract=off */
#define QO_FMA(c, x, w) c = (v8f)_mm256_fmadd_ps((__m256)(x), (__m256)(w), (__m256)(c))
                v8f w = ld8(b0 + kk);
                QO_FMA(c00, x0, w); QO_FMA(c10, x1, w); QO_FMA(c20, x2, w);
                w = ld8(b1 + kk);
                QO_FMA(c01, x0, w); QO_FMA(c11, x1, w); QO_FMA(c21, x2, w);
                w = ld8(b2 + kk);
                QO_FMA(c02, x0, w); QO_FMA(c12, x1, w); QO_FMA(c22, x2, w);
                w = ld8(b3 + kk);
                QO_FMA(c03, x0, w); QO_FMA(c13, x1, w); QO_FMA(c23, x2, w);
#undef QO_FMA
            }
            float r[3][4] = {
                {hsum8(c00), hsum8(c01), hsum8(c02), hsum8(c03)},
                {hsum8(c10), hsum8(c11), hsum8(c12), hsum8(c13)},
                {hsum8(c20), hsum8(c21), hsum8(c22), hsum8(c23)}};
            for (size_t kk = k8; kk < k; kk++)
                for (int ii = 0; ii < 3; ii++)
                    for (int jj = 0; jj < 4; jj++)
                        r[ii][jj] += a[(i + ii) * lda + kk] *
                                     b[(j + jj) * ldb + kk];
            for (int ii = 0; ii < 3; ii++)
                for (int jj = 0; jj < 4; jj++) {
                    float *dst = c + (i + ii) * ldc + j + jj;
                    *dst = accumulate ? *dst + r[ii][jj] : r[ii][jj];
                }
        }
        for (; j < n; j++)
            for (int ii = 0; ii < 3; ii++) {
                const float *ar = a + (i + ii) * lda, *br = b + j * ldb;
                v8f acc = {0};
                for (size_t kk = 0; kk < k8; kk += 8)
                    acc += ld8(ar + kk) * ld8(br + kk);
                float s = hsum8(acc);
                for (size_t kk = k8; kk < k; kk++) s += ar[kk] * br[kk];
                float *dst = c + (i + ii) * ldc + j;
                *dst = accumulate ? *dst + s : s;
            }
    }
    for (; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            const float *ar = a + i * lda, *br = b + j * ldb;
            v8f acc = {0};
            for (size_t kk = 0; kk < k8; kk += 8)
                acc += ld8(ar + kk) * ld8(br + kk);
            float s = hsum8(acc);
            for (size_t kk = k8; kk < k; kk++) s += ar[kk] * br[kk];
            float *dst = c + i * ldc + j;
            *dst = accumulate ? *dst + s : s;
        }
}

/* K-block of the fp32 contraction: partial sums over KC-wide slices are
 * added in order. Changing it changes only the fp32 summation order, which
 * is how the tests measure the rounding-noise band of an implementation
 * that accumulates in fp32. */
static size_t g_gemm_kc = 512;
void qo_set_gemm_kc(size_t kc) { g_gemm_kc = kc ? kc : 512; }

static void gemm_nt_serial(const float *a, size_t lda, const float *b,
                           size_t ldb, float *c, size_t ldc, size_t m,
                           size_t n, size_t k) {
    const size_t KC = g_gemm_kc;
    for (size_t k0 = 0; k0 < k || (k == 0 && k0 == 0); k0 += KC) {
        size_t kc = k - k0 < KC ? k - k0 : KC;
        gemm_chunk(a + k0, lda, b + k0, ldb, c, ldc, m, n, kc, k0 > 0);
        if (k == 0) break;
    }
}

void qo_gemm_nt_f32(const float *a, size_t lda, const float *b, size_t ldb,
                    float *c, size_t ldc, size_t m, size_t n, size_t k) {
    const size_t MB = 96, NB = 128;
    size_t tm = (m + MB - 1) / MB, tn = (n + NB - 1) / NB;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
    for (size_t bi = 0; bi < tm; bi++)
        for (size_t bj = 0; bj < tn; bj++) {
            size_t mi = m - bi * MB < MB ? m - bi * MB : MB;
            size_t nj = n - bj * NB < NB ? n - bj * NB : NB;
            gemm_nt_serial(a + bi * MB * lda, lda, b + bj * NB * ldb, ldb,
                           c + bi * MB * ldc + bj * NB, ldc, mi, nj, k);
        }
}

/* ---------------------------------------------------------------------- */
/* linears                                                                */

static float *to_f32_rows(const uint16_t *x, size_t ld, size_t rows,
                          size_t k) {
    float *out = malloc(sizeof(float) * rows * k);
    if (!out) return NULL;
#pragma omp parallel for schedule(static) if (rows * k > 65536)
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < k; c++) out[r * k + c] = bf(x[r * ld + c]);
    return out;
}

void qo_linear(uint16_t *y, size_t ldy, const uint16_t *x, size_t ldx,
               const uint16_t *w, const uint16_t *bias, size_t rows,
               size_t k, size_t n) {
    /* h3_shaders.metal:788-816: fp32 accumulation of bf16 products (bias
     * folded in), one RNE rounding of the sum. */
    float *xf = to_f32_rows(x, ldx, rows, k);
    float *wf = to_f32_rows(w, k, n, k);
    float *acc = malloc(sizeof(float) * rows * n);
    qo_gemm_nt_f32(xf, k, wf, k, acc, n, rows, n, k);
#pragma omp parallel for schedule(static) if (rows * n > 65536)
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < n; c++) {
            float s = acc[r * n + c];
            if (bias) s += bf(bias[c]);
            y[r * ldy + c] = rne(s);
        }
    free(xf);
    free(wf);
    free(acc);
}

void qo_linear_i8(uint16_t *y, size_t ldy, const uint16_t *x, size_t ldx,
                  const int8_t *q, const float *scales, const uint16_t *bias,
                  size_t rows, size_t k, size_t n) {
    /* Weight-only int8: the contraction runs on the exact integer weights
     * and the per-output-channel scale multiplies the fp32 sum, which is
     * the dequantised product sum_k x (q s) up to fp32 rounding. */
    float *xf = to_f32_rows(x, ldx, rows, k);
    float *wf = malloc(sizeof(float) * n * k);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n * k; i++) wf[i] = (float)q[i];
    float *acc = malloc(sizeof(float) * rows * n);
    qo_gemm_nt_f32(xf, k, wf, k, acc, n, rows, n, k);
#pragma omp parallel for schedule(static) if (rows * n > 65536)
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < n; c++) {
            float s = acc[r * n + c] * scales[c];
            if (bias) s += bf(bias[c]);
            y[r * ldy + c] = rne(s);
        }
    free(xf);
    free(wf);
    free(acc);
}

void qo_quantize_int8_rows(int8_t *q, float *scales, const uint16_t *w,
                           size_t rows, size_t cols) {
    /* h3_shaders.metal:1320-1390, clip = 1.0: m = max|w|; scale = m/127
     * (1/127 for an all-zero row); q = clamp(rint(w * (127/m)), +-127). */
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++) {
        const uint16_t *row = w + r * cols;
        float mx = 0.0f;
        for (size_t c = 0; c < cols; c++) {
            float a = fabsf(bf(row[c]));
            if (a > mx) mx = a;
        }
        float clipped = mx * 1.0f;
        float scale = clipped > 0.0f ? clipped / 127.0f : 1.0f / 127.0f;
        float inverse = clipped > 0.0f ? 127.0f / clipped : 127.0f;
        scales[r] = scale;
        for (size_t c = 0; c < cols; c++) {
            int v = (int)rintf(bf(row[c]) * inverse);
            if (v > 127) v = 127;
            if (v < -127) v = -127;
            q[r * cols + c] = (int8_t)v;
        }
    }
}

void qo_dequant_int8_rows(float *w, const int8_t *q, const float *scales,
                          size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++)
            w[r * cols + c] = (float)q[r * cols + c] * scales[r];
}

/* ---------------------------------------------------------------------- */
/* normalisation / elementwise                                            */

void qo_layer_norm_mod(uint16_t *out, const uint16_t *in,
                       const uint16_t *modulation, const uint32_t *row_map,
                       size_t rows, size_t width, uint32_t slots,
                       uint32_t scale_slot, int shift_slot, float eps) {
    qo_layer_norm_mod_r(out, in, modulation, row_map, rows, width, slots,
                        scale_slot, shift_slot, eps, 0);
}

void qo_layer_norm_mod_r(uint16_t *out, const uint16_t *in,
                         const uint16_t *modulation, const uint32_t *row_map,
                         size_t rows, size_t width, uint32_t slots,
                         uint32_t scale_slot, int shift_slot, float eps,
                         int torch_rounding) {
    /* h3_shaders.metal:4767-4815: affine-free two-pass LayerNorm, then
     * x_hat * (1 + scale[row_map[r]]) (+ shift for the shift variant). */
#pragma omp parallel for schedule(static) if (rows * width > 65536)
    for (size_t r = 0; r < rows; r++) {
        const uint16_t *x = in + r * width;
        double sum = 0.0;
        for (size_t c = 0; c < width; c++) sum += bf(x[c]);
        float mean = (float)(sum / (double)width);
        double sq = 0.0;
        for (size_t c = 0; c < width; c++) {
            float d = bf(x[c]) - mean;
            sq += (double)d * (double)d;
        }
        float inv = (float)(1.0 / sqrt(sq / (double)width + (double)eps));
        const uint16_t *mod = modulation + (size_t)row_map[r] * slots * width;
        for (size_t c = 0; c < width; c++) {
            float nrm = (bf(x[c]) - mean) * inv;
            float one_plus = 1.0f + bf(mod[scale_slot * width + c]);
            if (torch_rounding) {
                nrm = round_bf(nrm);
                one_plus = round_bf(one_plus);
            }
            float v = nrm * one_plus;
            if (shift_slot >= 0) {
                if (torch_rounding) v = round_bf(v);
                v += bf(mod[(size_t)shift_slot * width + c]);
            }
            out[r * width + c] = rne(v);
        }
    }
}

void qo_rms_norm_one(uint16_t *out, const uint16_t *in, const uint16_t *w,
                     size_t rows, size_t width, float eps) {
    /* h3_shaders.metal:4817-4850: x * rsqrt(mean x^2 + eps) * (w + 1). */
    for (size_t r = 0; r < rows; r++) {
        const uint16_t *x = in + r * width;
        double sq = 0.0;
        for (size_t c = 0; c < width; c++) sq += (double)bf(x[c]) * bf(x[c]);
        float inv = (float)(1.0 / sqrt(sq / (double)width + (double)eps));
        for (size_t c = 0; c < width; c++)
            out[r * width + c] = rne(bf(x[c]) * inv * (bf(w[c]) + 1.0f));
    }
}

void qo_head_rms_norm(uint16_t *t, size_t ld, const uint16_t *w, size_t rows,
                      size_t heads, size_t head_dim, float eps) {
    /* h3_shaders.metal:4309-4329: per (row, head), single rounding of
     * x * inv * w. */
#pragma omp parallel for schedule(static) if (rows * heads > 4096)
    for (size_t r = 0; r < rows; r++)
        for (size_t h = 0; h < heads; h++) {
            uint16_t *x = t + r * ld + h * head_dim;
            double sq = 0.0;
            for (size_t d = 0; d < head_dim; d++)
                sq += (double)bf(x[d]) * bf(x[d]);
            float inv =
                (float)(1.0 / sqrt(sq / (double)head_dim + (double)eps));
            for (size_t d = 0; d < head_dim; d++)
                x[d] = rne(bf(x[d]) * inv * bf(w[d]));
        }
}

void qo_qk_rope(uint16_t *t, size_t ld, const float *cos_t, const float *sin_t,
                size_t rows, size_t heads, size_t head_dim) {
    /* h3_shaders.metal:4864-4896: interleaved pairs (2p, 2p+1), fp32,
     * each output rounded once. */
    size_t half = head_dim / 2;
#pragma omp parallel for schedule(static) if (rows * heads > 4096)
    for (size_t r = 0; r < rows; r++)
        for (size_t h = 0; h < heads; h++) {
            uint16_t *x = t + r * ld + h * head_dim;
            for (size_t p = 0; p < half; p++) {
                float c = cos_t[r * half + p], s = sin_t[r * half + p];
                float a = bf(x[2 * p]), b = bf(x[2 * p + 1]);
                x[2 * p] = rne(a * c - b * s);
                x[2 * p + 1] = rne(a * s + b * c);
            }
        }
}

void qo_gate(uint16_t *out, const uint16_t *residual, const uint16_t *branch,
             const uint16_t *modulation, const uint32_t *row_map, size_t rows,
             size_t width, uint32_t slots, uint32_t gate_slot) {
    qo_gate_r(out, residual, branch, modulation, row_map, rows, width, slots,
              gate_slot, 0);
}

void qo_gate_r(uint16_t *out, const uint16_t *residual, const uint16_t *branch,
               const uint16_t *modulation, const uint32_t *row_map,
               size_t rows, size_t width, uint32_t slots, uint32_t gate_slot,
               int torch_rounding) {
    /* h3_shaders.metal:3583-3599: res + branch * gate, one rounding. */
#pragma omp parallel for schedule(static) if (rows * width > 65536)
    for (size_t r = 0; r < rows; r++) {
        const uint16_t *g =
            modulation + ((size_t)row_map[r] * slots + gate_slot) * width;
        for (size_t c = 0; c < width; c++) {
            size_t i = r * width + c;
            float prod = bf(branch[i]) * bf(g[c]);
            if (torch_rounding) prod = round_bf(prod);
            out[i] = rne(bf(residual[i]) + prod);
        }
    }
}

static float gelu_tanh_f(float v) {
    /* h3_shaders.metal:3385-3408 (approximate): saturates at |inner| >= 10. */
    float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    if (inner <= -10.0f) return 0.0f;
    if (inner >= 10.0f) return v;
    return 0.5f * v * (1.0f + tanhf(inner));
}

void qo_gelu_tanh(uint16_t *out, const uint16_t *in, size_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (size_t i = 0; i < n; i++) out[i] = rne(gelu_tanh_f(bf(in[i])));
}

static float silu_f(float v) { return v / (1.0f + expf(-v)); }

void qo_silu(uint16_t *out, const uint16_t *in, size_t n) {
    /* h3_shaders.metal:3284-3291. */
    for (size_t i = 0; i < n; i++) out[i] = rne(silu_f(bf(in[i])));
}

void qo_swiglu(uint16_t *out, const uint16_t *fc1, size_t rows,
               size_t width) {
    /* h3_shaders.metal:5078-5095: silu(gate) rounded, times up, rounded. */
#pragma omp parallel for schedule(static) if (rows * width > 65536)
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < width; c++) {
            float g = bf(fc1[r * 2 * width + c]);
            float u = bf(fc1[r * 2 * width + width + c]);
            out[r * width + c] = rne(round_bf(silu_f(g)) * u);
        }
}

void qo_t2i_limits(uint32_t *limits, uint32_t rows, uint32_t text_rows,
                   int text_causal) {
    /* qwen_dit.m:1373-1440 (t2i): text row r sees keys [0, r] (causal) or
     * the whole text prefix; image rows see all rows. */
    for (uint32_t r = 0; r < rows; r++)
        limits[r] = r < text_rows ? (text_causal ? r + 1 : text_rows) : rows;
}

void qo_attention(uint16_t *out, size_t ldo, const uint16_t *q, size_t ldq,
                  const uint16_t *k, size_t ldk, const uint16_t *v, size_t ldv,
                  const uint32_t *limits, size_t q_rows, size_t kv_rows,
                  size_t heads, size_t head_dim, float scale) {
    qo_attention_ex(out, ldo, q, ldq, k, ldk, v, ldv, limits, q_rows, kv_rows,
                    heads, head_dim, scale, 0);
}

void qo_attention_ex(uint16_t *out, size_t ldo, const uint16_t *q, size_t ldq,
                     const uint16_t *k, size_t ldk, const uint16_t *v, size_t ldv,
                     const uint32_t *limits, size_t q_rows, size_t kv_rows,
                     size_t heads, size_t head_dim, float scale,
                     size_t prescale_rows) {
    /* tests/test_prefix_kernel.c:72-97: for each row, softmax over keys
     * [0, limit) of (q.k) * scale in fp32, times V; one bf16 rounding.
     * Rows below prescale_rows follow h3_shaders.metal:4397-4401 (the t2i
     * text rows): q is multiplied by the scale and re-rounded to bf16
     * before the contraction, and the scores are not scaled again. */
    const size_t QB = 48;
    size_t D = head_dim;
    float *kf = malloc(sizeof(float) * heads * kv_rows * D);
    float *vt = malloc(sizeof(float) * heads * D * kv_rows);
#pragma omp parallel for schedule(static)
    for (size_t h = 0; h < heads; h++)
        for (size_t r = 0; r < kv_rows; r++)
            for (size_t d = 0; d < D; d++) {
                kf[(h * kv_rows + r) * D + d] = bf(k[r * ldk + h * D + d]);
                vt[(h * D + d) * kv_rows + r] = bf(v[r * ldv + h * D + d]);
            }
    size_t nqb = (q_rows + QB - 1) / QB;
#pragma omp parallel
    {
        float *qf = malloc(sizeof(float) * QB * D);
        float *s = malloc(sizeof(float) * QB * kv_rows);
        float *o = malloc(sizeof(float) * QB * D);
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (size_t h = 0; h < heads; h++)
            for (size_t qb = 0; qb < nqb; qb++) {
                size_t r0 = qb * QB;
                size_t nr = q_rows - r0 < QB ? q_rows - r0 : QB;
                uint32_t lmax = 0;
                for (size_t i = 0; i < nr; i++) {
                    uint32_t l = limits[r0 + i];
                    if (l > kv_rows) l = (uint32_t)kv_rows;
                    if (l > lmax) lmax = l;
                }
                for (size_t i = 0; i < nr; i++)
                    for (size_t d = 0; d < D; d++) {
                        const float x = bf(q[(r0 + i) * ldq + h * D + d]);
                        qf[i * D + d] = r0 + i < prescale_rows ? bf(rne(x * scale)) : x;
                    }
                gemm_nt_serial(qf, D, kf + h * kv_rows * D, D, s, kv_rows, nr,
                               lmax, D);
                for (size_t i = 0; i < nr; i++) {
                    uint32_t l = limits[r0 + i];
                    if (l > kv_rows) l = (uint32_t)kv_rows;
                    float *row = s + i * kv_rows;
                    float m = -3.402823466e+38f;
                    const float sc = r0 + i < prescale_rows ? 1.0f : scale;
                    for (uint32_t j = 0; j < l; j++) {
                        row[j] *= sc;
                        if (row[j] > m) m = row[j];
                    }
                    float denom = 0.0f;
                    for (uint32_t j = 0; j < l; j++) {
                        row[j] = expf(row[j] - m);
                        denom += row[j];
                        if (g_attn_p_mode == 1) row[j] = bf(rne(row[j]));
                    }
                    float invd = denom > 0.0f ? 1.0f / denom : 0.0f;
                    for (uint32_t j = 0; j < l; j++) row[j] *= invd;
                    for (uint32_t j = l; j < lmax; j++) row[j] = 0.0f;
                }
                gemm_nt_serial(s, kv_rows, vt + h * D * kv_rows, kv_rows, o, D,
                               nr, D, lmax);
                for (size_t i = 0; i < nr; i++)
                    for (size_t d = 0; d < D; d++)
                        out[(r0 + i) * ldo + h * D + d] =
                            lmax ? rne(o[i * D + d]) : 0;
            }
        free(qf);
        free(s);
        free(o);
    }
    free(kf);
    free(vt);
}

void qo_modulation_reorder(uint16_t *slots_out, const uint16_t *raw,
                           size_t mod_rows, size_t hidden,
                           int shift_variant) {
    /* qwen_dit.m:1159-1186: copy the scales, tanh the gates in fp32 with a
     * truncating bf16 store. */
    size_t nraw = shift_variant ? 6 : 4;
    for (size_t r = 0; r < mod_rows; r++) {
        const uint16_t *src = raw + r * nraw * hidden;
        uint16_t *dst = slots_out + r * nraw * hidden;
        /* source chunk indices per block: shift, scale, gate */
        size_t sc1 = shift_variant ? 1 : 0, g1 = shift_variant ? 2 : 1;
        size_t sc2 = shift_variant ? 4 : 2, g2 = shift_variant ? 5 : 3;
        for (size_t c = 0; c < hidden; c++) {
            dst[0 * hidden + c] = src[sc1 * hidden + c];
            dst[1 * hidden + c] = src[sc2 * hidden + c];
            dst[2 * hidden + c] =
                qo_f32_to_bf16_trunc(tanhf(bf(src[g1 * hidden + c])));
            dst[3 * hidden + c] =
                qo_f32_to_bf16_trunc(tanhf(bf(src[g2 * hidden + c])));
            if (shift_variant) {
                dst[4 * hidden + c] = src[0 * hidden + c];
                dst[5 * hidden + c] = src[3 * hidden + c];
            }
        }
    }
}

/* ---------------------------------------------------------------------- */
/* model                                                                  */

/* Weight stream ids (also used by the GPU library's seeded create). */
enum {
    S_IMG_IN = 1, S_IMG_IN_B, S_TXT_NORM, S_TXT_IN1, S_TXT_IN1_B, S_TXT_IN2,
    S_TXT_IN2_B, S_TIME_L1, S_TIME_L1_B, S_TIME_L2, S_TIME_L2_B, S_MOD,
    S_MOD_B, S_NORM_OUT, S_NORM_OUT_B, S_PROJ_OUT, S_PROJ_OUT_B
};
enum {
    L_QKV = 1, L_QKV_B, L_OUT, L_OUT_B, L_FC1, L_FC1_B, L_FC2, L_FC2_B,
    L_NORM_Q, L_NORM_K
};
#define LAYER_STREAM(l, f) ((uint64_t)256 * (uint64_t)((l) + 1) + (f))

static const float W_STD = 0.02f;

static int lin_init(qo_lin *l, uint32_t n, uint32_t k, uint64_t seed,
                    uint64_t stream, uint64_t bstream, int bias, int int8) {
    memset(l, 0, sizeof(*l));
    l->n = n;
    l->k = k;
    l->int8 = int8;
    l->w = malloc(sizeof(uint16_t) * (size_t)n * k);
    if (!l->w) return 0;
    qo_fill_normal_bf16(l->w, (size_t)n * k, seed, stream, W_STD, 0.0f);
    if (bias) {
        l->bias = malloc(sizeof(uint16_t) * n);
        qo_fill_normal_bf16(l->bias, n, seed, bstream, W_STD, 0.0f);
    }
    if (int8) {
        l->q = malloc((size_t)n * k);
        l->scales = malloc(sizeof(float) * n);
        qo_quantize_int8_rows(l->q, l->scales, l->w, n, k);
        free(l->w);
        l->w = NULL;
    }
    return 1;
}

static void lin_free(qo_lin *l) {
    free(l->w);
    free(l->q);
    free(l->scales);
    free(l->bias);
    memset(l, 0, sizeof(*l));
}

void qo_apply_linear(const qo_lin *l, uint16_t *y, size_t ldy,
                     const uint16_t *x, size_t ldx, size_t rows) {
    if (l->int8)
        qo_linear_i8(y, ldy, x, ldx, l->q, l->scales, l->bias, rows, l->k,
                     l->n);
    else
        qo_linear(y, ldy, x, ldx, l->w, l->bias, rows, l->k, l->n);
}

int qo_model_init_random(qo_model *m, const qo_config *cfg, uint64_t seed,
                         uint32_t layers_to_build) {
    memset(m, 0, sizeof(*m));
    m->cfg = *cfg;
    uint32_t H = cfg->hidden, F = cfg->mlp_width;
    int b = cfg->has_bias, q8 = cfg->int8_weights;
    uint32_t nmod = (cfg->adaln_shift ? 6 : 4) * H;
    uint32_t nout = (cfg->adaln_shift ? 2 : 1) * H;
    /* Global projections stay bf16 (as the reference keeps them). */
    lin_init(&m->img_in, H, cfg->z_dim, seed, S_IMG_IN, S_IMG_IN_B, b, 0);
    m->txt_norm = malloc(sizeof(uint16_t) * cfg->text_dim);
    qo_fill_normal_bf16(m->txt_norm, cfg->text_dim, seed, S_TXT_NORM, W_STD,
                        0.0f);
    lin_init(&m->txt_in1, H, cfg->text_dim, seed, S_TXT_IN1, S_TXT_IN1_B, b, 0);
    lin_init(&m->txt_in2, H, H, seed, S_TXT_IN2, S_TXT_IN2_B, b, 0);
    lin_init(&m->time_l1, H, 256, seed, S_TIME_L1, S_TIME_L1_B, b, 0);
    lin_init(&m->time_l2, H, H, seed, S_TIME_L2, S_TIME_L2_B, b, 0);
    lin_init(&m->mod, nmod, H, seed, S_MOD, S_MOD_B, b, 0);
    lin_init(&m->norm_out, nout, H, seed, S_NORM_OUT, S_NORM_OUT_B, b, 0);
    lin_init(&m->proj_out, cfg->z_dim, H, seed, S_PROJ_OUT, S_PROJ_OUT_B, b, 0);
    m->layer = calloc(layers_to_build ? layers_to_build : 1, sizeof(qo_layer));
    uint32_t f1 = cfg->mlp_act == QO_MLP_SWIGLU ? 2 * F : F;
    for (uint32_t l = 0; l < layers_to_build; l++) {
        qo_layer *L = &m->layer[l];
        lin_init(&L->qkv, 3 * H, H, seed, LAYER_STREAM(l, L_QKV),
                 LAYER_STREAM(l, L_QKV_B), b, q8);
        lin_init(&L->out, H, H, seed, LAYER_STREAM(l, L_OUT),
                 LAYER_STREAM(l, L_OUT_B), b, q8);
        lin_init(&L->fc1, f1, H, seed, LAYER_STREAM(l, L_FC1),
                 LAYER_STREAM(l, L_FC1_B), b, q8);
        lin_init(&L->fc2, H, F, seed, LAYER_STREAM(l, L_FC2),
                 LAYER_STREAM(l, L_FC2_B), b, q8);
        L->norm_q = malloc(sizeof(uint16_t) * 128);
        L->norm_k = malloc(sizeof(uint16_t) * 128);
        qo_fill_normal_bf16(L->norm_q, 128, seed, LAYER_STREAM(l, L_NORM_Q),
                            W_STD, 1.0f);
        qo_fill_normal_bf16(L->norm_k, 128, seed, LAYER_STREAM(l, L_NORM_K),
                            W_STD, 1.0f);
    }
    m->cfg.layers = layers_to_build;
    return 1;
}

void qo_model_free(qo_model *m) {
    lin_free(&m->img_in);
    lin_free(&m->txt_in1);
    lin_free(&m->txt_in2);
    lin_free(&m->time_l1);
    lin_free(&m->time_l2);
    lin_free(&m->mod);
    lin_free(&m->norm_out);
    lin_free(&m->proj_out);
    free(m->txt_norm);
    for (uint32_t l = 0; l < m->cfg.layers; l++) {
        lin_free(&m->layer[l].qkv);
        lin_free(&m->layer[l].out);
        lin_free(&m->layer[l].fc1);
        lin_free(&m->layer[l].fc2);
        free(m->layer[l].norm_q);
        free(m->layer[l].norm_k);
    }
    free(m->layer);
    memset(m, 0, sizeof(*m));
}

void qo_embed(const qo_model *m, const uint16_t *text_in, uint32_t text_rows,
              const uint16_t *latents, uint32_t image_rows, uint16_t *joint) {
    /* qwen_dit.m:1031-1083. */
    size_t H = m->cfg.hidden;
    if (text_rows) {
        uint16_t *normed = malloc(sizeof(uint16_t) * text_rows * m->cfg.text_dim);
        uint16_t *wide = malloc(sizeof(uint16_t) * text_rows * H);
        qo_rms_norm_one(normed, text_in, m->txt_norm, text_rows,
                        m->cfg.text_dim, 1e-6f);
        qo_apply_linear(&m->txt_in1, wide, H, normed, m->cfg.text_dim,
                        text_rows);
        qo_gelu_tanh(wide, wide, (size_t)text_rows * H);
        qo_apply_linear(&m->txt_in2, joint, H, wide, H, text_rows);
        free(normed);
        free(wide);
    }
    if (image_rows)
        qo_apply_linear(&m->img_in, joint + (size_t)text_rows * H, H, latents,
                        m->cfg.z_dim, image_rows);
}

void qo_conditioning(const qo_model *m, const float *features,
                     uint32_t mod_rows, uint16_t *temb, uint16_t *modulation,
                     uint16_t *norm_out_mod) {
    /* qwen_dit.m:1098-1192. */
    size_t H = m->cfg.hidden;
    uint16_t *fb = malloc(sizeof(uint16_t) * mod_rows * 256);
    uint16_t *wide = malloc(sizeof(uint16_t) * mod_rows * H);
    uint16_t *st = malloc(sizeof(uint16_t) * mod_rows * H);
    size_t nmod = m->mod.n;
    uint16_t *raw = malloc(sizeof(uint16_t) * mod_rows * nmod);
    qo_f32_to_bf16_array(features, fb, (size_t)mod_rows * 256);
    qo_apply_linear(&m->time_l1, wide, H, fb, 256, mod_rows);
    qo_silu(wide, wide, (size_t)mod_rows * H);
    qo_apply_linear(&m->time_l2, temb, H, wide, H, mod_rows);
    qo_silu(st, temb, (size_t)mod_rows * H);
    qo_apply_linear(&m->norm_out, norm_out_mod, m->norm_out.n, st, H, mod_rows);
    qo_apply_linear(&m->mod, raw, nmod, st, H, mod_rows);
    qo_modulation_reorder(modulation, raw, mod_rows, H, m->cfg.adaln_shift);
    free(fb);
    free(wide);
    free(st);
    free(raw);
}

void qo_block(const qo_model *m, int layer, uint16_t *hidden,
              const uint16_t *modulation, const float *rope_cos,
              const float *rope_sin, const uint32_t *row_map, uint32_t rows,
              uint32_t text_rows, const uint32_t *limits,
              uint16_t *debug_attn) {
    /* qwen_dit.m:1220-1476 with the fused layout of this build: q|k|v in
     * one [rows, 3H] buffer, gate fused after each projection. */
    const qo_layer *L = &m->layer[layer];
    size_t H = m->cfg.hidden, F = m->cfg.mlp_width, heads = m->cfg.heads;
    uint32_t slots = m->cfg.adaln_shift ? 6 : 4;
    int sh = m->cfg.adaln_shift;
    uint16_t *mod = malloc(sizeof(uint16_t) * rows * H);
    uint16_t *qkv = malloc(sizeof(uint16_t) * rows * 3 * H);
    uint16_t *attn = malloc(sizeof(uint16_t) * rows * H);
    uint16_t *branch = malloc(sizeof(uint16_t) * rows * H);
    size_t f1 = m->cfg.mlp_act == QO_MLP_SWIGLU ? 2 * F : F;
    uint16_t *wide = malloc(sizeof(uint16_t) * rows * f1);
    uint16_t *act = m->cfg.mlp_act == QO_MLP_SWIGLU
                        ? malloc(sizeof(uint16_t) * rows * F)
                        : wide;
    uint32_t *lim = malloc(sizeof(uint32_t) * rows);
    if (limits)
        memcpy(lim, limits, sizeof(uint32_t) * rows);
    else
        qo_t2i_limits(lim, rows, text_rows, m->cfg.text_causal);

    qo_layer_norm_mod(mod, hidden, modulation, row_map, rows, H, slots, 0,
                      sh ? 4 : -1, 1e-6f);
    qo_apply_linear(&L->qkv, qkv, 3 * H, mod, H, rows);
    qo_head_rms_norm(qkv, 3 * H, L->norm_q, rows, heads, 128, 1e-6f);
    qo_head_rms_norm(qkv + H, 3 * H, L->norm_k, rows, heads, 128, 1e-6f);
    qo_qk_rope(qkv, 3 * H, rope_cos, rope_sin, rows, heads, 128);
    qo_qk_rope(qkv + H, 3 * H, rope_cos, rope_sin, rows, heads, 128);
    /* t2i: text rows pre-scale q (h3_shaders.metal:4397-4401); ti2i prefix
     * tables run every row through the flash prefix kernel, which does not */
    qo_attention_ex(attn, H, qkv, 3 * H, qkv + H, 3 * H, qkv + 2 * H, 3 * H, lim,
                    rows, rows, heads, 128, 1.0f / sqrtf(128.0f),
                    limits ? 0 : text_rows);
    if (debug_attn) memcpy(debug_attn, attn, sizeof(uint16_t) * rows * H);
    qo_apply_linear(&L->out, branch, H, attn, H, rows);
    qo_gate(hidden, hidden, branch, modulation, row_map, rows, H, slots, 2);
    qo_layer_norm_mod(mod, hidden, modulation, row_map, rows, H, slots, 1,
                      sh ? 5 : -1, 1e-6f);
    qo_apply_linear(&L->fc1, wide, f1, mod, H, rows);
    if (m->cfg.mlp_act == QO_MLP_SWIGLU)
        qo_swiglu(act, wide, rows, F);
    else
        qo_gelu_tanh(act, wide, (size_t)rows * F);
    qo_apply_linear(&L->fc2, branch, H, act, F, rows);
    qo_gate(hidden, hidden, branch, modulation, row_map, rows, H, slots, 3);
    free(mod);
    free(qkv);
    free(attn);
    free(branch);
    if (act != wide) free(act);
    free(wide);
    free(lim);
}

void qo_block_rows(const qo_model *m, int layer, const uint16_t *hidden,
                   const uint16_t *modulation, const float *rope_cos,
                   const float *rope_sin, const uint32_t *row_map,
                   uint32_t rows, uint32_t text_rows, const uint32_t *sample,
                   uint32_t n_sample, uint16_t *out) {
    /* qo_block restricted to the output rows listed in `sample`: every row
     * goes through LN1 + QKV + q/k norm + RoPE (the sampled rows attend
     * all of their keys), the rest of the block runs on the sampled rows
     * only. Row-wise stages are identical to qo_block's; t2i limits. */
    const qo_layer *L = &m->layer[layer];
    size_t H = m->cfg.hidden, F = m->cfg.mlp_width, heads = m->cfg.heads;
    uint32_t slots = m->cfg.adaln_shift ? 6 : 4;
    int sh = m->cfg.adaln_shift;
    size_t f1 = m->cfg.mlp_act == QO_MLP_SWIGLU ? 2 * F : F;
    uint16_t *mod = malloc(sizeof(uint16_t) * rows * H);
    uint16_t *qkv = malloc(sizeof(uint16_t) * rows * 3 * H);
    uint16_t *q_s = malloc(sizeof(uint16_t) * n_sample * H);
    uint16_t *h_s = malloc(sizeof(uint16_t) * n_sample * H);
    uint16_t *attn = malloc(sizeof(uint16_t) * n_sample * H);
    uint16_t *branch = malloc(sizeof(uint16_t) * n_sample * H);
    uint16_t *mod_s = malloc(sizeof(uint16_t) * n_sample * H);
    uint16_t *wide = malloc(sizeof(uint16_t) * n_sample * f1);
    uint16_t *act = m->cfg.mlp_act == QO_MLP_SWIGLU
                        ? malloc(sizeof(uint16_t) * n_sample * F)
                        : wide;
    uint32_t *lim_all = malloc(sizeof(uint32_t) * rows);
    uint32_t *lim = malloc(sizeof(uint32_t) * n_sample);
    uint32_t *rm_s = malloc(sizeof(uint32_t) * n_sample);
    qo_t2i_limits(lim_all, rows, text_rows, m->cfg.text_causal);
    qo_layer_norm_mod(mod, hidden, modulation, row_map, rows, H, slots, 0,
                      sh ? 4 : -1, 1e-6f);
    qo_apply_linear(&L->qkv, qkv, 3 * H, mod, H, rows);
    qo_head_rms_norm(qkv, 3 * H, L->norm_q, rows, heads, 128, 1e-6f);
    qo_head_rms_norm(qkv + H, 3 * H, L->norm_k, rows, heads, 128, 1e-6f);
    qo_qk_rope(qkv, 3 * H, rope_cos, rope_sin, rows, heads, 128);
    qo_qk_rope(qkv + H, 3 * H, rope_cos, rope_sin, rows, heads, 128);
    /* sampled rows, text rows first so the t2i text rule covers a prefix */
    uint32_t n_text = 0;
    for (uint32_t i = 0; i < n_sample; i++) n_text += sample[i] < text_rows;
    uint32_t *order = malloc(sizeof(uint32_t) * n_sample);
    uint32_t no = 0;
    for (int pass = 0; pass < 2; pass++)
        for (uint32_t i = 0; i < n_sample; i++)
            if ((sample[i] < text_rows) == (pass == 0)) order[no++] = i;
    for (uint32_t j = 0; j < n_sample; j++) {
        const uint32_t r = sample[order[j]];
        memcpy(q_s + (size_t)j * H, qkv + (size_t)r * 3 * H, sizeof(uint16_t) * H);
        memcpy(h_s + (size_t)j * H, hidden + (size_t)r * H, sizeof(uint16_t) * H);
        lim[j] = lim_all[r];
        rm_s[j] = row_map[r];
    }
    qo_attention_ex(attn, H, q_s, H, qkv + H, 3 * H, qkv + 2 * H, 3 * H, lim,
                    n_sample, rows, heads, 128, 1.0f / sqrtf(128.0f), n_text);
    qo_apply_linear(&L->out, branch, H, attn, H, n_sample);
    qo_gate(h_s, h_s, branch, modulation, rm_s, n_sample, H, slots, 2);
    qo_layer_norm_mod(mod_s, h_s, modulation, rm_s, n_sample, H, slots, 1,
                      sh ? 5 : -1, 1e-6f);
    qo_apply_linear(&L->fc1, wide, f1, mod_s, H, n_sample);
    if (m->cfg.mlp_act == QO_MLP_SWIGLU)
        qo_swiglu(act, wide, n_sample, F);
    else
        qo_gelu_tanh(act, wide, (size_t)n_sample * F);
    qo_apply_linear(&L->fc2, branch, H, act, F, n_sample);
    qo_gate(h_s, h_s, branch, modulation, rm_s, n_sample, H, slots, 3);
    for (uint32_t j = 0; j < n_sample; j++)
        memcpy(out + (size_t)order[j] * H, h_s + (size_t)j * H, sizeof(uint16_t) * H);
    free(order);
    free(mod);
    free(qkv);
    free(q_s);
    free(h_s);
    free(attn);
    free(branch);
    free(mod_s);
    if (act != wide) free(act);
    free(wide);
    free(lim_all);
    free(lim);
    free(rm_s);
}

void qo_final(const qo_model *m, const uint16_t *hidden,
              const uint16_t *norm_out_mod, const uint32_t *row_map,
              uint32_t rows, uint16_t *output) {
    /* qwen_dit.m:1478-1496: scale-only (or scale+shift) LN, then proj_out. */
    size_t H = m->cfg.hidden;
    int sh = m->cfg.adaln_shift;
    uint16_t *mod = malloc(sizeof(uint16_t) * rows * H);
    qo_layer_norm_mod(mod, hidden, norm_out_mod, row_map, rows, H, sh ? 2 : 1,
                      0, sh ? 1 : -1, 1e-6f);
    qo_apply_linear(&m->proj_out, output, m->cfg.z_dim, mod, H, rows);
    free(mod);
}

int qo_forward(const qo_model *m, const uint16_t *text_in, uint32_t text_rows,
               const uint16_t *latents, uint32_t image_rows, float sigma,
               const float *rope_cos, const float *rope_sin, uint32_t layers,
               uint16_t *output) {
    /* qwen_dit.m:1498-1568: row_map text -> 1 (t = 0 row), image -> 0. */
    if (layers > m->cfg.layers) return 0;
    uint32_t rows = text_rows + image_rows;
    size_t H = m->cfg.hidden;
    uint16_t *joint = malloc(sizeof(uint16_t) * rows * H);
    uint32_t *row_map = malloc(sizeof(uint32_t) * rows);
    for (uint32_t i = 0; i < rows; i++) row_map[i] = i < text_rows ? 1u : 0u;
    qo_embed(m, text_in, text_rows, latents, image_rows, joint);
    float sig[2] = {sigma, 0.0f}, feat[512];
    qo_timestep_features(sig, 2, feat);
    uint32_t slots = m->cfg.adaln_shift ? 6 : 4;
    uint16_t *temb = malloc(sizeof(uint16_t) * 2 * H);
    uint16_t *mod = malloc(sizeof(uint16_t) * 2 * slots * H);
    uint16_t *nout = malloc(sizeof(uint16_t) * 2 * m->norm_out.n);
    qo_conditioning(m, feat, 2, temb, mod, nout);
    for (uint32_t l = 0; l < layers; l++)
        qo_block(m, (int)l, joint, mod, rope_cos, rope_sin, row_map, rows,
                 text_rows, NULL, NULL);
    qo_final(m, joint, nout, row_map, rows, output);
    free(joint);
    free(row_map);
    free(temb);
    free(mod);
    free(nout);
    return 1;
}

void qo_prefix_limits(const qo_segment *segs, uint32_t seg_count, uint32_t *limits) {
    /* qwen_dit.m:1651-1665 */
    uint32_t start = 0;
    for (uint32_t s = 0; s < seg_count; s++) {
        for (uint32_t r = 0; r < segs[s].rows; r++)
            limits[start + r] = segs[s].is_image ? start + segs[s].rows : start + r + 1;
        start += segs[s].rows;
    }
}

int qo_forward_ti2i(const qo_model *m, const uint16_t *text_in, uint32_t text_total,
                    const uint16_t *latents, uint32_t image_total, const qo_segment *segs,
                    uint32_t seg_count, float sigma, const float *rope_cos,
                    const float *rope_sin, uint32_t layers, uint16_t *output) {
    if (!seg_count || !segs[seg_count - 1].is_image || layers > m->cfg.layers) return 0;
    uint32_t rows = 0;
    for (uint32_t s = 0; s < seg_count; s++) {
        const uint32_t have = segs[s].is_image ? image_total : text_total;
        if (segs[s].src_offset > have || segs[s].rows > have - segs[s].src_offset) return 0;
        rows += segs[s].rows;
    }
    const size_t H = m->cfg.hidden;
    const uint32_t target = segs[seg_count - 1].rows, prefix = rows - target;
    /* qwen_dit.m:1572-1648: project every source row, then scatter runs */
    uint16_t *proj = malloc(sizeof(uint16_t) * (size_t)(text_total + image_total) * H);
    uint16_t *joint = malloc(sizeof(uint16_t) * (size_t)rows * H);
    uint32_t *row_map = malloc(sizeof(uint32_t) * rows);
    uint32_t *limits = malloc(sizeof(uint32_t) * rows);
    if (!proj || !joint || !row_map || !limits) {
        free(proj);
        free(joint);
        free(row_map);
        free(limits);
        return 0;
    }
    qo_embed(m, text_in, text_total, latents, image_total, proj);
    uint32_t at = 0;
    for (uint32_t s = 0; s < seg_count; s++) {
        const size_t src = (size_t)(segs[s].is_image ? text_total : 0) + segs[s].src_offset;
        memcpy(joint + (size_t)at * H, proj + src * H, sizeof(uint16_t) * segs[s].rows * H);
        at += segs[s].rows;
    }
    /* qwen_dit.m:1725-1729: only the target run reads the sampled step */
    for (uint32_t i = 0; i < rows; i++) row_map[i] = i < prefix ? 1u : 0u;
    qo_prefix_limits(segs, seg_count, limits);
    float sig[2] = {sigma, 0.0f}, feat[512];
    qo_timestep_features(sig, 2, feat);
    const uint32_t slots = m->cfg.adaln_shift ? 6 : 4;
    uint16_t *temb = malloc(sizeof(uint16_t) * 2 * H);
    uint16_t *mod = malloc(sizeof(uint16_t) * 2 * slots * H);
    uint16_t *nout = malloc(sizeof(uint16_t) * 2 * m->norm_out.n);
    qo_conditioning(m, feat, 2, temb, mod, nout);
    for (uint32_t l = 0; l < layers; l++)
        qo_block(m, (int)l, joint, mod, rope_cos, rope_sin, row_map, rows, 0, limits, NULL);
    qo_final(m, joint, nout, row_map, rows, output);
    free(proj);
    free(joint);
    free(row_map);
    free(limits);
    free(temb);
    free(mod);
    free(nout);
    return 1;
}

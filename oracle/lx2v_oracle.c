/*
 * lx2v_oracle.c -- CPU restatement of lightx2v-rs's quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Build: gcc -O2 -ffp-contract=off (no fast-math), see oracle/Makefile.
 * Rust never contracts a*b+c into an FMA, so neither may this file.
 *
 * Parity status of each part is recorded in the test that pins it
 * (tests/test_oracle_*.py); every function below cites the reference line
 * it restates.
 */
#include "lx2v_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- Rust `as` cast helpers -------------------------------------------- */

/* float -> u8: saturating, truncating, NaN -> 0. */
static uint8_t as_u8(float f) {
    if (isnan(f) || f <= 0.0f) return 0;
    if (f >= 255.0f) return 255;
    return (uint8_t)f;
}

/* float -> i8: saturating, truncating, NaN -> 0. */
static int8_t as_i8(float f) {
    if (isnan(f)) return 0;
    if (f <= -128.0f) return -128;
    if (f >= 127.0f) return 127;
    return (int8_t)f;
}

/* float -> i32: saturating, truncating, NaN -> 0. */
static int32_t as_i32(float f) {
    if (isnan(f)) return 0;
    if (f <= -2147483648.0f) return INT32_MIN;
    if (f >= 2147483648.0f) return INT32_MAX;
    return (int32_t)f;
}

/* f32::clamp: NaN passes through. */
static float rclamp(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* 2f32.powi(e) for |e| small: every intermediate is a power of two, so the
 * repeated-multiplication lowering is exact. */
static float pow2i(int e) { return ldexpf(1.0f, e); }

/* ---- Rng: crates/lightx2v-core/src/rng.rs ------------------------------ */

#define GOLDEN 0x9E3779B97F4A7C15ull

void orc_rng_new(orc_rng *r, uint64_t seed) { r->state = seed + GOLDEN; } /* rng.rs:13-18 */

uint64_t orc_rng_next_u64(orc_rng *r) { /* rng.rs:20-27 */
    r->state += GOLDEN;
    uint64_t z = r->state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float orc_rng_next_f32(orc_rng *r) { /* rng.rs:29-31 */
    return (float)(orc_rng_next_u64(r) >> 40) / (float)(1ull << 24);
}

void orc_rng_uniform(orc_rng *r, float *out, size_t n, float a) { /* rng.rs:34-36 */
    for (size_t i = 0; i < n; i++) out[i] = (orc_rng_next_f32(r) * 2.0f - 1.0f) * a;
}

void orc_rng_normal(orc_rng *r, float *out, size_t n) { /* rng.rs:39-54 */
    const float two_pi = 2.0f * 3.14159265358979323846f; /* 2.0 * f32 PI, exact doubling */
    size_t len = 0;
    while (len < n) {
        float u1 = fmaxf(orc_rng_next_f32(r), 1e-7f);
        float u2 = orc_rng_next_f32(r);
        float rad = sqrtf(-2.0f * logf(u1));
        float t = two_pi * u2;
        out[len++] = rad * cosf(t);
        if (len < n) out[len++] = rad * sinf(t);
    }
}

/* ---- e4m3 codecs ------------------------------------------------------- */

uint8_t orc_f32_to_e4m3_ref(float v) { /* quant.rs:376-406 */
    if (v == 0.0f) return signbit(v) ? 0x80 : 0x00;
    uint8_t sign = signbit(v) ? 0x80 : 0x00;
    float a = fabsf(v);
    if (!isfinite(a) || a >= 464.0f) return sign | 0x7E;
    int32_t e = as_i32(floorf(log2f(a)));
    if (e < -9) {
        /* (a / (2^-9 / 8)).round() as u8, then min(7) */
        uint8_t m = as_u8(roundf(a / (pow2i(-9) / 8.0f)));
        return sign | (m < 7 ? m : 7);
    }
    if (e > 8) return sign | 0x7E;
    uint8_t exp = (uint8_t)(e + 7); /* `(e + 7) as u8` wraps: -2 -> 254, -1 -> 255 */
    uint8_t mant = as_u8(roundf((a / pow2i(e) - 1.0f) * 8.0f));
    if (mant >= 8) {
        if (exp >= 15) return sign | 0x7E;
        return sign | (uint8_t)((uint8_t)(exp + 1) << 3);
    }
    return sign | (uint8_t)(exp << 3) | mant; /* u8 << 3 drops the high bits */
}

float orc_e4m3_to_f32_ref(uint8_t code) { /* quant.rs:409-420 */
    float sign = (code & 0x80) ? -1.0f : 1.0f;
    uint8_t exp = (code >> 3) & 0xF;
    uint8_t mant = code & 0x7;
    if (exp == 0) return sign * ((float)mant / 8.0f) * pow2i(-9);
    if (exp == 0xF && mant == 0x7) return NAN;
    return sign * (1.0f + (float)mant / 8.0f) * pow2i((int)exp - 7);
}

uint8_t orc_f32_to_e4m3_canon(float v) {
    uint8_t sign = signbit(v) ? 0x80 : 0x00;
    float a = fabsf(v);
    if (a >= 0x1p-6f || isnan(a)) return orc_f32_to_e4m3_ref(v);
    if (a > 0x1p-7f) return sign | 0x08; /* nearest of {0, 2^-6} */
    return sign;                         /* signed zero */
}

float orc_e4m3_to_f32_ocp(uint8_t code) {
    float sign = (code & 0x80) ? -1.0f : 1.0f;
    int exp = (code >> 3) & 0xF;
    int mant = code & 0x7;
    if (exp == 0xF && mant == 0x7) return NAN;
    if (exp == 0) return sign * (float)mant * pow2i(-9);
    return sign * (1.0f + (float)mant / 8.0f) * pow2i(exp - 7);
}

uint8_t orc_f32_to_e4m3_ocp_rne(float v) {
    if (isnan(v)) return 0x7F;
    uint8_t sign = signbit(v) ? 0x80 : 0x00;
    float a = fabsf(v);
    if (a >= 0x1p-6f) {
        uint32_t b;
        memcpy(&b, &a, 4);
        b += 0x7FFFFu + ((b >> 20) & 1u); /* RNE from 23 to 3 mantissa bits */
        int e8 = (int)(b >> 23) - 127 + 7;
        uint32_t m = (b >> 20) & 7u;
        if (e8 > 15 || (e8 == 15 && m == 7)) return sign | 0x7E; /* saturate */
        return sign | (uint8_t)(e8 << 3) | (uint8_t)m;
    }
    /* subnormal grid m * 2^-9; m == 8 is the encoding of 2^-6 (0x08) */
    float m = nearbyintf(a * 512.0f);
    return sign | (uint8_t)m;
}

/* ---- f16 / bf16 -------------------------------------------------------- */

uint16_t orc_f32_to_f16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {
        if (ax > 0x7F800000u) return sign | 0x7E00u | (uint16_t)((ax >> 13) & 0x3FFu);
        return sign | 0x7C00u;
    }
    if (ax >= 0x477FF000u) return sign | 0x7C00u; /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                      /* >= 2^-14: normal */
        uint32_t r = ax + 0x0FFFu + ((ax >> 13) & 1u);
        r -= (uint32_t)(127 - 15) << 23;
        return sign | (uint16_t)(r >> 13);
    }
    float a;
    memcpy(&a, &ax, 4);
    float m = nearbyintf(a * 16777216.0f); /* subnormal grid m * 2^-24 */
    return sign | (uint16_t)m;
}

static float f16_bits_to_f32(uint16_t h) {
    float sign = (h & 0x8000u) ? -1.0f : 1.0f;
    int e = (h >> 10) & 0x1F;
    int m = h & 0x3FF;
    if (e == 0) return sign * (float)m * pow2i(-24);
    if (e == 31) return m ? NAN : sign * INFINITY;
    return sign * (1.0f + (float)m / 1024.0f) * pow2i(e - 15);
}

float orc_f16_round(float v) { return f16_bits_to_f32(orc_f32_to_f16_bits(v)); }

uint16_t orc_f32_to_bf16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float orc_bf16_round(float v) {
    uint32_t x = (uint32_t)orc_f32_to_bf16_bits(v) << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

float orc_gelu_tanh(float x) { /* crates/lightx2v-cpu/src/lib.rs:151-153 */
    const float c = sqrtf(2.0f / 3.14159265358979323846f);
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

/* ---- Q8 ------------------------------------------------------------------ */

size_t orc_q8_ref_group(size_t cols) { return cols % 128 == 0 ? 128 : cols; }

void orc_q8_quantize(const float *data, size_t rows, size_t cols, size_t group,
                     int8_t *q, float *scales) { /* quant.rs:154-178 */
    size_t n = rows * cols, gi = 0;
    for (size_t g0 = 0; g0 < n; g0 += group, gi++) {
        size_t len = n - g0 < group ? n - g0 : group;
        float amax = 0.0f;
        for (size_t i = 0; i < len; i++) amax = fmaxf(amax, fabsf(data[g0 + i]));
        float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        for (size_t i = 0; i < len; i++)
            q[g0 + i] = as_i8(rclamp(roundf(data[g0 + i] / s), -127.0f, 127.0f));
        scales[gi] = s;
    }
}

void orc_q8_dequantize(const int8_t *q, const float *scales, size_t rows,
                       size_t cols, size_t group, float *out) { /* quant.rs:180-186 */
    size_t n = rows * cols;
    for (size_t i = 0; i < n; i++) out[i] = (float)q[i] * scales[i / group];
}

/* ---- Q4 ------------------------------------------------------------------ */

static float q4_code(float v, float is, float z) { /* quant.rs:247 */
    return rclamp(roundf(v * is + z), 0.0f, 15.0f);
}

void orc_q4_quantize(const float *data, size_t rows, size_t cols, size_t group,
                     int hqq, uint8_t *codes, float *scales, float *zeros) { /* quant.rs:226-292 */
    size_t n = rows * cols, gi = 0;
    for (size_t g0 = 0; g0 < n; g0 += group, gi++) {
        const float *w = data + g0;
        size_t len = n - g0 < group ? n - g0 : group;
        float lo = FLT_MAX, hi = -FLT_MAX;
        for (size_t i = 0; i < len; i++) {
            lo = fminf(lo, w[i]);
            hi = fmaxf(hi, w[i]);
        }
        float is = hi > lo ? 15.0f / (hi - lo) : 1.0f;
        float z = -lo * is;
        if (hqq) { /* quant.rs:248-276 */
            const float p = 0.7f, kappa = 1.01f;
            float beta = 10.0f;
            float best = FLT_MAX, best_z = z;
            for (int it = 0; it < 20; it++) {
                float err = 0.0f, zsum = 0.0f;
                for (size_t i = 0; i < len; i++) {
                    float v = w[i];
                    float c = q4_code(v, is, z);
                    float r = (c - z) / is;
                    float e = v - r;
                    err += fabsf(e);
                    float a = fabsf(e);
                    float sh = 0.0f;
                    if (a > 0.0f) {
                        float sg = signbit(e) ? -1.0f : 1.0f; /* f32::signum */
                        sh = sg * fmaxf(a - powf(a, p - 1.0f) / beta, 0.0f);
                    }
                    zsum += c - (v - sh) * is;
                }
                err = err / (float)len;
                if (err >= best) break;
                best = err;
                best_z = z;
                z = zsum / (float)len;
                beta *= kappa;
            }
            z = best_z;
        }
        for (size_t i = 0; i < len; i++) codes[g0 + i] = as_u8(q4_code(w[i], is, z));
        scales[gi] = orc_f16_round(1.0f / is); /* quant.rs:280-281 */
        zeros[gi] = orc_f16_round(z);
    }
}

void orc_q4_quantize_sym(const float *data, size_t rows, size_t cols, size_t group,
                         uint8_t *codes, float *scales, float *zeros) {
    size_t n = rows * cols, gi = 0;
    for (size_t g0 = 0; g0 < n; g0 += group, gi++) {
        size_t len = n - g0 < group ? n - g0 : group;
        float amax = 0.0f;
        for (size_t i = 0; i < len; i++) amax = fmaxf(amax, fabsf(data[g0 + i]));
        float s = amax > 0.0f ? amax / 7.0f : 1.0f;
        for (size_t i = 0; i < len; i++) {
            float q = rclamp(roundf(data[g0 + i] / s), -8.0f, 7.0f);
            codes[g0 + i] = (uint8_t)(as_i8(q) + 8);
        }
        scales[gi] = s;
        zeros[gi] = 8.0f;
    }
}

void orc_q4_dequantize(const uint8_t *codes, const float *scales, const float *zeros,
                       size_t rows, size_t cols, size_t group, float *out) { /* quant.rs:294-303 */
    size_t n = rows * cols;
    for (size_t i = 0; i < n; i++) {
        size_t g = i / group;
        out[i] = ((float)codes[i] - zeros[g]) * scales[g];
    }
}

void orc_q4_pack(const uint8_t *codes, size_t n, uint8_t *packed) { /* quant.rs:306-311 */
    for (size_t i = 0; i < n; i += 2) {
        uint8_t hi = i + 1 < n ? codes[i + 1] : 0;
        packed[i / 2] = (uint8_t)(codes[i] | (uint8_t)(hi << 4));
    }
}

void orc_q4_unpack(const uint8_t *packed, size_t n, uint8_t *codes) { /* quant.rs:324-326 */
    for (size_t i = 0; i < n; i++) codes[i] = (packed[i / 2] >> (4 * (i % 2))) & 15;
}

/* ---- FP8 ----------------------------------------------------------------- */

size_t orc_fp8_ref_group(size_t cols) { return cols % 128 == 0 ? 128 : cols; }

void orc_fp8_quantize(const float *data, size_t rows, size_t cols, size_t group,
                      int canon, uint8_t *q, float *scales) { /* quant.rs:423-447 */
    size_t n = rows * cols, gi = 0;
    for (size_t g0 = 0; g0 < n; g0 += group, gi++) {
        size_t len = n - g0 < group ? n - g0 : group;
        float amax = 0.0f;
        for (size_t i = 0; i < len; i++) amax = fmaxf(amax, fabsf(data[g0 + i]));
        float s = amax > 0.0f ? amax / 448.0f : 1.0f;
        for (size_t i = 0; i < len; i++) {
            float v = data[g0 + i] / s;
            q[g0 + i] = canon ? orc_f32_to_e4m3_canon(v) : orc_f32_to_e4m3_ref(v);
        }
        scales[gi] = s;
    }
}

void orc_fp8_dequantize(const uint8_t *q, const float *scales, size_t rows,
                        size_t cols, size_t group, float *out) { /* quant.rs:449-455 */
    size_t n = rows * cols;
    for (size_t i = 0; i < n; i++) out[i] = orc_e4m3_to_f32_ref(q[i]) * scales[i / group];
}

/* ---- linear -------------------------------------------------------------- */

static void linear_rows(const float *x, size_t x_row, size_t r0, size_t r1,
                        const float *w, size_t n, size_t k, const float *bias,
                        int act, float *y, size_t y_row) {
    for (size_t r = r0; r < r1; r++) {
        const float *xr = x + (x_row + r) * k;
        float *yr = y + (y_row + r) * n;
        for (size_t o = 0; o < n; o++) {
            const float *wr = w + o * k;
            float acc = 0.0f;
            for (size_t i = 0; i < k; i++) acc += xr[i] * wr[i];
            if (bias) acc += bias[o];
            yr[o] = act == 1 ? orc_gelu_tanh(acc) : acc;
        }
    }
}

void orc_linear(const float *x, size_t x_row, size_t rows, const float *w,
                size_t n, size_t k, const float *bias, int act, float *y,
                size_t y_row, int nthreads) { /* crates/lightx2v-cpu/src/lib.rs:296-326 */
#ifdef _OPENMP
    if (nthreads > 1) {
        long nr = (long)rows;
#pragma omp parallel for num_threads(nthreads) schedule(static)
        for (long r = 0; r < nr; r++)
            linear_rows(x, x_row, (size_t)r, (size_t)r + 1, w, n, k, bias, act, y, y_row);
        return;
    }
#endif
    (void)nthreads;
    linear_rows(x, x_row, 0, rows, w, n, k, bias, act, y, y_row);
}

void orc_linear_f64(const float *x, size_t rows, const float *w, size_t n,
                    size_t k, const float *bias, double *y) {
    for (size_t r = 0; r < rows; r++)
        for (size_t o = 0; o < n; o++) {
            double acc = 0.0;
            for (size_t i = 0; i < k; i++) acc += (double)x[r * k + i] * (double)w[o * k + i];
            if (bias) acc += (double)bias[o];
            y[r * n + o] = acc;
        }
}

/* ---- norms around the linears ---------------------------------------------- */

void orc_layer_norm(const float *x, size_t rows, size_t dim, int kind, const float *w,
                    const float *b, const float *mods, size_t scale, size_t shift, float eps,
                    float *out) { /* crates/lightx2v-cpu/src/lib.rs:328-361 */
    for (size_t r = 0; r < rows; r++) {
        const float *row = x + r * dim;
        float sum = 0.0f; /* Iterator::sum: a sequential fold */
        for (size_t j = 0; j < dim; j++) sum += row[j];
        const float mean = sum / (float)dim;
        float sq = 0.0f;
        for (size_t j = 0; j < dim; j++) {
            const float d = row[j] - mean;
            sq += d * d; /* powi(2) */
        }
        const float var = sq / (float)dim;
        const float inv = 1.0f / sqrtf(var + eps);
        for (size_t j = 0; j < dim; j++) {
            const float n = (row[j] - mean) * inv;
            out[r * dim + j] = kind == 0 ? n * w[j] + b[j]
                                         : n * (1.0f + mods[scale * dim + j]) + mods[shift * dim + j];
        }
    }
}

void orc_residual_norm(float *h, const float *a, size_t rows, size_t dim, const float *mods,
                       long gate, int kind, const float *w, const float *b, size_t scale,
                       size_t shift, float eps, float *normed) { /* lib.rs:363-388 */
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < dim; j++) {
            const float gv = gate >= 0 ? mods[(size_t)gate * dim + j] : 1.0f;
            h[r * dim + j] += a[r * dim + j] * gv;
        }
    orc_layer_norm(h, rows, dim, kind, w, b, mods, scale, shift, eps, normed);
}

void orc_gate_residual(float *h, const float *a, size_t rows, size_t dim, const float *mods,
                       size_t gate) { /* lib.rs:390-400 */
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < dim; j++) h[r * dim + j] += a[r * dim + j] * mods[gate * dim + j];
}

/* ---- head split ----------------------------------------------------------- */

/* crates/lightx2v-cpu/src/lib.rs:406-455: columns [col_off, col_off + heads*hd)
 * of each of `rows` rows (row stride src_stride) -> out [heads, rows, hd];
 * with rms_w: x * inv * w[j], inv = 1 / sqrt(mean(x^2) + eps), the mean a
 * sequential f32 fold of the squares; with cos / sin ([rows, hd/2]): each
 * head's interleaved pairs (2i, 2i+1) rotated, a*c - b*s and a*s + b*c.
 * The cos / sin index is r * (hd / 2) + i, the [rows, hd/2] layout that the
 * trait documents (core/src/backend.rs:258) and wgpu indexes
 * (shaders/head_split.wgsl:33,45). The CPU loop writes r * hd / 2 + i
 * (cpu/src/lib.rs:447), which is the same for every even hd and differs
 * for odd hd, where the trait's layout is the one followed. */
void orc_head_split(const float *src, size_t rows, size_t src_stride, size_t col_off, size_t heads, size_t hd,
                    const float *rms_w, const float *cos_t, const float *sin_t, float eps, float *out) {
    const size_t d = heads * hd;
    float *tmp = (float *)malloc(d * sizeof(float));
    for (size_t r = 0; r < rows; r++) {
        const float *row = src + r * src_stride + col_off;
        if (rms_w) {
            float ss = 0.0f;
            for (size_t j = 0; j < d; j++) ss += row[j] * row[j];
            const float ms = ss / (float)d;
            const float inv = 1.0f / sqrtf(ms + eps);
            for (size_t j = 0; j < d; j++) tmp[j] = row[j] * inv * rms_w[j];
        } else {
            for (size_t j = 0; j < d; j++) tmp[j] = row[j];
        }
        if (cos_t && sin_t) {
            for (size_t h = 0; h < heads; h++)
                for (size_t i = 0; i < hd / 2; i++) {
                    const float a = tmp[h * hd + 2 * i], b = tmp[h * hd + 2 * i + 1];
                    const float c = cos_t[r * (hd / 2) + i], s = sin_t[r * (hd / 2) + i];
                    tmp[h * hd + 2 * i] = a * c - b * s;
                    tmp[h * hd + 2 * i + 1] = a * s + b * c;
                }
        }
        for (size_t h = 0; h < heads; h++)
            for (size_t j = 0; j < hd; j++) out[(h * rows + r) * hd + j] = tmp[h * hd + j];
    }
    free(tmp);
}

/* The same in f64 throughout (test pin: the f32 restatement must sit
 * within f32 rounding of it). */
void orc_head_split_f64(const float *src, size_t rows, size_t src_stride, size_t col_off, size_t heads, size_t hd,
                        const float *rms_w, const float *cos_t, const float *sin_t, float eps, double *out) {
    const size_t d = heads * hd;
    double *tmp = (double *)malloc(d * sizeof(double));
    for (size_t r = 0; r < rows; r++) {
        const float *row = src + r * src_stride + col_off;
        double inv = 1.0;
        if (rms_w) {
            double ss = 0.0;
            for (size_t j = 0; j < d; j++) ss += (double)row[j] * row[j];
            inv = 1.0 / sqrt(ss / (double)d + (double)eps);
        }
        for (size_t j = 0; j < d; j++) tmp[j] = rms_w ? (double)row[j] * inv * rms_w[j] : (double)row[j];
        if (cos_t && sin_t) {
            for (size_t h = 0; h < heads; h++)
                for (size_t i = 0; i < hd / 2; i++) {
                    const double a = tmp[h * hd + 2 * i], b = tmp[h * hd + 2 * i + 1];
                    const double c = cos_t[r * (hd / 2) + i], s = sin_t[r * (hd / 2) + i];
                    tmp[h * hd + 2 * i] = a * c - b * s;
                    tmp[h * hd + 2 * i + 1] = a * s + b * c;
                }
        }
        for (size_t h = 0; h < heads; h++)
            for (size_t j = 0; j < hd; j++) out[(h * rows + r) * hd + j] = tmp[h * hd + j];
    }
    free(tmp);
}

/* ---- attention ------------------------------------------------------------ */

static void attention_row(const float *q, const float *k, const float *v, size_t heads, size_t sq,
                          size_t sk, size_t d, const uint8_t *mask, float *out, size_t h,
                          size_t qi, float *scores) { /* lib.rs:171-203, one (head, query) */
    const float scale = 1.0f / sqrtf((float)d);
    for (size_t ki = 0; ki < sk; ki++) {
        if (mask && !mask[qi * sk + ki]) {
            scores[ki] = -INFINITY;
            continue;
        }
        float s = 0.0f;
        for (size_t j = 0; j < d; j++) s += q[(h * sq + qi) * d + j] * k[(h * sk + ki) * d + j];
        scores[ki] = s * scale;
    }
    /* softmax_row, lib.rs:155-166 */
    float m = -INFINITY;
    for (size_t ki = 0; ki < sk; ki++) m = fmaxf(m, scores[ki]); /* f32::max ignores NaN */
    float sum = 0.0f;
    for (size_t ki = 0; ki < sk; ki++) {
        scores[ki] = expf(scores[ki] - m);
        sum += scores[ki];
    }
    const float inv = 1.0f / sum;
    for (size_t ki = 0; ki < sk; ki++) scores[ki] *= inv;
    for (size_t j = 0; j < d; j++) {
        float acc = 0.0f;
        for (size_t ki = 0; ki < sk; ki++) acc += scores[ki] * v[(h * sk + ki) * d + j];
        out[(qi * heads + h) * d + j] = acc;
    }
}

void orc_attention(const float *q, const float *k, const float *v, size_t heads, size_t sq,
                   size_t sk, size_t d, const uint8_t *mask, float *out, int nthreads) {
    const long rows = (long)(heads * sq);
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads > 1 ? nthreads : 1)
#endif
    {
        float *scores = (float *)malloc((sk ? sk : 1) * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (long r = 0; r < rows; r++)
            attention_row(q, k, v, heads, sq, sk, d, mask, out, (size_t)r / sq, (size_t)r % sq, scores);
        free(scores);
    }
    (void)nthreads;
}

/* ---- activation quantization (build-defined) ----------------------------- */

void orc_act_quant_e4m3(const float *x, size_t rows, size_t cols, uint8_t *q,
                        float *s) {
    for (size_t r = 0; r < rows; r++) {
        const float *xr = x + r * cols;
        float amax = 0.0f;
        for (size_t c = 0; c < cols; c++) amax = fmaxf(amax, fabsf(xr[c]));
        float inv = 1.0f, sc = 1.0f;
        if (amax > 0x1p-64f) {
            inv = 448.0f / amax;
            sc = amax / 448.0f;
        }
        for (size_t c = 0; c < cols; c++) {
            float t = xr[c] * inv;
            t = fminf(fmaxf(t, -448.0f), 448.0f);
            q[r * cols + c] = orc_f32_to_e4m3_ocp_rne(t);
        }
        s[r] = sc;
    }
}

/* Build-defined MX e4m3 quantization (the FFN hand-off format): per block of
 * 32 consecutive columns of a row, the power-of-two scale 2^k with k the
 * smallest integer such that amax * 2^-k <= 448, clamped to [-127, 127],
 * where amax = max |v| of the block; codes = OCP e4m3 RNE of clamp(v * 2^-k,
 * +-448).  k comes from amax's bits (no division): amax = 1.m * 2^(E-127)
 * lies in (448 * 2^(k-1), 448 * 2^k] exactly when k = E - 135 + [1.m > 1.75].
 * Scales are stored as E8M0 bytes k + 127, block-major: s[(c/32) * rows + r].
 * Value of a code: e4m3 * 2^k. */
int orc_mx_exponent(float amax) {
    uint32_t b;
    memcpy(&b, &amax, 4);
    b &= 0x7FFFFFFFu;
    int e = (int)(b >> 23);
    int k = e - 135 + ((b & 0x7FFFFFu) > 0x600000u ? 1 : 0);
    return k < -127 ? -127 : (k > 127 ? 127 : k);
}

void orc_act_quant_mx(const float *x, size_t rows, size_t cols, uint8_t *q, uint8_t *s) {
    for (size_t r = 0; r < rows; r++) {
        for (size_t b = 0; b < cols / 32; b++) {
            const float *v = x + r * cols + b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
            int k = orc_mx_exponent(amax);
            float inv = ldexpf(1.0f, -k);
            for (int i = 0; i < 32; i++) {
                float t = fminf(fmaxf(v[i] * inv, -448.0f), 448.0f);
                q[r * cols + b * 32 + i] = orc_f32_to_e4m3_ocp_rne(t);
            }
            s[b * rows + r] = (uint8_t)(k + 127);
        }
    }
}

void orc_dequant_mx(const uint8_t *q, const uint8_t *s, size_t rows, size_t cols, float *out) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++)
            out[r * cols + c] = ldexpf(orc_e4m3_to_f32_ocp(q[r * cols + c]), (int)s[(c / 32) * rows + r] - 127);
}

/* ---- element-wise maps over arrays (for large test inputs) ------------------- */

void orc_map_e4m3_ref(const float *v, size_t n, uint8_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_e4m3_ref(v[i]);
}
void orc_map_e4m3_canon(const float *v, size_t n, uint8_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_e4m3_canon(v[i]);
}
void orc_map_e4m3_ocp(const float *v, size_t n, uint8_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_e4m3_ocp_rne(v[i]);
}
void orc_map_decode_ref(const uint8_t *c, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_e4m3_to_f32_ref(c[i]);
}
void orc_map_decode_ocp(const uint8_t *c, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_e4m3_to_f32_ocp(c[i]);
}
void orc_map_gelu(const float *x, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_gelu_tanh(x[i]);
}
void orc_map_f16_round(const float *x, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_round(x[i]);
}

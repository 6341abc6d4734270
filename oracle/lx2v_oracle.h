/*
 * lx2v_oracle.h -- CPU restatement of lightx2v-rs's quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library under
 * lightx2v-rs_amd/) links, loads or calls this code.  Only tests/, the
 * smoke() check in __graft_entry__.py and the cpu_baseline leg of bench.py
 * use it, and only as the checker / the timed CPU baseline.
 *
 * Every function names the reference file:line it restates (paths relative
 * to the lightx2v-rs repository root).  Arithmetic follows Rust semantics:
 * f32 ops are IEEE single with no contraction (build with
 * -ffp-contract=off), `round` is half-away-from-zero (roundf), float->int
 * `as` casts saturate (NaN -> 0), int->u8 `as` casts wrap, `u8 << 3` drops
 * the high bits, and libm calls are glibc's (log2f, logf, tanhf, powf,
 * sinf, cosf), exactly as the reference binary on Linux calls them.
 */
#ifndef LX2V_ORACLE_H
#define LX2V_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Rng: crates/lightx2v-core/src/rng.rs:8-54 ------------------------ */
typedef struct { uint64_t state; } orc_rng;
void     orc_rng_new(orc_rng *r, uint64_t seed);              /* rng.rs:13-18 */
uint64_t orc_rng_next_u64(orc_rng *r);                         /* rng.rs:20-27 */
float    orc_rng_next_f32(orc_rng *r);                         /* rng.rs:29-31 */
void     orc_rng_uniform(orc_rng *r, float *out, size_t n, float a);  /* rng.rs:34-36 */
void     orc_rng_normal(orc_rng *r, float *out, size_t n);     /* rng.rs:39-54 */

/* ---- scalar codecs ----------------------------------------------------- */
/* quant.rs:376-406, verbatim including the e in {-9,-8,-7} wrap quirk. */
uint8_t orc_f32_to_e4m3_ref(float v);
/* quant.rs:409-420, verbatim: exponent field 0 decodes m * 2^-12. */
float   orc_e4m3_to_f32_ref(uint8_t code);
/* Build-defined weight encoder: quant.rs:376-406 for |v| >= 2^-6 (where
 * its result does not depend on how log2f rounds), 0x08 (2^-6) for
 * 2^-7 < |v| < 2^-6, signed zero for |v| <= 2^-7.  Never emits an
 * exponent-0 (subnormal) or NaN code, so on every code it emits the
 * reference decoder (quant.rs:409-420) and the OCP e4m3fn decoder agree. */
uint8_t orc_f32_to_e4m3_canon(float v);
/* OCP OFP8 e4m3fn decode (subnormals m * 2^-9, 0x7F/0xFF NaN). */
float   orc_e4m3_to_f32_ocp(uint8_t code);
/* OCP e4m3fn encode, round-to-nearest-even, input already clamped to
 * [-448, 448] by the caller (NaN -> 0x7F). */
uint8_t orc_f32_to_e4m3_ocp_rne(float v);
/* IEEE binary16 round-to-nearest-even and back (half 2.7.1 f16::from_f32,
 * used by quant.rs:280). */
float   orc_f16_round(float v);
uint16_t orc_f32_to_f16_bits(float v);
/* bfloat16 round-to-nearest-even and back (NaN kept quiet). */
float   orc_bf16_round(float v);
uint16_t orc_f32_to_bf16_bits(float v);
/* crates/lightx2v-cpu/src/lib.rs:151-153 */
float   orc_gelu_tanh(float x);

/* ---- Q8: quant.rs:142-205 --------------------------------------------- */
/* quant.rs:154-178 with the group as a parameter (the reference picks 128
 * when it divides cols, else cols; pass that to reproduce it exactly). */
void orc_q8_quantize(const float *data, size_t rows, size_t cols, size_t group,
                     int8_t *q, float *scales);
/* quant.rs:180-186 */
void orc_q8_dequantize(const int8_t *q, const float *scales, size_t rows,
                       size_t cols, size_t group, float *out);
size_t orc_q8_ref_group(size_t cols);                          /* quant.rs:156-160 */

/* ---- Q4: quant.rs:207-356 --------------------------------------------- */
/* quant.rs:226-292 (min/max RTN, optional HQQ zero refinement, f16-rounded
 * scale and zero).  `group` must already be the effective group
 * (quant.rs:228-232: the requested group if it divides cols, else cols). */
void orc_q4_quantize(const float *data, size_t rows, size_t cols, size_t group,
                     int hqq, uint8_t *codes, float *scales, float *zeros);
/* Build-defined symmetric 4-bit layout of the benchmark (values -8..7 with
 * an f32 scale absmax/7 per group), expressed in the reference's Q4 type:
 * code = q + 8, zero = 8.0, scale = s, so (code - zero) * scale == q * s. */
void orc_q4_quantize_sym(const float *data, size_t rows, size_t cols, size_t group,
                         uint8_t *codes, float *scales, float *zeros);
/* quant.rs:294-303 */
void orc_q4_dequantize(const uint8_t *codes, const float *scales, const float *zeros,
                       size_t rows, size_t cols, size_t group, float *out);
/* quant.rs:306-311: two codes per byte, element 2i in the low nibble. */
void orc_q4_pack(const uint8_t *codes, size_t n, uint8_t *packed);
/* quant.rs:313-336 (codes only). */
void orc_q4_unpack(const uint8_t *packed, size_t n, uint8_t *codes);

/* ---- FP8: quant.rs:358-460 -------------------------------------------- */
/* quant.rs:423-447 with the group as a parameter; canon=0 uses
 * orc_f32_to_e4m3_ref, canon=1 uses orc_f32_to_e4m3_canon. */
void orc_fp8_quantize(const float *data, size_t rows, size_t cols, size_t group,
                      int canon, uint8_t *q, float *scales);
/* quant.rs:449-455 */
void orc_fp8_dequantize(const uint8_t *q, const float *scales, size_t rows,
                        size_t cols, size_t group, float *out);
size_t orc_fp8_ref_group(size_t cols);                         /* quant.rs:425-429 */

/* ---- linear: crates/lightx2v-cpu/src/lib.rs:296-326 --------------------- */
/* y[(y_row+r)*N + o] = act(sum_i x[(x_row+r)*K + i] * w[o*K + i] + b[o]),
 * sequential f32 accumulation, mul then add.  act: 0 none, 1 gelu_tanh.
 * nthreads <= 1 runs the reference's single thread; > 1 splits rows over
 * OpenMP threads with the same per-element operation order (bit-identical). */
void orc_linear(const float *x, size_t x_row, size_t rows, const float *w,
                size_t n, size_t k, const float *bias, int act, float *y,
                size_t y_row, int nthreads);
/* f64 brute force of the same sum (for pinning the f32 loop on small
 * shapes). */
void orc_linear_f64(const float *x, size_t rows, const float *w, size_t n,
                    size_t k, const float *bias, double *y);

/* ---- build-defined activation quantization (no reference counterpart) --- */
/* Per row: amax = max|x|; inv = 448/amax, s = amax/448 (amax == 0: inv = s =
 * 1); q = OCP-e4m3-RNE(clamp(x * inv, -448, 448)).  Dequantized value is
 * e4m3_ocp(q) * s. */
void orc_act_quant_e4m3(const float *x, size_t rows, size_t cols, uint8_t *q,
                        float *s);

/* ---- norms around the linears: crates/lightx2v-cpu/src/lib.rs:328-400 ----- */
/* NormKind (backend.rs:47-52): kind 0 = Affine, LN(x) * w[j] + b[j];
 * kind 1 = Mod, LN(x) * (1 + mods[scale*dim + j]) + mods[shift*dim + j].
 * mean and variance are the reference's sequential f32 sums. */
void orc_layer_norm(const float *x, size_t rows, size_t dim, int kind, const float *w,
                    const float *b, const float *mods, size_t scale, size_t shift, float eps,
                    float *out);                                      /* lib.rs:328-361 */
/* h += a * (gate >= 0 ? mods[gate*dim + j] : 1), then normed = norm(h). */
void orc_residual_norm(float *h, const float *a, size_t rows, size_t dim, const float *mods,
                       long gate, int kind, const float *w, const float *b, size_t scale,
                       size_t shift, float eps, float *normed);       /* lib.rs:363-388 */
/* h += a * mods[gate*dim + j]. */
void orc_head_split(const float *src, size_t rows, size_t src_stride, size_t col_off, size_t heads, size_t hd,
                    const float *rms_w, const float *cos_t, const float *sin_t, float eps, float *out);
void orc_head_split_f64(const float *src, size_t rows, size_t src_stride, size_t col_off, size_t heads, size_t hd,
                        const float *rms_w, const float *cos_t, const float *sin_t, float eps, double *out);
void orc_gate_residual(float *h, const float *a, size_t rows, size_t dim, const float *mods,
                       size_t gate);                                  /* lib.rs:390-400 */

/* ---- attention: crates/lightx2v-cpu/src/lib.rs:155-203 -------------------- */
/* q [heads, sq, d], k / v [heads, sk, d]; mask [sq, sk] (1 = allowed) or
 * NULL; out [sq, heads*d].  scores = (q.k sequential f32) * (1/sqrtf(d)),
 * forbidden pairs -inf; softmax_row: max fold, expf(s - m), sequential sum,
 * multiply by 1/sum; out = sequential sum over keys of p * v.  nthreads > 1
 * splits (head, query) rows over OpenMP threads, same per-row order. */
void orc_attention(const float *q, const float *k, const float *v, size_t heads, size_t sq,
                   size_t sk, size_t d, const uint8_t *mask, float *out, int nthreads);

/* ---- element-wise maps of the scalar functions above over arrays ---------- */
void orc_map_e4m3_ref(const float *v, size_t n, uint8_t *out);
void orc_map_e4m3_canon(const float *v, size_t n, uint8_t *out);
void orc_map_e4m3_ocp(const float *v, size_t n, uint8_t *out);
void orc_map_decode_ref(const uint8_t *c, size_t n, float *out);
void orc_map_decode_ocp(const uint8_t *c, size_t n, float *out);
void orc_map_gelu(const float *x, size_t n, float *out);
void orc_map_f16_round(const float *x, size_t n, float *out);

#ifdef __cplusplus
}
#endif
#endif

/*
 * lightx2v_hip.h -- C ABI of the MI355X (gfx950) quantized-linear backend.
 *
 * This is the drop-in boundary a `lightx2v-hip` crate binds to implement the
 * lightx2v-rs `Backend` trait's linear path (crates/lightx2v-core/src/
 * backend.rs:145-212).  Every entry point names the trait method it replaces.
 * Plain pointers and sizes only; no torch, no C++ types.
 *
 * Conventions
 *  - Every function returns an int status (LX2V_OK == 0).  On failure the
 *    thread-local message from lx2v_hip_last_error() says why.  The trait's
 *    methods are infallible and panic on misuse; a binding maps a non-zero
 *    status to `panic!` with that message, except lx2v_hip_create's
 *    LX2V_ERR_NO_DEVICE, which maps to `try_new() -> None` (the CLI's
 *    `skip:` path, crates/lightx2v-cli/src/main.rs:199-236).
 *  - Host-facing data is f32, as the trait's (backend.rs:9-11).  Device
 *    buffers hold f32 or bf16 activations (the backend's own precision):
 *    upload/download/write convert at the boundary.
 *  - One context = one device + one HIP stream.  Every op is stream-ordered
 *    and asynchronous except download (blocking) and the create/free calls.
 *    A context is used by one thread at a time (the reference CPU backend is
 *    !Send, crates/lightx2v-cpu/src/lib.rs:107-124).
 *  - Weights are copied into HBM during the weight_* call in the reference's
 *    packed byte layouts; the caller keeps ownership of host memory
 *    (backend.rs:178-188; crates/lightx2v-cpu/src/lib.rs:249-284).
 */
#ifndef LIGHTX2V_HIP_H
#define LIGHTX2V_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LX2V_HIP_ABI_VERSION 3

typedef struct lx2v_hip_ctx lx2v_hip_ctx;
typedef struct lx2v_hip_buf lx2v_hip_buf;
typedef struct lx2v_hip_weight lx2v_hip_weight;

/* status codes */
enum {
    LX2V_OK = 0,
    LX2V_ERR_NO_DEVICE = 1,   /* no usable gfx950 device: the `skip:` path  */
    LX2V_ERR_BAD_SHAPE = 2,   /* sizes/offsets out of range or inconsistent */
    LX2V_ERR_ALIAS = 3,       /* output overlaps an input (backend.rs:13-14) */
    LX2V_ERR_HIP = 4,         /* a HIP runtime call failed                  */
    LX2V_ERR_BAD_ARG = 5,     /* null handle, unknown enum value            */
    LX2V_ERR_OOM = 6,         /* device allocation failed                   */
    LX2V_ERR_UNSUPPORTED = 7, /* valid request this build does not serve    */
    LX2V_ERR_BUSY = 8         /* the device scratch is held by another context
                                 (lx2v_hip_linear_noalloc; no reference
                                 counterpart)                               */
};

/* Act (backend.rs:38-43) */
enum { LX2V_ACT_NONE = 0, LX2V_ACT_GELU_TANH = 1 };

/* device activation dtypes.  E4M3 buffers hold per-token quantized
 * activations (e4m3 codes [rows, cols] plus one f32 scale per row, value =
 * code * scale) and are made only by lx2v_hip_alloc_e4m3.  MXE4M3 buffers
 * hold MX-scaled e4m3 activations (codes [rows, cols] plus one power-of-two
 * scale per 32 columns of a row, value = code * 2^k) and are made only by
 * lx2v_hip_alloc_mx. */
enum { LX2V_DTYPE_F32 = 0, LX2V_DTYPE_BF16 = 1, LX2V_DTYPE_E4M3 = 2, LX2V_DTYPE_MXE4M3 = 3 };

/* weight formats (quant.rs:134-140 plus the native f32 matrix) */
enum { LX2V_WFMT_F32 = 0, LX2V_WFMT_Q8 = 1, LX2V_WFMT_Q4 = 2, LX2V_WFMT_FP8 = 3 };

/* How linear contracts an FP8 weight (no reference counterpart: the
 * reference has no activation quantization, backend.rs:9-11).
 *  FP8_ACT_E4M3: per-token dynamic e4m3 activations, fp8 MFMA (default);
 *  FP8_ACT_BF16: bf16 activations, weights dequantized to bf16, bf16 MFMA. */
enum { LX2V_FP8_ACT_E4M3 = 0, LX2V_FP8_ACT_BF16 = 1 };

/* How linear contracts a native f32 weight (lx2v_hip_weight_f32).
 *  NATIVE_BF16: the weight's bf16 copy (RNE, made at upload) times bf16
 *    activations on the bf16 MFMA, f32 accumulation -- for cols % 64 == 0
 *    (default).  Both operands are rounded to bf16 (8 significant bits,
 *    relative error up to 2^-9 each), which is looser than either reference
 *    backend: the CPU one is f32 throughout, and wgpu keeps f32 activations
 *    and rounds the weight to f16 (11 significant bits) only when every
 *    |w| <= 65000 (crates/lightx2v-wgpu/src/lib.rs:877-905, linear.wgsl:8).
 *    Measured against the f32 oracle: rel-L2 about 3e-3 per call.
 *  NATIVE_F32: f32 operands and f32 arithmetic (the scalar kernel), the CPU
 *    reference's own precision (crates/lightx2v-cpu/src/lib.rs:296-326);
 *    select it with lx2v_hip_set_native_mode where that precision matters. */
enum { LX2V_NATIVE_BF16 = 0, LX2V_NATIVE_F32 = 1 };

/* ---- errors / context --------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). */
const char *lx2v_hip_last_error(void);

/* Number of visible HIP devices (0 on a host without a GPU; never fails). */
int lx2v_hip_device_count(int *count);

/* WgpuBackend::try_new (crates/lightx2v-wgpu/src/lib.rs:282-287): create a
 * context on `device`.  LX2V_ERR_NO_DEVICE when no usable gfx950 device. */
int lx2v_hip_create(int device, lx2v_hip_ctx **out);
int lx2v_hip_destroy(lx2v_hip_ctx *ctx);

/* Backend::name (backend.rs:158): "hip:<device name> (gfx950)". */
int lx2v_hip_name(const lx2v_hip_ctx *ctx, char *out, size_t cap);

/* dtype of buffers created by lx2v_hip_alloc / lx2v_hip_upload from now on
 * (default LX2V_DTYPE_F32). */
int lx2v_hip_set_act_dtype(lx2v_hip_ctx *ctx, int dtype);
/* LX2V_FP8_ACT_* used by lx2v_hip_linear for FP8 weights. */
int lx2v_hip_set_fp8_act(lx2v_hip_ctx *ctx, int mode);
/* LX2V_NATIVE_* used by lx2v_hip_linear for native f32 weights (no
 * reference counterpart: the reference picks its precision per backend). */
int lx2v_hip_set_native_mode(lx2v_hip_ctx *ctx, int mode);

/* ---- buffers (backend.rs:160-177) -------------------------------------- */

/* Backend::alloc (backend.rs:161-162): zero-filled, `len` elements. */
int lx2v_hip_alloc(lx2v_hip_ctx *ctx, size_t len, lx2v_hip_buf **out);
int lx2v_hip_alloc_dtype(lx2v_hip_ctx *ctx, size_t len, int dtype, lx2v_hip_buf **out);
/* Backend::upload (backend.rs:163). */
int lx2v_hip_upload(lx2v_hip_ctx *ctx, const float *data, size_t len, lx2v_hip_buf **out);
/* Backend::write (backend.rs:171-172): overwrite the first `len` elements. */
int lx2v_hip_write(lx2v_hip_ctx *ctx, lx2v_hip_buf *buf, const float *data, size_t len);
/* Backend::download (backend.rs:173-174): blocking; `len` == buffer length. */
int lx2v_hip_download(lx2v_hip_ctx *ctx, const lx2v_hip_buf *buf, float *out, size_t len);
/* Backend::buf_len (backend.rs:175). */
int lx2v_hip_buf_len(const lx2v_hip_buf *buf, size_t *len);
int lx2v_hip_buf_dtype(const lx2v_hip_buf *buf, int *dtype);
/* Backend::copy (backend.rs:176-177): dst[dst_off..][..len] = src[src_off..][..len]. */
int lx2v_hip_copy(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t src_off,
                  lx2v_hip_buf *dst, size_t dst_off, size_t len);
/* Drop of the trait's Buf. */
int lx2v_hip_buf_free(lx2v_hip_ctx *ctx, lx2v_hip_buf *buf);

/* ---- weights (backend.rs:178-188) -------------------------------------- */

/* Backend::weight (backend.rs:178): native f32 [rows, cols] row-major.
 * With cols % 64 == 0 the weight also keeps a bf16 copy (2 bytes per
 * element) for the bf16 MFMA (LX2V_NATIVE_BF16). */
int lx2v_hip_weight_f32(lx2v_hip_ctx *ctx, const float *data, size_t rows, size_t cols,
                        lx2v_hip_weight **out);
/* Backend::weight_q8 (backend.rs:179-182) over quant.rs:142-151's Q8:
 * q int8 [rows, cols], scales f32 [rows, cols/group]. */
int lx2v_hip_weight_q8(lx2v_hip_ctx *ctx, const int8_t *q, const float *scales,
                       size_t rows, size_t cols, size_t group, lx2v_hip_weight **out);
/* Backend::weight_q4 (backend.rs:183-185) over quant.rs:207-220's Q4:
 * codes 0..15, one per byte (packed == 0, the Q4 struct's `q`) or two per
 * byte with element 2i in the low nibble (packed == 1, Q4::packed,
 * quant.rs:305-311); scales and zeros f32 [rows, cols/group];
 * dequantized value (code - zero) * scale (quant.rs:294-303). */
int lx2v_hip_weight_q4(lx2v_hip_ctx *ctx, const uint8_t *codes, int packed,
                       const float *scales, const float *zeros, size_t rows,
                       size_t cols, size_t group, lx2v_hip_weight **out);
/* Backend::weight_fp8 (backend.rs:186-188) over quant.rs:364-373's Fp8E4M3:
 * e4m3 codes [rows, cols], scales f32 [rows, cols/group] (group == cols is
 * the per-output-channel case).  Codes with exponent field 0 and a non-zero
 * mantissa (reference value m * 2^-12 * s, at most 3.9e-6 * the group's
 * absmax) are stored as signed zero so the fp8 MFMA, which decodes OCP
 * e4m3fn, sees the reference value of every other code exactly; the count
 * is reported by lx2v_hip_weight_info.  Group 128 (cols % 128 == 0): the
 * fp8 MFMA kernels apply the group scales by rescaling their running sums
 * by s[g-1] / s[g] at each group boundary, from a ratio table built here
 * (a copy of the scales to the host and back); a weight with a scale that
 * is zero, negative or not finite, or with two groups of a channel more
 * than 2^60 apart, runs on the bf16 MFMA kernel instead. */
int lx2v_hip_weight_fp8(lx2v_hip_ctx *ctx, const uint8_t *q, const float *scales,
                        size_t rows, size_t cols, size_t group, lx2v_hip_weight **out);
/* Drop of the trait's Weight. */
int lx2v_hip_weight_free(lx2v_hip_ctx *ctx, lx2v_hip_weight *w);

typedef struct {
    int fmt;            /* LX2V_WFMT_* */
    size_t rows, cols, group;
    size_t device_bytes;  /* codes, scales (and zeros), the bf16 GEMM's
                             stage-major copy of the scales, and FP8 group
                             128's ratio table and last-group scales */
    size_t canonicalized; /* FP8 exponent-0 codes stored as zero */
} lx2v_hip_weight_info_t;
int lx2v_hip_weight_info(const lx2v_hip_weight *w, lx2v_hip_weight_info_t *info);

/* Test hook, no trait counterpart: the weight as the device decodes it
 * (the decode the GEMMs use), f32 [rows, cols] into host memory.  For every
 * format this equals the reference's dequantize() bit for bit
 * (quant.rs:180-186, 294-303, 449-455); for FP8 the reference decode of
 * the codes as passed in (exponent-0 codes included). */
int lx2v_hip_weight_dequantize(lx2v_hip_ctx *ctx, const lx2v_hip_weight *w, float *out,
                               size_t len);

/* ---- device-side quantizers (reference runs these on the host) ---------- */

/* Q8::quantize (quant.rs:154-178) of the f32 matrix in `src` (f32 buffer),
 * group given explicitly (the reference uses 128 when it divides cols). */
int lx2v_hip_quantize_q8(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows,
                         size_t cols, size_t group, lx2v_hip_weight **out);
/* Symmetric 4-bit in the Q4 layout: s = absmax/7, q = clamp(round(v/s),-8,7),
 * code = q + 8, zero = 8 (the HQQ path of quant.rs:226-292 stays on host). */
int lx2v_hip_quantize_q4_sym(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows,
                             size_t cols, size_t group, lx2v_hip_weight **out);
/* Fp8E4M3::quantize (quant.rs:423-447) with the canonical encoder:
 * quant.rs:376-406 for |v/s| >= 2^-6, 0x08 (2^-6) for 2^-7 < |v/s| < 2^-6,
 * signed zero below; never emits an exponent-0 or NaN code. */
int lx2v_hip_quantize_fp8(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows,
                          size_t cols, size_t group, lx2v_hip_weight **out);

/* Q4::quantize (quant.rs:226-292) with the reference's arithmetic: affine
 * min/max codes, with hqq != 0 the HQQ-refined zero point (quant.rs:248-276),
 * scale 1/is and zero rounded to f16 as stored (quant.rs:280-281); codes
 * packed two per byte, element 2i in the low nibble.  The group must be even
 * and divide cols (the caller applies the reference's fallback to cols,
 * quant.rs:227-231).  HQQ's powf is taken in double: glibc's powf differs
 * from that in the last ulp for ~0.06% of arguments. */
int lx2v_hip_quantize_q4(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows,
                         size_t cols, size_t group, int hqq, lx2v_hip_weight **out);
/* Fp8E4M3::quantize (quant.rs:423-447) with f32_to_e4m3 (quant.rs:376-406)
 * verbatim, exponent wrap included: the weight then holds exactly what
 * weight_fp8 would hold for the reference's Fp8E4M3 (codes canonicalized
 * for the MFMA, the reference bytes kept for dequantize / export). */
int lx2v_hip_quantize_fp8_ref(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows,
                              size_t cols, size_t group, lx2v_hip_weight **out);
/* Read a weight back in the reference's layouts (no reference counterpart:
 * the host struct a Backend::weight_* call consumed, for writing a
 * quantized checkpoint, export.rs:44-130): codes_bytes = rows*cols (Q8 i8,
 * FP8 the reference bytes), rows*cols/2 rounded up (Q4 packed) or
 * 4*rows*cols (F32 values); scales [rows * cols/group] f32 (not for F32);
 * zeros likewise, Q4 only. */
int lx2v_hip_weight_export(lx2v_hip_ctx *ctx, const lx2v_hip_weight *w, void *codes,
                           size_t codes_bytes, float *scales, float *zeros);

/* ---- the norms and residuals around the linears ---------------------------
 * Backend::layer_norm / residual_norm / gate_residual (backend.rs:214-256,
 * CPU reference crates/lightx2v-cpu/src/lib.rs:328-400): the producers of the
 * block linears' inputs and the consumer of their outputs.  NormKind
 * (backend.rs:47-52): AFFINE is LN(x) * w + b, MOD is LN(x) * (1 +
 * mods[scale]) + mods[shift] over rows of `mods` ([slots, dim]).
 * Extension: `out` / `normed` may be an E4M3 buffer (lx2v_hip_alloc_e4m3,
 * cols == dim) or an MXE4M3 buffer (lx2v_hip_alloc_mx): the norm then writes
 * the quantized activations an FP8 linear contracts, in the same pass (no
 * separate quantize_act).  Mean and variance are summed across lanes, not
 * sequentially. */
enum { LX2V_NORM_AFFINE = 0, LX2V_NORM_MOD = 1 };
typedef struct {
    int kind;                     /* LX2V_NORM_AFFINE or LX2V_NORM_MOD */
    const lx2v_hip_buf *w, *b;    /* AFFINE: [dim] each */
    size_t scale, shift;          /* MOD: rows of mods */
} lx2v_hip_norm_t;
/* out = norm(x) over rows of width dim (backend.rs:214-225). */
int lx2v_hip_layer_norm(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t rows, size_t dim,
                        const lx2v_hip_norm_t *norm, const lx2v_hip_buf *mods, float eps,
                        lx2v_hip_buf *out);
/* In place on h: h += a * mods[gate] (has_gate) or h += a, then normed =
 * norm(h), the norm reading the unrounded sum (backend.rs:227-241). */
int lx2v_hip_residual_norm(lx2v_hip_ctx *ctx, lx2v_hip_buf *h, const lx2v_hip_buf *a, size_t rows,
                           size_t dim, const lx2v_hip_buf *mods, int has_gate, size_t gate,
                           const lx2v_hip_norm_t *norm, float eps, lx2v_hip_buf *normed);
/* linear followed by gate_residual in one call: h[h_row + r] += act(x W^T +
 * b)[r] * mods[gate] for r < rows (no reference counterpart: dit.rs runs
 * `linear` into a temporary, then `gate_residual`, after the attention O,
 * cross-attention O and FFN-down projections).  Results equal that pair's
 * with the temporary in h's dtype, bit for bit.  On the FP8 e4m3 path the
 * add rides in the GEMM's epilogue (no temporary is written); elsewhere the
 * pair runs as two launches. */
int lx2v_hip_linear_residual(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows,
                             const lx2v_hip_weight *w, const lx2v_hip_buf *bias, int act, lx2v_hip_buf *h,
                             size_t h_row, const lx2v_hip_buf *mods, size_t gate);
/* In place on h: h += a * mods[gate] (backend.rs:243-252). */
int lx2v_hip_gate_residual(lx2v_hip_ctx *ctx, lx2v_hip_buf *h, const lx2v_hip_buf *a, size_t rows,
                           size_t dim, const lx2v_hip_buf *mods, size_t gate);

/* Backend::head_split (backend.rs:255-273; CPU lib.rs:406-455): columns
 * [col_off, col_off + heads*head_dim) of `rows` rows of width src_stride ->
 * out as [heads, rows, head_dim].  rms_w ([heads*head_dim], or NULL): RMS-
 * normalised across all heads first, x * (1 / sqrt(mean(x^2) + eps)) * w.
 * rope_cos / rope_sin ([rows, head_dim/2] each, both or neither): each
 * head's interleaved pairs (2i, 2i+1) rotated, (a c - b s, a s + b c).
 * src / out F32 or BF16 (out's dtype is the output's); rms_w and the tables
 * F32 or BF16.  out must not overlap src.  The mean of squares is a lane
 * reduction (the reference folds it sequentially: rel. 1e-7 differences);
 * every other operation rounds as the reference's. */
int lx2v_hip_head_split(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows, size_t src_stride, size_t col_off,
                        size_t heads, size_t head_dim, const lx2v_hip_buf *rms_w, const lx2v_hip_buf *rope_cos,
                        const lx2v_hip_buf *rope_sin, float eps, lx2v_hip_buf *out);

/* ---- attention (backend.rs:273-305) -----------------------------------------
 * q [heads, sq, head_dim], k / v [heads, sk, head_dim] (F32 or BF16, one
 * dtype); out [sq, heads*head_dim] (F32 or BF16), heads merged.  Scores
 * q.k / sqrt(head_dim), softmax over keys; masked pairs are -inf (a query
 * with no allowed key gives NaN, as the reference).  head_dim 64 and 128
 * run on the bf16 MFMA: q, k, v and the softmax weights P rounded to bf16,
 * f32 accumulation and softmax -- against the reference's f32 attention
 * (cpu/src/lib.rs:171-203) on the same f32 inputs, rel-L2 about 3e-3 and
 * max-abs about 5e-3 of the output's range (measured on gfx950 for sk 64 ..
 * 2048).  Other head_dim up to 256 run on a per-query kernel in f32
 * (rel-L2 <= 1e-5).
 * out may also be an MXE4M3 buffer (lx2v_hip_alloc_mx, cols == heads *
 * head_dim, rows >= sq; head_dim 64 or 128): the epilogue then writes the
 * MX quantization (lx2v_hip_alloc_mx's rule) of the f32 output, the
 * attention-O linear's input without a quantization pass (no reference
 * counterpart: the reference's attention writes f32); a query with no
 * allowed key keeps NaN codes.  Every entry point
 * below that takes `out` accepts it the same way.
 * Where heads * ceil(sq / 256) is at most half the GPU's CUs (head_dim 64 /
 * 128), each (head, 256-query) item runs as 2, 4 or 8 pieces over parts of
 * its keys whose partial sums a second pass merges; those pieces live in a
 * context workspace grown on first use (like linear's), so such a call,
 * like linear, must run once eagerly before graph capture.
 * LIGHTX2V_HIP_ATTN_SPLIT=0 in the environment turns this off. */
int lx2v_hip_attention(lx2v_hip_ctx *ctx, const lx2v_hip_buf *q, const lx2v_hip_buf *k,
                       const lx2v_hip_buf *v, size_t heads, size_t sq, size_t sk, size_t head_dim,
                       lx2v_hip_buf *out);
/* Backend::causal_attention: mask is the host's [sq, sk] bool array (one byte
 * per pair, nonzero = allowed) or NULL (= attention).  The mask is copied to
 * the device on every call and the call returns once the host array may be
 * reused; lx2v_hip_mask_upload + lx2v_hip_attention_masked keep a mask
 * resident instead. */
int lx2v_hip_causal_attention(lx2v_hip_ctx *ctx, const lx2v_hip_buf *q, const lx2v_hip_buf *k,
                              const lx2v_hip_buf *v, size_t heads, size_t sq, size_t sk,
                              size_t head_dim, const uint8_t *mask, lx2v_hip_buf *out);
/* A mask resident in HBM with its per-tile summary (no reference counterpart:
 * the reference passes the mask per call; the MemRoPE mask is the same for
 * every layer of a step). */
typedef struct lx2v_hip_mask lx2v_hip_mask;
int lx2v_hip_mask_upload(lx2v_hip_ctx *ctx, const uint8_t *mask, size_t sq, size_t sk,
                         lx2v_hip_mask **out);
/* The MemRoPE block mask built on the device from temporal indices: pair
 * (i, j) allowed iff tk[j] <= tq[i], the mask dit.rs:643-653 builds on the
 * host from the chunk's token temporal indices and kv_cache_temporal (no
 * reference counterpart: it replaces the [sq, sk] byte array's host build
 * and upload, 87.6 MB per step at the Wan shape, with 8 (sq + sk) bytes). */
int lx2v_hip_mask_temporal(lx2v_hip_ctx *ctx, const size_t *tq, size_t sq, const size_t *tk, size_t sk,
                           lx2v_hip_mask **out);
int lx2v_hip_mask_free(lx2v_hip_ctx *ctx, lx2v_hip_mask *mask);
int lx2v_hip_attention_masked(lx2v_hip_ctx *ctx, const lx2v_hip_buf *q, const lx2v_hip_buf *k,
                              const lx2v_hip_buf *v, size_t heads, size_t sq, size_t sk,
                              size_t head_dim, const lx2v_hip_mask *mask, lx2v_hip_buf *out);

/* ---- KV cache / MemRoPE (backend.rs:333-392) ---------------------------------
 * One layer's cache: K and V rows of [heads, head_dim] in HBM (the context's
 * activation dtype when the cache is made), with one temporal index and one
 * slot kind per row on the host, as the reference's KvCache
 * (crates/lightx2v-cpu/src/lib.rs:126-146).  K / V arguments are
 * [heads, rows, head_dim], F32 or BF16.  The cache grows past its capacity
 * as the reference's Vec does; growing, the update, kv and free are not
 * allowed during graph capture. */
typedef struct lx2v_hip_kv lx2v_hip_kv;
/* SlotKind (crates/lightx2v-core/src/memrope.rs:31-37) */
enum { LX2V_SLOT_SINK = 0, LX2V_SLOT_LONG_EMA = 1, LX2V_SLOT_SHORT_EMA = 2, LX2V_SLOT_RECENT = 3, LX2V_SLOT_NEW = 4 };
/* The MemRopeConfig fields the update reads (config.rs:265-278); the new
 * window is MemRopeConfig::new_frames() = 3 (config.rs:298-300). */
typedef struct {
    size_t cache_frames;
    size_t sink_frames;
    float ema_alpha_long;
    float ema_alpha_short;
} lx2v_hip_memrope_t;
/* kv_cache_new (backend.rs:333-335) */
int lx2v_hip_kv_cache_new(lx2v_hip_ctx *ctx, size_t heads, size_t head_dim, size_t capacity_tokens,
                          lx2v_hip_kv **out);
int lx2v_hip_kv_cache_free(lx2v_hip_ctx *ctx, lx2v_hip_kv *cache);
/* kv_cache_append (backend.rs:337-349): rows appended as New. */
int lx2v_hip_kv_cache_append(lx2v_hip_ctx *ctx, lx2v_hip_kv *cache, const lx2v_hip_buf *k, const lx2v_hip_buf *v,
                             size_t rows, const size_t *temporal);
/* kv_cache_put (backend.rs:351-366): overwrite the block's own rows when the
 * same temporal run is cached (EMA slots skipped), else append. */
int lx2v_hip_kv_cache_put(lx2v_hip_ctx *ctx, lx2v_hip_kv *cache, const lx2v_hip_buf *k, const lx2v_hip_buf *v,
                          size_t rows, const size_t *temporal);
/* kv_cache_len / kv_cache_temporal (backend.rs:368-372); kinds: the slot
 * kind per row (the reference's pub KvCache::kinds, lib.rs:138-139). */
int lx2v_hip_kv_cache_len(const lx2v_hip_kv *cache, size_t *rows);
int lx2v_hip_kv_cache_temporal(const lx2v_hip_kv *cache, size_t *out, size_t cap);
int lx2v_hip_kv_cache_kinds(const lx2v_hip_kv *cache, uint8_t *out, size_t cap);
/* kv_cache_kv (backend.rs:374-375): new [heads, rows, head_dim] buffers in
 * the cache's dtype.  _read writes into the caller's buffers instead. */
int lx2v_hip_kv_cache_kv(lx2v_hip_ctx *ctx, const lx2v_hip_kv *cache, lx2v_hip_buf **k, lx2v_hip_buf **v);
int lx2v_hip_kv_cache_read(lx2v_hip_ctx *ctx, const lx2v_hip_kv *cache, lx2v_hip_buf *k, lx2v_hip_buf *v);
/* kv_cache_memrope_update (backend.rs:377-387): seed the zero EMA frames,
 * graduate New -> Recent, fold the oldest Recent (else New) frame into the
 * EMA slots and evict it while over cache_frames, mark the sinks. */
int lx2v_hip_kv_cache_memrope_update(lx2v_hip_ctx *ctx, lx2v_hip_kv *cache, const lx2v_hip_memrope_t *cfg,
                                     size_t frame_tokens);
/* causal_attention over the whole cache in place (no reference counterpart:
 * the reference copies the cache out with kv_cache_kv first, dit.rs:655-666).
 * q [heads, sq, head_dim] in the cache's dtype; mask [sq, rows] resident or
 * NULL. */
int lx2v_hip_kv_cache_attention(lx2v_hip_ctx *ctx, const lx2v_hip_buf *q, const lx2v_hip_kv *cache, size_t heads,
                                size_t sq, size_t head_dim, const lx2v_hip_mask *mask, lx2v_hip_buf *out);

/* Synthetic data for benchmarks (Rng::normal, rng.rs:39-54, drawn per element
 * index on the device; values agree with the host Rng to libm ulps):
 * buf[i] = normal(seed)[i] * std. */
int lx2v_hip_fill_normal(lx2v_hip_ctx *ctx, lx2v_hip_buf *buf, uint64_t seed, float std);

/* ---- pre-quantized activations (no reference counterpart) ----------------
 * The reference keeps activations f32 (backend.rs:9-11); these let a
 * producer hand linear e4m3 activations directly, so an FP8 linear runs
 * only its GEMM (the per-token quantization linear otherwise performs on
 * its input is done once, here). */

/* A [rows, cols] E4M3 activation buffer (len = rows * cols). */
int lx2v_hip_alloc_e4m3(lx2v_hip_ctx *ctx, size_t rows, size_t cols, lx2v_hip_buf **out);
/* xq rows [0, rows) = per-token e4m3 quantization (the rule linear applies
 * to FP8 weights: s = absmax / 448, code = RNE e4m3 of clamp(x * 448 /
 * absmax)) of x rows [x_row, x_row + rows); x is F32 or BF16 with xq's
 * cols per row, rows <= xq's rows. */
int lx2v_hip_quantize_act(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows,
                          lx2v_hip_buf *xq);

/* A [rows, cols] MXE4M3 activation buffer (len = rows * cols, cols a
 * multiple of 32).  It is what an FP8 linear writes when a second FP8
 * linear consumes its output directly (FFN up -> FFN down): the producing
 * GEMM's epilogue quantizes each 32-column block of a row with the scale
 * 2^k, k the smallest integer such that max |v| * 2^-k <= 448 (k in
 * [-127, 127]), codes = RNE e4m3 of v * 2^-k, and the consuming GEMM feeds
 * the scales to the block-scaled fp8 MFMA.  The per-32 scale is never
 * coarser than the per-token one of E4M3 buffers. */
int lx2v_hip_alloc_mx(lx2v_hip_ctx *ctx, size_t rows, size_t cols, lx2v_hip_buf **out);
/* xq rows [0, rows) = MX e4m3 quantization (the rule above) of x rows
 * [x_row, x_row + rows); x is F32 or BF16 with xq's cols per row, rows <=
 * xq's rows. */
int lx2v_hip_quantize_mx(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows,
                         lx2v_hip_buf *xq);
/* Test hook: an MXE4M3 buffer's raw contents, copied to host: codes [rows,
 * cols] and E8M0 scale bytes [cols / 32, rows] (block-major). */
int lx2v_hip_download_mx(lx2v_hip_ctx *ctx, const lx2v_hip_buf *buf, uint8_t *codes, uint8_t *scales);
/* Raw codes [rows, cols] and row scales [rows] of an E4M3 buffer (a test hook,
 * like download_mx; plain lx2v_hip_download returns the decoded values). */
int lx2v_hip_download_e4m3(lx2v_hip_ctx *ctx, const lx2v_hip_buf *buf, uint8_t *codes, float *scales);

/* ---- the op (backend.rs:198-212) ----------------------------------------- */

/* Backend::linear: y[y_row + i, :] = act(x[x_row + i, :] . W^T + b) for
 * i < rows; x has row stride w.cols, y row stride w.rows, bias (nullable)
 * has w.rows elements.  y must not overlap x or bias (LX2V_ERR_ALIAS).
 * An E4M3 or MXE4M3 x (its cols == w.cols) needs an FP8 weight and skips
 * the activation quantization.  y is F32, BF16 or MXE4M3 (its cols ==
 * w.rows; the result is MX-quantized in the GEMM's epilogue).  MXE4M3 on
 * either side needs an FP8 weight with one scale per output channel or per
 * 128 columns, w.cols a multiple of 128 and that buffer's row offset a
 * multiple of 16; otherwise LX2V_ERR_UNSUPPORTED. */
int lx2v_hip_linear(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows,
                    const lx2v_hip_weight *w, const lx2v_hip_buf *bias, int act,
                    lx2v_hip_buf *y, size_t y_row);

/* No counterpart in the reference: lx2v_hip_linear for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, plan, kernels and results as
 * lx2v_hip_linear, bit for bit; its workspaces (the per-token e4m3
 * activations and row scales, a bf16 bias's f32 copy, f32 activations' bf16
 * copy, split K's f32 partial sums) live in a device array of 48 MiB per
 * device instead of the context's, so it calls no hipMalloc / hipFree and
 * records no profiler events.  A call needing more (roughly rows * cols >
 * 48 MiB with f32 / bf16 activations, plus S * rows * w.rows * 4 bytes where
 * K is split S ways) fails with LX2V_ERR_UNSUPPORTED and a message and
 * enqueues nothing; pre-quantized E4M3 / MXE4M3 activations need no
 * activation workspace.  The array keeps the last call's contents.  One
 * context at a time holds a device's array: a call (or the launch of a graph
 * that captured such calls) while another context's work on it is still in
 * flight fails with LX2V_ERR_BUSY and enqueues nothing; calls of one context
 * are ordered on its stream.  A context is used by one thread at a time. */
int lx2v_hip_linear_noalloc(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows,
                            const lx2v_hip_weight *w, const lx2v_hip_buf *bias, int act,
                            lx2v_hip_buf *y, size_t y_row);

/* Test hook: the per-token e4m3 activation quantization linear applies to
 * x rows [x_row, x_row + rows) of width cols (FP8_ACT_E4M3), copied to host:
 * q [rows, cols] codes, s [rows] scales. */
int lx2v_hip_act_quant(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows,
                       size_t cols, uint8_t *q, float *s);

/* ---- HIP graphs (no reference counterpart: the wgpu backend batches
 * dispatches into command encoders instead, crates/lightx2v-wgpu/src/
 * lib.rs:441-505) ------------------------------------------------------------
 * Capture a fixed sequence of linear / quantize_act / copy calls on the
 * context stream once and replay it with one launch.  Between begin and end
 * only those calls are allowed (anything that allocates, frees, transfers
 * host memory or synchronises fails with LX2V_ERR_UNSUPPORTED); run the
 * sequence once eagerly first so workspaces are already large enough.
 * Replays read and write the buffers captured, at their current contents. */
typedef struct lx2v_hip_graph lx2v_hip_graph;
int lx2v_hip_graph_begin(lx2v_hip_ctx *ctx);
int lx2v_hip_graph_end(lx2v_hip_ctx *ctx, lx2v_hip_graph **out);
int lx2v_hip_graph_launch(lx2v_hip_ctx *ctx, const lx2v_hip_graph *g);
int lx2v_hip_graph_free(lx2v_hip_ctx *ctx, lx2v_hip_graph *g);

/* ---- sync / profiling (backend.rs:189-196) -------------------------------- */

/* Backend::sync (backend.rs:189-190). */
int lx2v_hip_sync(lx2v_hip_ctx *ctx);
/* Per-kernel timing with HIP events on the context stream.  Off by default;
 * LIGHTX2V_PROFILE=1 (any value but 0) at create time or this call turns it
 * on (the reference's switch, crates/lightx2v-cpu/src/lib.rs:27-34). */
int lx2v_hip_profile_enable(lx2v_hip_ctx *ctx, int on);
/* Backend::profile_report (backend.rs:192-195): table of kernel, calls,
 * total ms, mean us, share.  Synchronises.  Writes "" when nothing was
 * recorded.  Truncates to cap-1 bytes. */
int lx2v_hip_profile_report(lx2v_hip_ctx *ctx, char *out, size_t cap);
/* Backend::profile_reset (backend.rs:196). */
int lx2v_hip_profile_reset(lx2v_hip_ctx *ctx);
/* Time a region of the context stream with HIP events, whatever the
 * per-kernel switch says: begin != 0 records the start, begin == 0 the end,
 * and the elapsed time joins the report as row `name` (one call per
 * begin/end pair).  Regions do not nest per name.  No reference counterpart
 * (the reference times ops on the host, crates/lightx2v-cpu/src/lib.rs:27-105). */
int lx2v_hip_profile_region(lx2v_hip_ctx *ctx, const char *name, int begin);
/* Machine-readable form of one row of the report: calls and total
 * milliseconds of kernel `name` (0, 0 if never recorded).  Synchronises. */
int lx2v_hip_profile_kernel(lx2v_hip_ctx *ctx, const char *name, uint64_t *calls,
                            double *total_ms);

#ifdef __cplusplus
}
#endif
#endif

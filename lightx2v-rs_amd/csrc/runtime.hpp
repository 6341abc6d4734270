// runtime.hpp -- host-side objects behind the C ABI (context, buffers,
// weights) and the launchers each kernel translation unit exports.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/lightx2v_hip.h"

// Byte offset of the E8M0 scale of 32-column block b of row r in an MX
// buffer: the four blocks of a 128-column group sit together,
// [cols / 128][srows][4], so a GEMM reads a row's scales for 128 columns of
// K with one 32-bit load and a stage's scales for BM rows are one
// contiguous run.
__host__ __device__ inline size_t mx_sidx(size_t r, size_t b, size_t srows) {
    return ((b >> 2) * srows + r) * 4 + (b & 3);
}

struct lx2v_hip_buf {
    void *ptr = nullptr;
    size_t len = 0;    // elements
    int dtype = LX2V_DTYPE_F32;
    // LX2V_DTYPE_E4M3 only: [rows, cols] codes at ptr, f32 row scales at
    // `scales` (inside the same allocation).
    size_t rows = 0, cols = 0;
    float *scales = nullptr;
    // LX2V_DTYPE_MXE4M3 only: [rows, cols] codes at ptr, E8M0 block scales
    // at `mxs` (same allocation), [cols / 128][srows][4] (mx_sidx), srows =
    // rows rounded up to 16.
    uint8_t *mxs = nullptr;
    size_t srows = 0;
    bool quantized() const { return dtype == LX2V_DTYPE_E4M3 || dtype == LX2V_DTYPE_MXE4M3; }
    size_t elem_bytes() const { return dtype == LX2V_DTYPE_BF16 ? 2 : quantized() ? 1 : 4; }
    size_t bytes() const { return len * elem_bytes(); }
};

struct lx2v_hip_weight {
    int fmt = LX2V_WFMT_F32;
    size_t rows = 0, cols = 0, group = 0;
    void *codes = nullptr;    // f32 [rows*cols] | i8 [rows*cols] | packed u8 [rows*cols/2] | e4m3 [rows*cols]
    float *scales = nullptr;  // [rows * cols/group]
    float *zeros = nullptr;   // Q4 only
    // Q4 only: every zero is 8 (the symmetric codes, quant.rs's packing of
    // q + 8): the bf16 GEMM then dequantizes (c - 8) s as fma(c, s, -8 s),
    // the same f32 value, and loads no zeros.
    bool zero8 = false;
    uint8_t *raw_e4m3 = nullptr;  // FP8: codes exactly as passed in (for the dequant hook), only
                                  // kept when canonicalization changed a code
    size_t device_bytes = 0;
    size_t canonicalized = 0;
    // Stage-major copy of the group scales (and Q4 zeros) that the
    // direct-to-LDS bf16 GEMM loads with each 64-column stage:
    // [cols / 64][rows][spr] f32, entry i of (stage s, row r) = the scale of
    // the group holding column 64 s + i * 64 / spr, spr = 1 (group % 64 ==
    // 0), 2 (group 32) or 4 (other multiples of 16).  Null where that kernel
    // does not apply (F32, cols % 64 != 0, group % 16 != 0).
    float *sscale = nullptr, *szero = nullptr;
    int spr = 0;
    // FP8 with group 128 (cols % 128 == 0): what the fp8 MFMA kernels apply
    // the group scales with.  Their accumulator T holds the sum so far in
    // units of the current group's scale, T_g = (s_{g-1} / s_g) T_{g-1} + P_g
    // (P_g the group's raw code products), and the epilogue multiplies by
    // the last group's scale: gratio [cols / 128][rows] f32 (row g = s_{g-1}
    // / s_g per channel, row 0 all ones), glast [rows].  gratio_ok: every
    // scale finite and > 0 and no channel's scales more than 2^60 apart, so
    // no ratio or partial sum overflows; other grouped weights take the
    // bf16 MFMA kernel (k_gemm_w16) instead.
    float *gratio = nullptr, *glast = nullptr;
    bool gratio_ok = false;
    // F32 weights with cols % 64 == 0: the bf16 copy (RNE) the bf16 MFMA
    // reads, [rows, cols].
    uint16_t *wbf16 = nullptr;
};

namespace lx2v {

// Per-kernel timing (Backend::profile_report).
struct Profiler {
    bool on = false;
    struct Pending {
        std::string name;
        hipEvent_t a, b;
    };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> pool;
    std::map<std::string, std::pair<uint64_t, double>> stats;  // calls, total ms
    std::map<std::string, hipEvent_t> open_regions;            // lx2v_hip_profile_region
};

// Device memory a context owns for one purpose, grown on demand.
struct Stage {
    void *ptr = nullptr;
    size_t bytes = 0;
};

}  // namespace lx2v

namespace lx2v {

// Device scratch of lx2v_hip_linear_noalloc (lx2v_scratch.hip): a
// file-scope device array of kScratchBytes per device, its address resolved
// by scratch_setup (with the device current; a failure is retried by the
// next setup or claim).
constexpr size_t kScratchBytes = size_t(48) << 20;
struct Scratch {
    uint8_t *ptr;
    size_t bytes;
};
hipError_t scratch_setup(int device);
// The array's address (null + *err if it cannot be resolved), for a call
// being captured into a graph: the graph's launches claim the array.
void *scratch_address(int device, hipError_t *err);
// Claim the device's array for one call of `owner` (a context), whose
// completion `owner_done` records on its stream.  Held: *ptr is the array,
// the device lock is held -- enqueue the work, record owner_done, then
// scratch_unlock.  Busy: another context's work on the array has not
// completed.  Error: *err says why (no lock held for Busy / Error).
enum class ScratchClaim { Held, Busy, Error };
ScratchClaim scratch_claim(int device, const void *owner, hipEvent_t owner_done, void **ptr, hipError_t *err);
void scratch_unlock(int device);
// `owner` is going away: it no longer holds the array.
void scratch_release(int device, const void *owner);

}  // namespace lx2v

// Everything a context mutates lives in it: two contexts driven from two
// threads share no host state (the only process-wide state is each thread's
// last-error string and, per device, the scratch array's address and which
// context holds it, under that device's lock).
struct lx2v_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string name;
    int act_dtype = LX2V_DTYPE_F32;
    int fp8_act = LX2V_FP8_ACT_E4M3;
    int native_mode = LX2V_NATIVE_BF16;
    int num_cu = 256;
    // Workspace: per-token e4m3 activations + row scales (grown on demand).
    void *ws = nullptr;
    size_t ws_bytes = 0;
    lx2v::Profiler prof;
    // Stream capture in progress (lx2v_hip_graph_begin): nothing may
    // allocate, free or synchronise until lx2v_hip_graph_end.
    bool capturing = false;
    lx2v::Stage stage;     // boundary conversions (bias, parameters)
    lx2v::Stage mask;      // causal_attention's host mask, uploaded per call, and its tile summary
    lx2v::Stage kv_spare;  // the MemRoPE update's output layout, swapped with the cache it updates
    lx2v::Stage resid;     // linear_residual's output where the add cannot ride in the GEMM
    lx2v::Stage attn;      // split attention's partial sums (attention_split)
    lx2v::Stage splitk;    // split-K fp8 GEMM partial sums (Fp8Plan::splits)
    // The no-alloc entry point's hold on the device scratch: recorded after
    // each of its calls (and each launch of a graph that holds such calls);
    // capture_scratch: the capture in progress recorded one.
    hipEvent_t scratch_done = nullptr;
    bool capture_scratch = false;
};

namespace lx2v {

// Records `name` around the kernels `fn` enqueues when profiling is on.
template <class F>
hipError_t timed(lx2v_hip_ctx *ctx, const char *name, F &&fn);

void prof_begin(lx2v_hip_ctx *ctx, const char *name, hipEvent_t *a, hipEvent_t *b);
void prof_end(lx2v_hip_ctx *ctx, hipEvent_t b);

template <class F>
hipError_t timed(lx2v_hip_ctx *ctx, const char *name, F &&fn) {
    if (!ctx->prof.on) {
        fn();
        return hipGetLastError();
    }
    hipEvent_t a = nullptr, b = nullptr;
    prof_begin(ctx, name, &a, &b);
    fn();
    hipError_t e = hipGetLastError();
    prof_end(ctx, b);
    return e;
}

// ---- launchers (k_misc.hip) -------------------------------------------------
void launch_convert(hipStream_t s, const void *src, int src_dtype, void *dst, int dst_dtype,
                    size_t n);
void launch_f32_to_bf16(hipStream_t s, const float *src, uint16_t *dst, size_t n);
void launch_fill_normal(hipStream_t s, void *dst, int dtype, size_t n, uint64_t seed, float std);
void launch_dequant(hipStream_t s, const lx2v_hip_weight *w, const uint8_t *fp8_codes, float *out);
// Fills w->sscale / w->szero (allocated, w->spr set) from w->scales / w->zeros.
void launch_stage_scales(hipStream_t s, const lx2v_hip_weight *w);
void launch_q4_pack(hipStream_t s, const uint8_t *codes, size_t n, uint8_t *packed);
void launch_act_quant(hipStream_t s, const void *x, int dtype, size_t rows, size_t cols,
                      uint8_t *q, float *scale);
// out[r, c] = e4m3(q[r, c]) * scale[r] (OCP decode), f32.
void launch_act_quant_mx(hipStream_t s, const void *x, int dtype, size_t rows, size_t cols, uint8_t *q,
                         uint8_t *scales, size_t srows);
void launch_decode_mx(hipStream_t s, const uint8_t *q, const uint8_t *scales, size_t rows, size_t cols, size_t srows,
                      float *out);
void launch_decode_e4m3_rows(hipStream_t s, const uint8_t *q, const float *scale, size_t rows, size_t cols,
                             float *out);
void launch_quantize_q8(hipStream_t s, const float *src, size_t rows, size_t cols, size_t group,
                        int8_t *q, float *scales);
void launch_quantize_q4_sym(hipStream_t s, const float *src, size_t rows, size_t cols,
                            size_t group, uint8_t *packed, float *scales, float *zeros);
void launch_quantize_fp8(hipStream_t s, const float *src, size_t rows, size_t cols, size_t group,
                         uint8_t *q, float *scales);

// ---- norms and residuals around the linears (k_norm.hip) ----------------------
// out = norm(x) (a == null) or, with a: x += a * gate (gate null: 1), out =
// norm(x); norm = (v - mean) * rsqrt(var + eps) * (mod ? 1 + pm : pm) + pa.
// x / a of dtype dt (F32 / BF16); pm, pa, gate f32 [dim]; out of dtype od:
// F32 / BF16 values, E4M3 codes (+ oscale [rows]) or MXE4M3 codes (+ omx
// block scales, mx_sidx layout with srows).
void launch_norm(hipStream_t s, void *x, const void *a, int dt, const float *gate, const float *pm, const float *pa,
                 int mod, float eps, size_t rows, size_t dim, void *out, int od, float *oscale, uint8_t *omx,
                 size_t srows);
// h += a * g[column] over rows x dim (h, a of dtype dt).
void launch_gate_residual(hipStream_t s, void *h, const void *a, int dt, const float *g, size_t rows, size_t dim);

// Backend::head_split: columns [col_off, col_off + heads hd) of rows x stride
// src (dtype dt) -> out [heads, rows, hd] (dtype od), optionally RMS-normed
// across heads with w [heads hd] (dtype wdt) and RoPE-rotated with cs / sn
// [rows, hd / 2] (dtype rdt); null = skip.
void launch_head_split(hipStream_t s, const void *src, int dt, size_t rows, size_t stride, size_t col_off,
                       size_t heads, size_t hd, const void *w, int wdt, const void *cs, const void *sn, int rdt,
                       float eps, void *out, int od);

// ---- attention (k_attn.hip) -------------------------------------------------------
// out [sq, heads*d] = softmax(q k^T / sqrt(d), mask) v; q [heads, sq, d], k / v
// [heads, kvs, d] of dtype dt, keys 0 .. sk - 1 of each head used (kvs >= sk); mask [sq, sk] bytes or null; tiles its summary
// (launch_mask_tiles_bits or launch_mask_temporal, mask_tile_count entries) or
// null; out of dtype odt.
// mbits: the mask as bits (launch_mask_pack, mask_word_count words), read by
// the MFMA kernel in mixed tiles; the per-query kernel reads the bytes.
bool attention_mfma_supported(size_t d);
size_t mask_tile_count(size_t sq, size_t sk);
size_t mask_word_count(size_t sq, size_t sk);
void launch_mask_pack(hipStream_t s, const uint8_t *mask, size_t sq, size_t sk, uint32_t *bits);
// The tile summary from the packed bits (launch_mask_pack's output).
void launch_mask_tiles_bits(hipStream_t s, const uint32_t *bits, size_t sq, size_t sk, uint8_t *tiles);
// All three forms of the mask "tk[k] <= tq[q]" from temporal indices.
void launch_mask_temporal(hipStream_t s, const uint64_t *tq, size_t sq, const uint64_t *tk, size_t sk, uint8_t *mask,
                          uint32_t *bits, uint8_t *tiles);
// The split mode's piece count S for this call (each (head, query tile) in
// S pieces over parts of its allowed key tiles, merged in a second pass; 1:
// the one-pass kernel) and the bytes of f32 partial sums it needs; `part`
// points to that many bytes when nsplit > 1.
int attention_split(size_t heads, size_t sq, size_t sk, size_t d, int num_cu, size_t *bytes);
void launch_attention(hipStream_t s, const void *q, const void *k, const void *v, int dt, size_t heads, size_t sq,
                      size_t sk, size_t kvs, size_t d, const uint8_t *mask, const uint32_t *mbits,
                      const uint8_t *tiles, void *out, int odt, uint8_t *omx = nullptr, size_t omx_rows = 0,
                      float *part = nullptr, int nsplit = 1);

// ---- KV cache (k_kv.hip) ---------------------------------------------------------
// [heads, rows, d] from src (head stride sstride rows, first row srow0) to dst
// (dstride, drow0), converting dtype sdt -> ddt (F32 / BF16).
void launch_kv_copy(hipStream_t s, const void *src, int sdt, size_t sstride, size_t srow0, void *dst, int ddt,
                    size_t dstride, size_t drow0, size_t heads, size_t rows, size_t d);
// The MemRoPE update's gather: dst row r of every head from plan[r] (old row,
// zeros, or an EMA slot row folded with the evicted rows; see k_kv.hip).
void launch_kv_remap(hipStream_t s, const void *src, size_t sstride, void *dst, size_t dstride, int dt, size_t heads,
                     size_t rows, size_t d, const int *plan, int ft, const int n_ev[2], const int init_at[2],
                     const int ev_at[2], const float alpha[2]);

// ---- reference-exact load-time quantizers (k_quant.hip) ------------------------
// Fp8E4M3::quantize with quant.rs's own encoder: raw codes, exponent wrap included.
void launch_quantize_fp8_ref(hipStream_t s, const float *src, size_t rows, size_t cols, size_t group, uint8_t *q,
                             float *scales);
// codes = raw with exponent-0 non-zero codes set to signed zero; *count += replaced.
void launch_fp8_canon(hipStream_t s, const uint8_t *raw, uint8_t *codes, size_t n, unsigned long long *count);
// Q4::quantize (affine, optional HQQ, f16-rounded scale / zero), packed codes.
void launch_quantize_q4_ref(hipStream_t s, const float *src, size_t rows, size_t cols, size_t group, int hqq,
                            uint8_t *packed, float *scales, float *zeros);

// ---- GEMM launchers -----------------------------------------------------------
// Y[m, n] = act(sum_k A[m,k] B[n,k] * scales + bias[n]); A/Y already offset to
// the first row.  Return false when the shape is not served by that kernel.

// Activation operand of the generic GEMM.
enum AMode { A_F32 = 0, A_BF16 = 1, A_E4M3 = 2 };

// k_gemm_generic.hip: any shape, any weight format (the correctness path
// for ragged / tiny shapes).
void launch_gemm_generic(hipStream_t s, const void *a, int amode, const float *a_scale,
                         const lx2v_hip_weight *w, const float *bias, int act, void *y,
                         int y_dtype, size_t M);

// k_gemm_fp8.hip: fp8 MFMA, per-output-channel weight scale (group == K).
// plan_gemm_fp8 picks the kernel configuration for a shape.
struct Fp8Plan {
    int kernel = -1;  // configuration index, or -1: the register-staged kernel (K % 128 != 0)
    // > 1: K split over this many workgroups per tile (configuration 0),
    // their f32 partial sums in Fp8Mx::part, summed by a second pass that
    // applies the scales, bias, activation and output form
    int splits = 1;
};
// MX e4m3 operands of a launch: A's block scales ([K / 128][a_rows][4],
// a_len bytes readable from a; a_scale is then null) and/or the output's
// (y_dtype LX2V_DTYPE_MXE4M3: codes to y, scales to this.y in the same
// layout with y_rows).  Both pointers start at the linear's row offset
// (4 bytes per row).
struct Fp8Mx {
    const uint8_t *a = nullptr;
    size_t a_len = 0, a_rows = 0;
    uint8_t *y = nullptr;
    size_t y_rows = 0;
    // Residual mode (y_dtype BF16 / F32, plans with gemm_fp8_residual_ok):
    // y is the residual stream h, updated in place,
    // h[m][n] += out[m][n] * gate[n] with out as the plain store would write it.
    const float *gate = nullptr;
    // Grouped weight scales (a plan made with grouped = true): the weight's
    // stage-major scale copy (lx2v_hip_weight::sscale, group 128); b_scale
    // is then ignored.
    const float *wgs = nullptr;
    // Split-K partial sums (plans with splits > 1): splits * M * N floats.
    float *part = nullptr;
};
bool gemm_fp8_supported(size_t M, size_t N, size_t K);
// Group-128 FP8 weights on the fp8 MFMA (needs the stage-major scale copy).
bool gemm_fp8_grouped_supported(size_t M, size_t N, size_t K, size_t group);
// Whether the plan's kernel takes Fp8Mx::gate (the residual epilogue).
bool gemm_fp8_residual_ok(const Fp8Plan &p);
// y_dtype / act / residual: the launch's output form (some configurations
// cover only bf16 / MX output, and the residual epilogue only some).
// allow_split: the caller can give the split-K partial sums a workspace.
Fp8Plan plan_gemm_fp8(int num_cu, size_t M, size_t N, size_t K, bool mx, bool mx_in, bool grouped = false,
                      int y_dtype = LX2V_DTYPE_BF16, int act = LX2V_ACT_NONE, bool residual = false,
                      bool allow_split = false);
void launch_gemm_fp8(hipStream_t s, int num_cu, const Fp8Plan &p, const uint8_t *a, const float *a_scale,
                     const uint8_t *b, const float *b_scale, const float *bias, int act, void *y,
                     int y_dtype, size_t M, size_t N, size_t K, const Fp8Mx &mx);

// k_gemm_w16.hip: bf16 MFMA with the weight dequantized to bf16 inside
// the GEMM (Q8, Q4, FP8 with any group).  The direct-to-LDS kernel takes
// bf16 activations with K % 64 == 0 and a group that is a multiple of 16;
// the register-staged one f32 or bf16 activations with K and the group
// multiples of 16 (32 for Q4).
bool gemm_w16_supported(const lx2v_hip_weight *w);
void launch_gemm_w16(hipStream_t s, int num_cu, const void *x, int x_dtype,
                     const lx2v_hip_weight *w, const float *bias, int act, void *y, int y_dtype,
                     size_t M);
bool gemm_w16_dma_supported(const lx2v_hip_weight *w, size_t M);
int plan_gemm_w16_dma(int num_cu, size_t M, size_t N);
void launch_gemm_w16_dma(hipStream_t s, int cfg, const uint16_t *x, const lx2v_hip_weight *w, const float *bias,
                         int act, void *y, int y_dtype, size_t M);
// bf16 x bf16 (native f32 weights through their bf16 copy): X [M, K] and
// W [N, K] bf16, K % 64 == 0.
bool gemm_bf16_supported(size_t M, size_t N, size_t K);
void launch_gemm_bf16(hipStream_t s, int num_cu, const uint16_t *x, const uint16_t *w, const float *bias, int act,
                      void *y, int y_dtype, size_t M, size_t N, size_t K);

}  // namespace lx2v

// device_common.hpp -- device-side helpers shared by every gfx950 kernel of
// the quantized-linear backend: vector types, the e4m3 / bf16 codecs the
// GEMMs and the dequant kernel share, buffer-resource loads and the GELU
// epilogue.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "../../include/lightx2v_hip.h"

namespace lx2v {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Max over the 64 lanes of a wave (every lane gets it).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// ---- bf16 ------------------------------------------------------------------

// f32 -> bf16 bits, round to nearest even, NaN kept quiet (bit-exact with the
// host rule used at upload/download).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// Two f32 -> packed bf16 pair (low half = a), RNE via the gfx950 conversion.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    f32x2_t v = {a, b};
    bf16x2_t r = __builtin_convertvector(v, bf16x2_t);
    return __builtin_bit_cast(uint32_t, r);
}

// Eight elements of an F32 (two 16-byte words) or BF16 (one word) buffer as f32.
template <int DT>
__device__ __forceinline__ void unpack8(const u32x4 *raw, float v[8]) {
    if (DT == LX2V_DTYPE_BF16) {
        const u32x4 a = raw[0];
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[2 * j] = __uint_as_float(w[j] << 16);
            v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            f32x4 a = __builtin_bit_cast(f32x4, raw[h]);
            v[4 * h] = a.x, v[4 * h + 1] = a.y, v[4 * h + 2] = a.z, v[4 * h + 3] = a.w;
        }
    }
}

// ---- e4m3 ------------------------------------------------------------------

// quant.rs:409-420 bit for bit: exponent field 0 decodes m * 2^-12 (the
// reference's value, not OCP's m * 2^-9), e=15/m=7 is +NaN (0x7FC00000).
__device__ __forceinline__ float e4m3_ref_decode(uint32_t c) {
    uint32_t e = (c >> 3) & 15u, m = c & 7u;
    float mag;
    if (e == 0) {
        mag = (float)m * 0x1p-12f;
    } else if (e == 15u && m == 7u) {
        return __uint_as_float(0x7FC00000u);
    } else {
        mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
    }
    return (c & 0x80u) ? -mag : mag;
}

// OCP e4m3fn decode (what the fp8 MFMA sees): subnormals m * 2^-9.
__device__ __forceinline__ float e4m3_ocp_decode(uint32_t c) {
    uint32_t e = (c >> 3) & 15u, m = c & 7u;
    float mag;
    if (e == 0) {
        mag = (float)m * 0x1p-9f;
    } else if (e == 15u && m == 7u) {
        return __uint_as_float(0x7FC00000u);
    } else {
        mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
    }
    return (c & 0x80u) ? -mag : mag;
}

// OCP e4m3fn encode, round to nearest even, |v| <= 448 (callers clamp).
__device__ __forceinline__ uint32_t e4m3_ocp_encode(float v) {
    uint32_t b = __float_as_uint(v);
    uint32_t sign = (b >> 24) & 0x80u;
    uint32_t ab = b & 0x7FFFFFFFu;
    if (ab > 0x7F800000u) return 0x7Fu;
    float a = __uint_as_float(ab);
    if (a >= 0x1p-6f) {
        ab += 0x7FFFFu + ((ab >> 20) & 1u);
        int e8 = (int)(ab >> 23) - 120;
        uint32_t m = (ab >> 20) & 7u;
        if (e8 > 15 || (e8 == 15 && m == 7u)) return sign | 0x7Eu;
        return sign | ((uint32_t)e8 << 3) | m;
    }
    return sign | (uint32_t)__builtin_rintf(a * 512.0f);
}

// Canonical weight encoder (see lx2v_hip_quantize_fp8): quant.rs:376-406 for
// |v| >= 2^-6 -- where floor(log2|v|) is the exact binade exponent whatever
// way a libm log2f rounds, so it is taken from the bits -- 0x08 for
// 2^-7 < |v| < 2^-6, signed zero below.
__device__ __forceinline__ uint32_t e4m3_canon_encode(float v) {
    uint32_t b = __float_as_uint(v);
    uint32_t sign = (b >> 24) & 0x80u;
    float a = __builtin_fabsf(v);
    if (!(a < 464.0f)) return sign | 0x7Eu;  // inf, NaN, >= 464 (quant.rs:382-385)
    if (a < 0x1p-6f) return a > 0x1p-7f ? (sign | 0x08u) : sign;
    int e = (int)((__float_as_uint(a) >> 23) & 0xFFu) - 127;  // exact floor(log2 a)
    if (e > 8) return sign | 0x7Eu;
    uint32_t exp = (uint32_t)(e + 7);
    float p = __uint_as_float((uint32_t)(e + 127) << 23);
    float t = (a / p - 1.0f) * 8.0f;
    uint32_t mant = (uint32_t)__builtin_roundf(t);  // half away from zero, t in [0, 8]
    if (mant >= 8u) {
        if (exp >= 15u) return sign | 0x7Eu;
        return sign | ((exp + 1u) << 3);
    }
    return sign | (exp << 3) | mant;
}

// Four clamped, scaled values -> four e4m3 codes (byte j = element j) with
// the hardware pack conversion, round to nearest even.  An exhaustive sweep
// of every f32 in [-448, 448] on gfx950 found it bit-identical to
// e4m3_ocp_encode, the rule the oracle restates.
// Without the clamp (quant4_sc): every finite value of a block scaled by
// 2^-mx_exponent(amax) lies within +-448 already (mx_exponent's bound);
// infinities and NaNs become NaN codes instead of +-448.  quant4_sc takes
// the block's scale 2^k (mx_scale) and divides by it inside gfx950's scaled
// conversion (v_cvt_scalef32_pk_fp8_f32), which saves the multiply per
// value; a probe on the GPU found it bit-identical to the unscaled pack of
// v * 2^-k (lo and hi words, k from -127 to 120, 75 M in-range values plus
// infinities, NaNs and out-of-range values).
__device__ __forceinline__ uint32_t quant4_sc(const float *v, float scale) {
    typedef short v2s __attribute__((ext_vector_type(2)));
    v2s r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32((v2s){0, 0}, v[0], v[1], scale, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, v[2], v[3], scale, true);
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint32_t quant4(const float *v, float inv) {
    float t[4];
#pragma unroll
    for (int j = 0; j < 4; j++) t[j] = fminf(fmaxf(v[j] * inv, -448.0f), 448.0f);
    int r = __builtin_amdgcn_cvt_pk_fp8_f32(t[0], t[1], 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(t[2], t[3], r, true);
    return (uint32_t)r;
}

// ---- MX e4m3 blocks (32 columns of a row, one power-of-two scale) -------------

// The block's scale exponent: the smallest k with amax * 2^-k <= 448,
// clamped to [-127, 127].  amax = 1.m * 2^(E-127) lies in (448 * 2^(k-1),
// 448 * 2^k] exactly when k = E - 135 + [1.m > 1.75], so no division.
__device__ __forceinline__ int mx_exponent(float amax) {
    const uint32_t b = __float_as_uint(amax) & 0x7FFFFFFFu;
    const int k = (int)(b >> 23) - 135 + ((b & 0x7FFFFFu) > 0x600000u ? 1 : 0);
    return k < -127 ? -127 : (k > 127 ? 127 : k);
}

// 2^-k as an f32 for k in [-127, 126] (every finite amax gives k <= 121).
__device__ __forceinline__ float mx_inv(int k) { return __uint_as_float((uint32_t)(127 - k) << 23); }
// The scale operand of quant4_sc: 2^k as an f32 for k in [-126, 127]; k =
// -127 gives the bit pattern 0, which the conversion reads as the E8M0
// scale 2^-127 (its exponent field).
__device__ __forceinline__ float mx_scale(int k) { return __uint_as_float((uint32_t)(127 + k) << 23); }

// ---- GELU (crates/lightx2v-cpu/src/lib.rs:151-153) --------------------------

__device__ __forceinline__ float gelu_tanh(float x) {
    const float c = 0.7978845608028654f;  // sqrt(2/pi) rounded to f32
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

// The GEMM epilogues' GELU: 0.5 x (1 + tanh(u)) == x / (1 + e^(-2u)) with
// u = sqrt(2/pi) (x + 0.044715 x^3), on the hardware exp2 and reciprocal
// (a few ulp; the oracle's own 1 + tanhf(u) loses more than that to
// cancellation for u < 0).  Limits: x -> -inf gives -0, x -> +inf gives x.
// The exponent -2 log2(e) u is evaluated as x (k0 + k1 x^2), the constants
// folded (seven VALU operations in all, two of them transcendental).
__device__ __forceinline__ float gelu_tanh_fast(float x) {
    constexpr float k0 = -2.8853900817779268f * 0.7978845608028654f;  // -2 log2(e) sqrt(2/pi)
    constexpr float k1 = k0 * 0.044715f;
    const float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(x * x, k1, k0));
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// ---- workgroup -> output tile ------------------------------------------------------

// Map a linear workgroup id to an output tile (tm, tn) so that the
// workgroups one XCD runs (ids congruent mod 8 go to the same XCD) form a
// compact block of tiles: bands of up to 4 tile-rows walked column by
// column, so an XCD's L2 holds the few A row-panels and B column-panels
// its workgroups share.
__device__ __forceinline__ int xcd_order(int bid, int nb) {
    const int per = nb / 8, rem = nb % 8;
    const int x = bid % 8, j = bid / 8;
    return x * per + (x < rem ? x : rem) + j;
}

__device__ __forceinline__ void band_tile(int id, int tiles_m, int tiles_n, int *tm, int *tn) {
    const int G = tiles_m < 4 ? tiles_m : 4;
    const int group = id / (G * tiles_n);
    const int first = group * G;
    const int gsz = (tiles_m - first) < G ? (tiles_m - first) : G;
    const int in = id - first * tiles_n;
    *tm = first + in % gsz;
    *tn = in / gsz;
}

__device__ __forceinline__ void xcd_tile(int bid, int nb, int tiles_m, int tiles_n, int *tm, int *tn) {
    band_tile(xcd_order(bid, nb), tiles_m, tiles_n, tm, tn);
}

// ---- epilogue stores ----------------------------------------------------------------

// Four consecutive outputs y[0..3] (16-byte aligned for f32, 8 for bf16).
__device__ __forceinline__ void store4(float *y, float a, float b, float c, float d) {
    *(f32x4 *)y = (f32x4){a, b, c, d};
}
__device__ __forceinline__ void store4(uint16_t *y, float a, float b, float c, float d) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    *(u32x2_t *)y = (u32x2_t){pack_bf16x2(a, b), pack_bf16x2(c, d)};
}
__device__ __forceinline__ void store1(float *y, float v) { *y = v; }
__device__ __forceinline__ void store1(uint16_t *y, float v) { *y = f32_to_bf16_bits(v); }

// ---- buffer resources ----------------------------------------------------------

// A raw buffer descriptor: loads at byte offsets >= num_bytes return zero,
// which is how the GEMMs zero-fill ragged M/N edges without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t num_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)num_bytes,
                                             0x00020000);
}

__device__ __forceinline__ u32x4 buffer_load_x4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x2 buffer_load_x2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}

__device__ __forceinline__ uint32_t buffer_load_x1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

// Offset that is always out of range (reads as zero; a store there is dropped).
constexpr uint32_t kOob = 0x80000000u;

// 16-byte vector store through a buffer descriptor: offsets >= num_bytes are
// dropped by the hardware range check.  CP: the instruction's cache-policy
// bits (gfx950: 1 = sc0, 2 = nt, 16 = sc1), a hint for where the written
// lines are kept; the values stored are the same for every CP.
template <int CP = 0>
__device__ __forceinline__ void buffer_store_x4(u32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, CP);
}
template <int CP = 0>
__device__ __forceinline__ void buffer_store_b8(uint8_t v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b8(v, r, (int)off, 0, CP);
}

// v_permlane32_swap: lanes 32..63 of x trade places with lanes 0..31 of y.
// Applied to x = y = v it hands lane l the value of lane l ^ 32 in one of
// the two results (see max_pair32).
__device__ __forceinline__ void swap32(uint32_t &x, uint32_t &y) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
    x = r[0];
    y = r[1];
}
// max(v, v of lane l ^ 32) in every lane.
__device__ __forceinline__ float max_pair32(float v) {
    uint32_t x = __float_as_uint(v), y = x;
    swap32(x, y);
    return fmaxf(__uint_as_float(x), __uint_as_float(y));
}

// Compile-time loop: f(std::integral_constant<int, i>) for i = 0 .. N - 1.
template <typename F, int... I>
__device__ __forceinline__ void static_for_seq(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_seq(f, std::make_integer_sequence<int, N>{});
}

}  // namespace lx2v

// k_quant.hip -- load-time weight quantizers with the reference's own
// arithmetic, so that a checkpoint quantized on the device holds the codes
// lightx2v-rs's host quantizers write (crates/lightx2v-core/src/quant.rs).
//
// Built with -ffp-contract=off: no multiply-add is fused, every f32
// operation rounds where the reference's Rust rounds it.
//
//   k_quantize_q4_ref  -- Q4::quantize (quant.rs:226-292): affine min/max
//     codes, optionally HQQ-refined zero point, scale and zero rounded to
//     f16; one thread per group, the group's sums in the reference's order.
//   k_quantize_fp8_ref -- Fp8E4M3::quantize (quant.rs:423-447) with
//     f32_to_e4m3 (quant.rs:376-406) verbatim, its exponent wrap for
//     2^-9 <= |v/s| < 2^-6 included.
#include <float.h>

#include "device_common.hpp"
#include "powf_arm.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

constexpr int kQThreads = 256;

// floor(log2f(a)) for a finite a > 0.  log2 is taken in double and rounded
// once to f32, i.e. the correctly rounded f32 log2; its floor equals the floor
// of glibc's log2f (the libm the reference links) on every f32 below 2^-6,
// checked exhaustively on the host.  At and above 2^-6 the two can only
// disagree for an a just below a power of two, and there both exponents
// give the same code (the mantissa rounds up into the next binade).
__device__ __forceinline__ int floor_log2f(float a) { return (int)floorf((float)log2((double)a)); }

// quant.rs:376-406 bit for bit, Rust cast semantics: `(e + 7) as u8`
// wraps (-2 -> 254, -1 -> 255), `u8 << 3` drops the high bits, float `as
// u8` saturates, f32::round is half away from zero.
__device__ __forceinline__ uint32_t e4m3_ref_encode(float v) {
    const uint32_t bits = __float_as_uint(v);
    const uint32_t sign = (bits >> 24) & 0x80u;
    if ((bits & 0x7FFFFFFFu) == 0) return sign;  // +-0
    const float a = __builtin_fabsf(v);
    if (!(a < 464.0f)) return sign | 0x7Eu;      // inf, NaN, >= 464
    const int e = floor_log2f(a);
    if (e < -9) {
        // (a / (2^-9 / 8)).round() as u8, then min(7); a * 2^12 < 8 here
        const uint32_t m = (uint32_t)__builtin_roundf(a * 0x1p12f);
        return sign | (m < 7u ? m : 7u);
    }
    if (e > 8) return sign | 0x7Eu;
    const uint32_t exp = (uint32_t)(e + 7) & 0xFFu;
    const float p = __uint_as_float((uint32_t)(e + 127) << 23);  // 2^e, e in [-9, 8]
    const float t = __builtin_roundf((a / p - 1.0f) * 8.0f);     // in [0, 8]
    const uint32_t mant = t > 0.0f ? (uint32_t)t : 0u;
    if (mant >= 8u) {
        if (exp >= 15u) return sign | 0x7Eu;
        return sign | (((exp + 1u) << 3) & 0xFFu);
    }
    return sign | ((exp << 3) & 0xFFu) | mant;
}

__global__ __launch_bounds__(kQThreads) void k_quantize_fp8_ref(const float *__restrict__ src, size_t ngroups,
                                                                size_t group, uint8_t *__restrict__ q,
                                                                float *__restrict__ scales) {
    const size_t g = blockIdx.x * (size_t)(kQThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (g >= ngroups) return;
    const float *w = src + g * group;
    float amax = 0.0f;  // max is exact, so the reduction order is free
    for (size_t i = lane; i < group; i += 64) amax = fmaxf(amax, __builtin_fabsf(w[i]));
    amax = wave_max(amax);
    const float s = amax > 0.0f ? amax / 448.0f : 1.0f;  // quant.rs:434
    for (size_t i = lane; i < group; i += 64) q[g * group + i] = (uint8_t)e4m3_ref_encode(w[i] / s);
    if (lane == 0) scales[g] = s;
}

// HQQ's code of v: (v * is + z).round().clamp(0, 15) (quant.rs:236).
__device__ __forceinline__ float q4_code(float v, float is, float z) {
    const float r = __builtin_roundf(v * is + z);
    return fminf(fmaxf(r, 0.0f), 15.0f);
}

// f32::powf(a, y) for a > 0 as glibc computes it (powf_arm.hpp: bit-identical
// to the libm on every positive f32 at y = 0.7 - 1).
__device__ __forceinline__ float powf_ref(float a, float y) { return powf_arm::powf_pos(a, y); }

__global__ __launch_bounds__(kQThreads) void k_quantize_q4_ref(const float *__restrict__ src, size_t ngroups,
                                                               size_t group, int hqq, uint8_t *__restrict__ packed,
                                                               float *__restrict__ scales,
                                                               float *__restrict__ zeros) {
    const size_t g = blockIdx.x * (size_t)kQThreads + threadIdx.x;
    if (g >= ngroups) return;
    const float *w = src + g * group;
    float lo = FLT_MAX, hi = -FLT_MAX;
    for (size_t i = 0; i < group; i++) {
        lo = fminf(lo, w[i]);
        hi = fmaxf(hi, w[i]);
    }
    const float is = hi > lo ? 15.0f / (hi - lo) : 1.0f;
    float z = -lo * is;
    if (hqq) {  // quant.rs:248-276: lp 0.7, beta 10, kappa 1.01, at most 20 iterations
        const float pm1 = 0.7f - 1.0f, kappa = 1.01f, len = (float)group;
        float beta = 10.0f, best = FLT_MAX, best_z = z;
        for (int it = 0; it < 20; it++) {
            float err = 0.0f, zsum = 0.0f;
            for (size_t i = 0; i < group; i++) {
                const float v = w[i];
                const float c = q4_code(v, is, z);
                const float r = (c - z) / is;
                const float e = v - r;
                const float a = __builtin_fabsf(e);
                err += a;
                float sh = 0.0f;
                if (a > 0.0f) {
                    const float sg = __builtin_signbit(e) ? -1.0f : 1.0f;  // f32::signum
                    sh = sg * fmaxf(a - powf_ref(a, pm1) / beta, 0.0f);
                }
                zsum += c - (v - sh) * is;
            }
            err = err / len;
            if (err >= best) break;
            best = err;
            best_z = z;
            z = zsum / len;
            beta *= kappa;
        }
        z = best_z;
    }
    // Two codes per byte, element 2i in the low nibble (quant.rs:305-311);
    // the group is even, so a byte never spans two groups.
    uint8_t *out = packed + g * group / 2;
    for (size_t i = 0; i < group; i += 2) {
        const uint32_t c0 = (uint32_t)q4_code(w[i], is, z), c1 = (uint32_t)q4_code(w[i + 1], is, z);
        out[i / 2] = (uint8_t)(c0 | (c1 << 4));
    }
    scales[g] = (float)(_Float16)(1.0f / is);  // half::f16::from_f32: round to nearest even
    zeros[g] = (float)(_Float16)z;
}

// codes[i] = raw[i] with an exponent-0, non-zero-mantissa code replaced by
// the signed zero (the reference decodes those m * 2^-12, the fp8 MFMA
// m * 2^-9); *count += the number replaced.
__global__ __launch_bounds__(kQThreads) void k_fp8_canon(const uint8_t *__restrict__ raw, uint8_t *__restrict__ codes,
                                                         size_t n, unsigned long long *__restrict__ count) {
    const size_t i = blockIdx.x * (size_t)kQThreads + threadIdx.x;
    bool changed = false;
    if (i < n) {
        const uint32_t c = raw[i];
        changed = (c & 0x78u) == 0 && (c & 7u) != 0;
        codes[i] = (uint8_t)(changed ? (c & 0x80u) : c);
    }
    const unsigned long long nw = __popcll(__ballot(changed));
    if ((threadIdx.x & 63) == 0 && nw) atomicAdd(count, nw);
}

size_t blocks_for(size_t n, size_t per_block) { return (n + per_block - 1) / per_block; }

}  // namespace

void launch_quantize_fp8_ref(hipStream_t s, const float *src, size_t rows, size_t cols, size_t group, uint8_t *q,
                             float *scales) {
    const size_t ng = rows * cols / group;
    if (ng == 0) return;
    hipLaunchKernelGGL(k_quantize_fp8_ref, dim3((unsigned)blocks_for(ng, kQThreads / 64)), dim3(kQThreads), 0, s,
                       src, ng, group, q, scales);
}

void launch_fp8_canon(hipStream_t s, const uint8_t *raw, uint8_t *codes, size_t n, unsigned long long *count) {
    if (n == 0) return;
    hipLaunchKernelGGL(k_fp8_canon, dim3((unsigned)blocks_for(n, kQThreads)), dim3(kQThreads), 0, s, raw, codes, n,
                       count);
}

void launch_quantize_q4_ref(hipStream_t s, const float *src, size_t rows, size_t cols, size_t group, int hqq,
                            uint8_t *packed, float *scales, float *zeros) {
    const size_t ng = rows * cols / group;
    if (ng == 0) return;
    hipLaunchKernelGGL(k_quantize_q4_ref, dim3((unsigned)blocks_for(ng, kQThreads)), dim3(kQThreads), 0, s, src, ng,
                       group, hqq, packed, scales, zeros);
}

}  // namespace lx2v

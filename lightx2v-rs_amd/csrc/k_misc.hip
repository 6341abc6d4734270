// k_misc.hip -- the small kernels around the GEMMs: dtype conversion,
// synthetic fill, weight dequantization (the bit-exact decode check),
// per-token e4m3 activation quantization, and the device-side weight
// quantizers (quant.rs:154-178, 423-447 and the symmetric Q4 layout).
//
// Built with -ffp-contract=off: the quantizers and the dequant must round
// exactly like the reference's separate f32 multiply / divide / add.
#include "device_common.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

constexpr int kThreads = 256;

inline unsigned grid_for(size_t n, int per_block) {
    size_t g = (n + per_block - 1) / per_block;
    return (unsigned)(g > 0x7FFFFFFF ? 0x7FFFFFFF : (g == 0 ? 1 : g));
}

// ---- conversion ----------------------------------------------------------------

__global__ void k_convert(const void *src, int sd, void *dst, int dd, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        float v = sd == LX2V_DTYPE_BF16 ? bf16_bits_to_f32(((const uint16_t *)src)[i])
                                        : ((const float *)src)[i];
        if (dd == LX2V_DTYPE_BF16)
            ((uint16_t *)dst)[i] = f32_to_bf16_bits(v);
        else
            ((float *)dst)[i] = v;
    }
}

__global__ void k_decode_e4m3_rows(const uint8_t *q, const float *scale, size_t cols, size_t n, float *out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = e4m3_ocp_decode(q[i]) * scale[i / cols];
}

// ---- Rng::normal per element (rng.rs:39-54) --------------------------------------

__device__ __forceinline__ uint64_t splitmix(uint64_t seed, uint64_t draw) {
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (draw + 2);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float u01(uint64_t z) {
    return (float)(z >> 40) / 16777216.0f;
}

__global__ void k_fill_normal(void *dst, int dtype, size_t n, uint64_t seed, float std) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        uint64_t pair = i >> 1;
        float u1 = fmaxf(u01(splitmix(seed, 2 * pair)), 1e-7f);
        float u2 = u01(splitmix(seed, 2 * pair + 1));
        float r = sqrtf(-2.0f * logf(u1));
        float t = 6.2831854820251465f * u2;
        float v = ((i & 1) ? r * sinf(t) : r * cosf(t)) * std;
        if (dtype == LX2V_DTYPE_BF16)
            ((uint16_t *)dst)[i] = f32_to_bf16_bits(v);
        else
            ((float *)dst)[i] = v;
    }
}

// ---- dequantization (quant.rs:180-186, 294-303, 449-455) ----------------------

__global__ void k_dequant(int fmt, const void *codes, const float *scales, const float *zeros,
                          size_t group, size_t n, float *out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        float v;
        if (fmt == LX2V_WFMT_F32) {
            v = ((const float *)codes)[i];
        } else if (fmt == LX2V_WFMT_Q8) {
            v = (float)((const int8_t *)codes)[i] * scales[i / group];
        } else if (fmt == LX2V_WFMT_Q4) {
            uint32_t byte = ((const uint8_t *)codes)[i >> 1];
            uint32_t c = (byte >> (4 * (i & 1))) & 15u;
            size_t g = i / group;
            v = ((float)c - zeros[g]) * scales[g];
        } else {
            v = e4m3_ref_decode(((const uint8_t *)codes)[i]) * scales[i / group];
        }
        out[i] = v;
    }
}

// ---- per-token e4m3 activation quantization ---------------------------------------
//
// One wave per row.  amax = max|x|; inv = 448/amax, s = amax/448 (both
// correctly rounded divisions; amax <= 2^-64 -> 1, 1); q = e4m3(clamp(x*inv,
// -448, 448)) rounded to nearest even.  Lane l owns the 8-element chunks
// l, l + 64, ... of its row and keeps them in registers between the max and
// the quantization, so the row is read from HBM once.


// W waves share a row (W = 1, 2 or 4; the workgroup holds 4 / W rows); T =
// chunks of 8 per lane, 64 * W * T * 8 >= cols, cols % 8 == 0.  Wave part p
// of a row owns chunks lane + 64 (p + W t).
template <int DT, int T, int W>
__global__ __launch_bounds__(kThreads) void k_act_quant_rows(const void *x, size_t rows, size_t cols,
                                                             uint8_t *q, float *scale) {
    constexpr int R = DT == LX2V_DTYPE_BF16 ? 1 : 2;  // 16-byte loads per chunk
    __shared__ float red[kThreads / 64];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, part = wv % W;
    const size_t row = blockIdx.x * (size_t)(kThreads / 64 / W) + wv / W;
    const bool live = row < rows;
    const int nch = (int)(cols / 8);
    const u32x4 *xr = (const u32x4 *)((const char *)x + (live ? row : 0) * cols * (DT == LX2V_DTYPE_BF16 ? 2 : 4));
    u32x4 raw[T][R];
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int c = lane + 64 * (part + W * t);
#pragma unroll
        for (int h = 0; h < R; h++) raw[t][h] = (live && c < nch) ? xr[(size_t)c * R + h] : (u32x4){};
    }
    float amax = 0.0f;
#pragma unroll
    for (int t = 0; t < T; t++) {
        float v[8];
        unpack8<DT>(raw[t], v);
#pragma unroll
        for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
    }
    amax = wave_max(amax);
    if (W > 1) {
        if (lane == 0) red[wv] = amax;
        __syncthreads();
        const int first = wv - part;
#pragma unroll
        for (int p = 0; p < W; p++) amax = fmaxf(amax, red[first + p]);
    }
    if (!live) return;
    float inv = 1.0f, s = 1.0f;
    if (amax > 0x1p-64f) {
        inv = 448.0f / amax;
        s = amax / 448.0f;
    }
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    u32x2_t *qr = (u32x2_t *)(q + row * cols);
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int c = lane + 64 * (part + W * t);
        if (c < nch) {
            float v[8];
            unpack8<DT>(raw[t], v);
            qr[c] = (u32x2_t){quant4(&v[0], inv), quant4(&v[4], inv)};
        }
    }
    if (lane == 0 && part == 0) scale[row] = s;
}

__device__ float block_max(float v, float *red) {
    v = wave_max(v);
    int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kThreads / 64; i++) r = fmaxf(r, red[i]);
    return r;
}

// Any width: two passes over the row from memory.
template <int DT>
__global__ __launch_bounds__(kThreads) void k_act_quant_any(const void *x, size_t cols, uint8_t *q,
                                                            float *scale) {
    __shared__ float red[kThreads / 64];
    const size_t row = blockIdx.x;
    auto ld = [&](size_t c) -> float {
        if (DT == LX2V_DTYPE_BF16) return bf16_bits_to_f32(((const uint16_t *)x)[row * cols + c]);
        return ((const float *)x)[row * cols + c];
    };
    float amax = 0.0f;
    for (size_t c = threadIdx.x; c < cols; c += kThreads) amax = fmaxf(amax, fabsf(ld(c)));
    amax = block_max(amax, red);
    float inv = 1.0f, s = 1.0f;
    if (amax > 0x1p-64f) {
        inv = 448.0f / amax;
        s = amax / 448.0f;
    }
    for (size_t c = threadIdx.x; c < cols; c += kThreads) {
        float t = fminf(fmaxf(ld(c) * inv, -448.0f), 448.0f);
        q[row * cols + c] = (uint8_t)e4m3_ocp_encode(t);
    }
    if (threadIdx.x == 0) scale[row] = s;
}

// ---- weight quantizers: one wave per group -------------------------------------------

__global__ __launch_bounds__(kThreads) void k_quantize_q8(const float *src, size_t ngroups,
                                                          size_t group, int8_t *q, float *scales) {
    size_t g = blockIdx.x * (size_t)(kThreads / 64) + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (g >= ngroups) return;
    const float *w = src + g * group;
    float amax = 0.0f;
    for (size_t i = lane; i < group; i += 64) amax = fmaxf(amax, fabsf(w[i]));
    amax = wave_max(amax);
    float s = amax > 0.0f ? amax / 127.0f : 1.0f;  // quant.rs:165
    for (size_t i = lane; i < group; i += 64) {
        float r = __builtin_roundf(w[i] / s);
        r = fminf(fmaxf(r, -127.0f), 127.0f);  // finite inputs: clamp == f32::clamp
        q[g * group + i] = (int8_t)(int)r;
    }
    if (lane == 0) scales[g] = s;
}

__global__ __launch_bounds__(kThreads) void k_quantize_q4_sym(const float *src, size_t ngroups,
                                                              size_t group, uint8_t *packed,
                                                              float *scales, float *zeros) {
    size_t g = blockIdx.x * (size_t)(kThreads / 64) + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (g >= ngroups) return;
    const float *w = src + g * group;
    float amax = 0.0f;
    for (size_t i = lane; i < group; i += 64) amax = fmaxf(amax, fabsf(w[i]));
    amax = wave_max(amax);
    float s = amax > 0.0f ? amax / 7.0f : 1.0f;
    for (size_t p = lane; p < group / 2; p += 64) {
        float r0 = fminf(fmaxf(__builtin_roundf(w[2 * p] / s), -8.0f), 7.0f);
        float r1 = fminf(fmaxf(__builtin_roundf(w[2 * p + 1] / s), -8.0f), 7.0f);
        uint32_t c0 = (uint32_t)((int)r0 + 8), c1 = (uint32_t)((int)r1 + 8);
        packed[(g * group) / 2 + p] = (uint8_t)(c0 | (c1 << 4));
    }
    if (lane == 0) {
        scales[g] = s;
        zeros[g] = 8.0f;
    }
}

__global__ __launch_bounds__(kThreads) void k_quantize_fp8(const float *src, size_t ngroups,
                                                           size_t group, uint8_t *q,
                                                           float *scales) {
    size_t g = blockIdx.x * (size_t)(kThreads / 64) + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (g >= ngroups) return;
    const float *w = src + g * group;
    float amax = 0.0f;
    for (size_t i = lane; i < group; i += 64) amax = fmaxf(amax, fabsf(w[i]));
    amax = wave_max(amax);
    float s = amax > 0.0f ? amax / 448.0f : 1.0f;  // quant.rs:434
    for (size_t i = lane; i < group; i += 64) q[g * group + i] = (uint8_t)e4m3_canon_encode(w[i] / s);
    if (lane == 0) scales[g] = s;
}

// ---- MX e4m3 activation quantization --------------------------------------------
//
// One thread per 32-column block of a row (cols % 32 == 0): amax = max |x|
// of the block, k = mx_exponent(amax), codes = e4m3(clamp(x * 2^-k, +-448))
// rounded to nearest even, scale byte k + 127 at s[mx_sidx(r, c / 32, srows)].

template <int DT>
__global__ __launch_bounds__(kThreads) void k_act_quant_mx(const void *x, size_t rows, size_t cols, uint8_t *q,
                                                           uint8_t *s, size_t srows) {
    constexpr int W = DT == LX2V_DTYPE_BF16 ? 1 : 2;  // 16-byte loads per 8 elements
    const size_t nb = cols / 32;
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= rows * nb) return;
    const size_t r = i / nb, b = i - r * nb;
    const u32x4 *src = (const u32x4 *)((const uint8_t *)x + (r * cols + b * 32) * (DT == LX2V_DTYPE_BF16 ? 2 : 4));
    u32x4 raw[4 * W];
#pragma unroll
    for (int j = 0; j < 4 * W; j++) raw[j] = src[j];
    float v[32];
#pragma unroll
    for (int c = 0; c < 4; c++) unpack8<DT>(raw + c * W, v + 8 * c);
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const int k = mx_exponent(amax);
    const float inv = mx_inv(k);
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; j++) w[j] = quant4(v + 4 * j, inv);
    u32x4 *dst = (u32x4 *)(q + r * cols + b * 32);
    dst[0] = (u32x4){w[0], w[1], w[2], w[3]};
    dst[1] = (u32x4){w[4], w[5], w[6], w[7]};
    s[mx_sidx(r, b, srows)] = (uint8_t)(k + 127);
}

__global__ void k_decode_mx(const uint8_t *q, const uint8_t *s, size_t rows, size_t cols, size_t srows, float *out) {
    const size_t n = rows * cols;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / cols, c = i - r * cols;
        out[i] = __builtin_amdgcn_ldexpf(e4m3_ocp_decode(q[i]), (int)s[mx_sidx(r, c / 32, srows)] - 127);
    }
}

}  // namespace

void launch_act_quant_mx(hipStream_t s, const void *x, int dtype, size_t rows, size_t cols, uint8_t *q,
                         uint8_t *scales, size_t srows) {
    const size_t n = rows * (cols / 32);
    if (n == 0) return;
    if (dtype == LX2V_DTYPE_BF16)
        hipLaunchKernelGGL(k_act_quant_mx<LX2V_DTYPE_BF16>, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s, x,
                           rows, cols, q, scales, srows);
    else
        hipLaunchKernelGGL(k_act_quant_mx<LX2V_DTYPE_F32>, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s, x,
                           rows, cols, q, scales, srows);
}

void launch_decode_mx(hipStream_t s, const uint8_t *q, const uint8_t *scales, size_t rows, size_t cols, size_t srows,
                      float *out) {
    const size_t n = rows * cols;
    if (n == 0) return;
    hipLaunchKernelGGL(k_decode_mx, dim3(grid_for(n, kThreads * 4)), dim3(kThreads), 0, s, q, scales, rows, cols,
                       srows, out);
}

void launch_convert(hipStream_t s, const void *src, int sd, void *dst, int dd, size_t n) {
    if (n == 0) return;
    hipLaunchKernelGGL(k_convert, dim3(grid_for(n, kThreads * 4)), dim3(kThreads), 0, s, src, sd, dst,
                       dd, n);
}

void launch_decode_e4m3_rows(hipStream_t s, const uint8_t *q, const float *scale, size_t rows, size_t cols,
                             float *out) {
    const size_t n = rows * cols;
    if (n == 0) return;
    hipLaunchKernelGGL(k_decode_e4m3_rows, dim3(grid_for(n, kThreads * 4)), dim3(kThreads), 0, s, q, scale, cols,
                       n, out);
}

void launch_fill_normal(hipStream_t s, void *dst, int dtype, size_t n, uint64_t seed, float std) {
    if (n == 0) return;
    hipLaunchKernelGGL(k_fill_normal, dim3(grid_for(n, kThreads * 4)), dim3(kThreads), 0, s, dst,
                       dtype, n, seed, std);
}

void launch_dequant(hipStream_t s, const lx2v_hip_weight *w, const uint8_t *fp8_codes, float *out) {
    size_t n = w->rows * w->cols;
    if (n == 0) return;
    const void *codes = w->fmt == LX2V_WFMT_FP8 ? (const void *)fp8_codes : w->codes;
    hipLaunchKernelGGL(k_dequant, dim3(grid_for(n, kThreads * 4)), dim3(kThreads), 0, s, w->fmt,
                       codes, w->scales, w->zeros, w->group ? w->group : 1, n, out);
}

// out[(s * rows + r) * spr + i] = in[r * (cols / group) + (64 s + i * 64 / spr) / group]
__global__ void k_stage_scales(const float *__restrict__ in, float *__restrict__ out, size_t rows, size_t cols,
                               size_t group, int spr, size_t n) {
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < n; t += (size_t)gridDim.x * blockDim.x) {
        const size_t i = t % spr, rs = t / spr, r = rs % rows, st = rs / rows;
        const size_t col = st * 64 + i * (64 / spr);
        out[t] = in[r * (cols / group) + col / group];
    }
}

void launch_stage_scales(hipStream_t s, const lx2v_hip_weight *w) {
    const size_t n = w->cols / 64 * w->rows * (size_t)w->spr;
    if (n == 0) return;
    const dim3 grid(grid_for(n, kThreads));
    hipLaunchKernelGGL(k_stage_scales, grid, dim3(kThreads), 0, s, w->scales, w->sscale, w->rows, w->cols,
                       w->group, w->spr, n);
    if (w->szero)
        hipLaunchKernelGGL(k_stage_scales, grid, dim3(kThreads), 0, s, w->zeros, w->szero, w->rows, w->cols,
                           w->group, w->spr, n);
}

template <int DT>
void act_quant_rows(hipStream_t s, const void *x, size_t rows, size_t cols, uint8_t *q, float *scale) {
    const size_t per = (cols / 8 + 63) / 64;  // chunks per lane with one wave per row
    const dim3 block(kThreads);
    auto grid = [&](int w) { return dim3((unsigned)((rows + (kThreads / 64 / w) - 1) / (kThreads / 64 / w))); };
    // W waves per row (one up to 2048 columns, two up to 4096, four beyond)
    // and T = the chunks a lane needs, so that no lane loads a chunk past
    // every row (1536 columns: 4.38 -> 4.27 us at 4680 rows against a
    // masked fourth chunk).
    const int w = per <= 4 ? 1 : (per <= 8 ? 2 : 4);
    const int t = (int)((per + w - 1) / w);
#define LX2V_AQ(T, W) \
    hipLaunchKernelGGL((k_act_quant_rows<DT, T, W>), grid(W), block, 0, s, x, rows, cols, q, scale)
    if (w == 1) {
        switch (t) {
            case 1: LX2V_AQ(1, 1); break;
            case 2: LX2V_AQ(2, 1); break;
            case 3: LX2V_AQ(3, 1); break;
            default: LX2V_AQ(4, 1); break;
        }
    } else if (w == 2) {
        if (t <= 3)
            LX2V_AQ(3, 2);
        else
            LX2V_AQ(4, 2);
    } else {
        switch (t) {
            case 3: LX2V_AQ(3, 4); break;
            case 4: LX2V_AQ(4, 4); break;
            case 5: LX2V_AQ(5, 4); break;
            case 6: LX2V_AQ(6, 4); break;
            case 7: LX2V_AQ(7, 4); break;
            default: LX2V_AQ(8, 4); break;
        }
    }
#undef LX2V_AQ
}

void launch_act_quant(hipStream_t s, const void *x, int dtype, size_t rows, size_t cols,
                      uint8_t *q, float *scale) {
    if (rows == 0) return;
    // Rows kept in registers: up to 8 chunks of 8 per lane over 4 waves
    // (16384 elements); wider or ragged rows take the two-pass kernel.
    const size_t per = (cols / 8 + 63) / 64;
    const bool fast = cols % 8 == 0 && per <= 32u;
    if (fast) {
        if (dtype == LX2V_DTYPE_BF16)
            act_quant_rows<LX2V_DTYPE_BF16>(s, x, rows, cols, q, scale);
        else
            act_quant_rows<LX2V_DTYPE_F32>(s, x, rows, cols, q, scale);
        return;
    }
    if (dtype == LX2V_DTYPE_BF16)
        hipLaunchKernelGGL(k_act_quant_any<LX2V_DTYPE_BF16>, dim3(rows), dim3(kThreads), 0, s, x, cols,
                           q, scale);
    else
        hipLaunchKernelGGL(k_act_quant_any<LX2V_DTYPE_F32>, dim3(rows), dim3(kThreads), 0, s, x, cols, q,
                           scale);
}

void launch_quantize_q8(hipStream_t s, const float *src, size_t rows, size_t cols, size_t group,
                        int8_t *q, float *scales) {
    size_t ng = rows * cols / group;
    if (ng == 0) return;
    hipLaunchKernelGGL(k_quantize_q8, dim3(grid_for(ng, kThreads / 64)), dim3(kThreads), 0, s, src, ng,
                       group, q, scales);
}

void launch_quantize_q4_sym(hipStream_t s, const float *src, size_t rows, size_t cols,
                            size_t group, uint8_t *packed, float *scales, float *zeros) {
    size_t ng = rows * cols / group;
    if (ng == 0) return;
    hipLaunchKernelGGL(k_quantize_q4_sym, dim3(grid_for(ng, kThreads / 64)), dim3(kThreads), 0, s, src,
                       ng, group, packed, scales, zeros);
}

void launch_quantize_fp8(hipStream_t s, const float *src, size_t rows, size_t cols, size_t group,
                         uint8_t *q, float *scales) {
    size_t ng = rows * cols / group;
    if (ng == 0) return;
    hipLaunchKernelGGL(k_quantize_fp8, dim3(grid_for(ng, kThreads / 64)), dim3(kThreads), 0, s, src,
                       ng, group, q, scales);
}

}  // namespace lx2v

// k_norm.hip -- the producers and consumers around the block linears:
// layer_norm / residual_norm (crates/lightx2v-cpu/src/lib.rs:328-388) with
// the activation quantization of the next FP8 linear fused into the same
// pass, and gate_residual (lib.rs:390-400).
//
//   layer_norm:    out = LN(x) * mul + add, LN(x) = (x - mean) / sqrt(var + eps),
//                  mul / add = w / b (NormKind::Affine) or 1 + mods[scale] /
//                  mods[shift] (NormKind::Mod);
//   residual_norm: h += a * gate (gate = mods[gate] or 1), then out = norm(h),
//                  the norm reading the unrounded sum;
//   gate_residual: h += a * mods[gate].
//
// `out` is F32 or BF16 (the reference's op), E4M3 (per-token e4m3 codes + row
// scale, the input an FP8 linear contracts, quantized by the rule of
// lx2v_hip_quantize_act) or MXE4M3 (one power-of-two scale per 32 columns).
// A row lives in registers: one to four waves per row, lane l owning the
// 8-element chunks l, l + 64 W, ..., so x / h / a are read once and the
// quantized row is written once.
//
// Reductions run across lanes, so mean and variance round differently from
// the reference's sequential f32 sums (relative 1e-7 level); every other
// operation rounds as the reference's.
#include "device_common.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

constexpr int kNThreads = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum (or max) over the W waves of a row: each wave's lane-0 value through LDS.
template <int W, bool MAX>
__device__ __forceinline__ float row_reduce(float v, float *red, int wv, int part, int lane) {
    v = MAX ? wave_max(v) : wave_sum(v);
    if constexpr (W > 1) {
        __syncthreads();  // red may still be read by the previous reduction
        if (lane == 0) red[wv] = v;
        __syncthreads();
        const int first = wv - part;
        v = red[first];
#pragma unroll
        for (int p = 1; p < W; p++) v = MAX ? fmaxf(v, red[first + p]) : v + red[first + p];
    }
    return v;
}

__device__ __forceinline__ void pack8(const float v[8], u32x4 *raw, int dt) {
    if (dt == LX2V_DTYPE_BF16) {
        raw[0] = (u32x4){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                         pack_bf16x2(v[6], v[7])};
    } else {
        raw[0] = __builtin_bit_cast(u32x4, (f32x4){v[0], v[1], v[2], v[3]});
        raw[1] = __builtin_bit_cast(u32x4, (f32x4){v[4], v[5], v[6], v[7]});
    }
}

struct NormArgs {
    void *x;            // layer_norm: x; residual_norm: h (updated in place)
    const void *a;      // residual addend (RES)
    const float *gate;  // RES: [dim] gate, or null for 1
    const float *pm;    // [dim]: w (affine) or mods[scale] (mod)
    const float *pa;    // [dim]: b (affine) or mods[shift] (mod)
    int mod;            // NormKind::Mod: multiply by 1 + pm
    float eps;
    size_t rows, dim;
    void *out;          // F32 / BF16 values, or e4m3 codes
    float *oscale;      // E4M3: [rows] row scales
    uint8_t *omx;       // MXE4M3: block scales (mx_sidx layout)
    size_t srows;
};

// DT: dtype of x / h / a; OD: dtype of out; T chunks of 8 per lane, W waves
// per row (64 W T 8 >= dim, dim % 8 == 0).
template <int DT, int OD, int T, int W, bool RES>
__global__ __launch_bounds__(kNThreads) void k_norm_rows(NormArgs p) {
    constexpr int R = DT == LX2V_DTYPE_BF16 ? 1 : 2;  // 16-byte words per chunk
    __shared__ float red[kNThreads / 64];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, part = wv % W;
    const size_t row = blockIdx.x * (size_t)(kNThreads / 64 / W) + wv / W;
    const bool live = row < p.rows;
    const int nch = (int)(p.dim / 8);
    u32x4 *xr = (u32x4 *)((char *)p.x + (live ? row : 0) * p.dim * (DT == LX2V_DTYPE_BF16 ? 2 : 4));
    const u32x4 *ar = (const u32x4 *)((const char *)p.a + (live ? row : 0) * p.dim * (DT == LX2V_DTYPE_BF16 ? 2 : 4));
    float v[T][8];
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int c = lane + 64 * (part + W * t);
        const bool in = live && c < nch;
        u32x4 raw[R];
#pragma unroll
        for (int h = 0; h < R; h++) raw[h] = in ? xr[(size_t)c * R + h] : (u32x4){};
        unpack8<DT>(raw, v[t]);
        if constexpr (RES) {
            u32x4 ra[R];
#pragma unroll
            for (int h = 0; h < R; h++) ra[h] = in ? ar[(size_t)c * R + h] : (u32x4){};
            float av[8];
            unpack8<DT>(ra, av);
            float g[8];
#pragma unroll
            for (int e = 0; e < 8; e++) g[e] = 1.0f;
            if (p.gate && in) {
                const f32x4 g0 = *(const f32x4 *)(p.gate + 8 * c), g1 = *(const f32x4 *)(p.gate + 8 * c + 4);
                g[0] = g0.x, g[1] = g0.y, g[2] = g0.z, g[3] = g0.w, g[4] = g1.x, g[5] = g1.y, g[6] = g1.z, g[7] = g1.w;
            }
#pragma unroll
            for (int e = 0; e < 8; e++) v[t][e] = v[t][e] + av[e] * g[e];  // h += a * gate
            if (in) {
                u32x4 w[R];
                pack8(v[t], w, DT);
#pragma unroll
                for (int h = 0; h < R; h++) xr[(size_t)c * R + h] = w[h];
            }
        }
#pragma unroll
        for (int e = 0; e < 8; e++) s += in ? v[t][e] : 0.0f;
    }
    const float dimf = (float)p.dim;
    const float mean = row_reduce<W, false>(s, red, wv, part, lane) / dimf;
    float q = 0.0f;
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int c = lane + 64 * (part + W * t);
        if (live && c < nch) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float d = v[t][e] - mean;
                q += d * d;
            }
        }
    }
    const float var = row_reduce<W, false>(q, red, wv, part, lane) / dimf;
    const float inv = 1.0f / sqrtf(var + p.eps);
    float amax = 0.0f;
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int c = lane + 64 * (part + W * t);
        if (live && c < nch) {
            const f32x4 m0 = *(const f32x4 *)(p.pm + 8 * c), m1 = *(const f32x4 *)(p.pm + 8 * c + 4);
            const f32x4 a0 = *(const f32x4 *)(p.pa + 8 * c), a1 = *(const f32x4 *)(p.pa + 8 * c + 4);
            const float mu[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
            const float ad[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float n = (v[t][e] - mean) * inv;
                v[t][e] = n * (p.mod ? 1.0f + mu[e] : mu[e]) + ad[e];
                amax = fmaxf(amax, fabsf(v[t][e]));
            }
        }
    }
    if constexpr (OD == LX2V_DTYPE_F32 || OD == LX2V_DTYPE_BF16) {
        if (!live) return;
        u32x4 *orow = (u32x4 *)((char *)p.out + row * p.dim * (OD == LX2V_DTYPE_BF16 ? 2 : 4));
        constexpr int RO = OD == LX2V_DTYPE_BF16 ? 1 : 2;
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int c = lane + 64 * (part + W * t);
            if (c < nch) {
                u32x4 w[RO];
                pack8(v[t], w, OD);
#pragma unroll
                for (int h = 0; h < RO; h++) orow[(size_t)c * RO + h] = w[h];
            }
        }
    } else if constexpr (OD == LX2V_DTYPE_E4M3) {
        // per-token: the lx2v_hip_quantize_act rule on the normalized row
        amax = row_reduce<W, true>(amax, red, wv, part, lane);
        if (!live) return;
        float qi = 1.0f, qs = 1.0f;
        if (amax > 0x1p-64f) {
            qi = 448.0f / amax;
            qs = amax / 448.0f;
        }
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        u32x2_t *qr = (u32x2_t *)((uint8_t *)p.out + row * p.dim);
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int c = lane + 64 * (part + W * t);
            if (c < nch) qr[c] = (u32x2_t){quant4(&v[t][0], qi), quant4(&v[t][4], qi)};
        }
        if (lane == 0 && part == 0) p.oscale[row] = qs;
    } else {
        // MX: the 32-column block of chunk c is chunks 4 (c / 4) .. + 3, held
        // by four neighbouring lanes (c = lane + 64 k)
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        u32x2_t *qr = (u32x2_t *)((uint8_t *)p.out + (live ? row : 0) * p.dim);
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int c = lane + 64 * (part + W * t);
            const bool in = live && c < nch;
            float bm = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) bm = fmaxf(bm, in ? fabsf(v[t][e]) : 0.0f);
            bm = fmaxf(bm, __shfl_xor(bm, 1, 64));
            bm = fmaxf(bm, __shfl_xor(bm, 2, 64));
            const int k = mx_exponent(bm);
            const float qi = mx_inv(k);
            if (in) {
                qr[c] = (u32x2_t){quant4(&v[t][0], qi), quant4(&v[t][4], qi)};
                if ((c & 3) == 0) p.omx[mx_sidx(row, (size_t)(c / 4), p.srows)] = (uint8_t)(k + 127);
            }
        }
    }
}

// Rows of any width (dim % 8 != 0 or > 16384): one workgroup per row,
// passes over the row from memory.  The residual sum is recomputed from h
// and a in every pass and h is written last, so the norm reads the
// unrounded sum as in the fast kernel.
template <int DT, int OD, bool RES>
__global__ __launch_bounds__(kNThreads) void k_norm_any(NormArgs p) {
    constexpr int NW = kNThreads / 64;
    __shared__ float red[NW];
    const size_t row = blockIdx.x, base = row * p.dim;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    auto ld = [&](const void *b, size_t i) -> float {
        if (DT == LX2V_DTYPE_BF16) return bf16_bits_to_f32(((const uint16_t *)b)[i]);
        return ((const float *)b)[i];
    };
    auto val = [&](size_t c) -> float {
        float v = ld(p.x, base + c);
        if constexpr (RES) v = v + ld(p.a, base + c) * (p.gate ? p.gate[c] : 1.0f);
        return v;
    };
    float s = 0.0f;
    for (size_t c = tid; c < p.dim; c += kNThreads) s += val(c);
    const float mean = row_reduce<NW, false>(s, red, wv, wv, lane) / (float)p.dim;
    float q = 0.0f;
    for (size_t c = tid; c < p.dim; c += kNThreads) {
        const float d = val(c) - mean;
        q += d * d;
    }
    const float var = row_reduce<NW, false>(q, red, wv, wv, lane) / (float)p.dim;
    const float inv = 1.0f / sqrtf(var + p.eps);
    auto outv = [&](size_t c) { return (val(c) - mean) * inv * (p.mod ? 1.0f + p.pm[c] : p.pm[c]) + p.pa[c]; };
    if constexpr (OD == LX2V_DTYPE_F32 || OD == LX2V_DTYPE_BF16) {
        for (size_t c = tid; c < p.dim; c += kNThreads) {
            const float o = outv(c);
            if (OD == LX2V_DTYPE_BF16)
                ((uint16_t *)p.out)[base + c] = f32_to_bf16_bits(o);
            else
                ((float *)p.out)[base + c] = o;
        }
    } else if constexpr (OD == LX2V_DTYPE_E4M3) {
        float amax = 0.0f;
        for (size_t c = tid; c < p.dim; c += kNThreads) amax = fmaxf(amax, fabsf(outv(c)));
        amax = row_reduce<NW, true>(amax, red, wv, wv, lane);
        float qi = 1.0f, qs = 1.0f;
        if (amax > 0x1p-64f) {
            qi = 448.0f / amax;
            qs = amax / 448.0f;
        }
        for (size_t c = tid; c < p.dim; c += kNThreads) {
            float t[4] = {outv(c), 0.0f, 0.0f, 0.0f};
            ((uint8_t *)p.out)[base + c] = (uint8_t)(quant4(t, qi) & 0xFFu);
        }
        if (tid == 0) p.oscale[row] = qs;
    } else {
        for (size_t b = tid; b < p.dim / 32; b += kNThreads) {
            float o[32], bm = 0.0f;
#pragma unroll
            for (int e = 0; e < 32; e++) {
                o[e] = outv(32 * b + e);
                bm = fmaxf(bm, fabsf(o[e]));
            }
            const int k = mx_exponent(bm);
            const float qi = mx_inv(k);
            uint32_t *dst = (uint32_t *)((uint8_t *)p.out + base + 32 * b);
#pragma unroll
            for (int e = 0; e < 8; e++) dst[e] = quant4(o + 4 * e, qi);
            p.omx[mx_sidx(row, b, p.srows)] = (uint8_t)(k + 127);
        }
    }
    if constexpr (RES) {
        __syncthreads();  // every pass above has read h
        for (size_t c = tid; c < p.dim; c += kNThreads) {
            const float v = val(c);
            if (DT == LX2V_DTYPE_BF16)
                ((uint16_t *)p.x)[base + c] = f32_to_bf16_bits(v);
            else
                ((float *)p.x)[base + c] = v;
        }
    }
}

// h += a * g, eight elements per thread (n % 8 == 0) or one.
template <int DT, bool V8>
__global__ __launch_bounds__(kNThreads) void k_gate_residual(void *h, const void *a, const float *g, size_t n,
                                                            size_t dim) {
    const size_t i = blockIdx.x * (size_t)kNThreads + threadIdx.x;
    if constexpr (V8) {
        constexpr int R = DT == LX2V_DTYPE_BF16 ? 1 : 2;
        if (i * 8 >= n) return;
        u32x4 rh[R], ra[R];
#pragma unroll
        for (int k = 0; k < R; k++) {
            rh[k] = ((const u32x4 *)h)[i * R + k];
            ra[k] = ((const u32x4 *)a)[i * R + k];
        }
        float vh[8], va[8];
        unpack8<DT>(rh, vh);
        unpack8<DT>(ra, va);
        const size_t c = (i * 8) % dim;
#pragma unroll
        for (int e = 0; e < 8; e++) vh[e] = vh[e] + va[e] * g[c + e];
        pack8(vh, rh, DT);
#pragma unroll
        for (int k = 0; k < R; k++) ((u32x4 *)h)[i * R + k] = rh[k];
    } else {
        if (i >= n) return;
        const size_t c = i % dim;
        if (DT == LX2V_DTYPE_BF16) {
            uint16_t *hp = (uint16_t *)h;
            const float v = bf16_bits_to_f32(hp[i]) + bf16_bits_to_f32(((const uint16_t *)a)[i]) * g[c];
            hp[i] = f32_to_bf16_bits(v);
        } else {
            ((float *)h)[i] = ((float *)h)[i] + ((const float *)a)[i] * g[c];
        }
    }
}

template <int DT, int OD, bool RES>
void norm_launch(hipStream_t s, const NormArgs &p) {
    const size_t per = (p.dim / 8 + 63) / 64;  // chunks of 8 per lane with one wave per row
    const dim3 block(kNThreads);
    auto grid = [&](int w) { return dim3((unsigned)((p.rows + (kNThreads / 64 / w) - 1) / (kNThreads / 64 / w))); };
    if (p.dim % 8 != 0 || per > 32) {
        hipLaunchKernelGGL((k_norm_any<DT, OD, RES>), dim3((unsigned)p.rows), block, 0, s, p);
    } else {
        // W waves per row (one up to 2048 columns, two up to 4096, four
        // beyond) and T chunks per lane, T the fewest that cover the row
        // for the common widths (1536: 3, 3072: 3 x 2, 5120: 3 x 4, 8960:
        // 5 x 4), so lanes load no chunk past every row.
        const int w = per <= 4 ? 1 : (per <= 8 ? 2 : 4);
        const int t = (int)((per + w - 1) / w);
#define LX2V_NR(T, W) hipLaunchKernelGGL((k_norm_rows<DT, OD, T, W, RES>), grid(W), block, 0, s, p)
        if (w == 1) {
            if (t <= 2)
                LX2V_NR(2, 1);
            else if (t == 3)
                LX2V_NR(3, 1);
            else
                LX2V_NR(4, 1);
        } else if (w == 2) {
            if (t <= 3)
                LX2V_NR(3, 2);
            else
                LX2V_NR(4, 2);
        } else {
            if (t <= 3)
                LX2V_NR(3, 4);
            else if (t == 4)
                LX2V_NR(4, 4);
            else if (t == 5)
                LX2V_NR(5, 4);
            else
                LX2V_NR(8, 4);
        }
#undef LX2V_NR
    }
}

template <int DT, bool RES>
void norm_launch_od(hipStream_t s, const NormArgs &p, int od) {
    switch (od) {
        case LX2V_DTYPE_F32: norm_launch<DT, LX2V_DTYPE_F32, RES>(s, p); break;
        case LX2V_DTYPE_BF16: norm_launch<DT, LX2V_DTYPE_BF16, RES>(s, p); break;
        case LX2V_DTYPE_E4M3: norm_launch<DT, LX2V_DTYPE_E4M3, RES>(s, p); break;
        default: norm_launch<DT, LX2V_DTYPE_MXE4M3, RES>(s, p); break;
    }
}

// ---- head_split (crates/lightx2v-cpu/src/lib.rs:406-455) -----------------------------
//
// Columns [col_off, col_off + heads hd) of each row -> out [heads, rows, hd],
// optionally RMS-normalised across all heads (x * inv * w, inv = 1 /
// sqrt(mean(x^2) + eps)) and rotated by RoPE (interleaved pairs, cos / sin
// [rows, hd / 2]).  One wave per row; lane l holds the 8-column chunks l,
// l + 64, ... of the row in registers (hd % 8 == 0, so a chunk lies in one
// head and holds 4 whole pairs).  The mean of squares is a lane reduction;
// every other operation rounds as the reference's (no contraction).

struct HeadSplitArgs {
    const void *src;
    size_t rows, stride, col_off, heads, hd;
    const void *w;      // [heads hd] or null
    const void *cs;     // cos [rows, hd / 2] or null (then sn is null too)
    const void *sn;
    int wdt, rdt;       // dtype of w, of cos / sin (F32 or BF16)
    float eps;
    void *out;
};

__device__ __forceinline__ float ld_param(const void *p, int dt, size_t i) {
    return dt == LX2V_DTYPE_BF16 ? bf16_bits_to_f32(((const uint16_t *)p)[i]) : ((const float *)p)[i];
}

// Parameters i .. i + N - 1 (N = 4 or 8, i a multiple of N) in one or two
// vector loads.
template <int N>
__device__ __forceinline__ void ld_params(const void *p, int dt, size_t i, float (&o)[N]) {
    if (dt == LX2V_DTYPE_BF16) {
        const uint32_t *q = (const uint32_t *)((const uint16_t *)p + i);
        uint32_t u[N / 2];
        if constexpr (N == 8) {
            const u32x4 t = *(const u32x4 *)q;
            u[0] = t.x, u[1] = t.y, u[2] = t.z, u[3] = t.w;
        } else {
            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
            const u32x2_t t = *(const u32x2_t *)q;
            u[0] = t.x, u[1] = t.y;
        }
#pragma unroll
        for (int e = 0; e < N / 2; e++) {
            o[2 * e] = bf16_bits_to_f32(u[e] & 0xFFFFu);
            o[2 * e + 1] = bf16_bits_to_f32(u[e] >> 16);
        }
    } else {
#pragma unroll
        for (int e = 0; e < N; e += 4) {
            const f32x4 t = *(const f32x4 *)((const float *)p + i + e);
            o[e] = t.x, o[e + 1] = t.y, o[e + 2] = t.z, o[e + 3] = t.w;
        }
    }
}

template <int DT, int OD, int T>
__global__ __launch_bounds__(kNThreads) void k_head_split(HeadSplitArgs p) {
    constexpr int R = DT == LX2V_DTYPE_BF16 ? 1 : 2;  // 16-byte words per input chunk
    constexpr int EB = DT == LX2V_DTYPE_BF16 ? 2 : 4;
    const int lane = threadIdx.x & 63;
    const size_t row = blockIdx.x * (size_t)(kNThreads / 64) + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // wave-uniform
    const size_t d = p.heads * p.hd;
    const int nch = (int)(d / 8);
    const u32x4 *xr = (const u32x4 *)((const char *)p.src + (row * p.stride + p.col_off) * EB);
    float v[T][8];
    float ss = 0.0f;
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int c = lane + 64 * t;
        u32x4 raw[R];
#pragma unroll
        for (int h = 0; h < R; h++) raw[h] = c < nch ? xr[(size_t)c * R + h] : (u32x4){};
        unpack8<DT>(raw, v[t]);
#pragma unroll
        for (int e = 0; e < 8; e++) ss += v[t][e] * v[t][e];
    }
    if (p.w) {
        const float ms = wave_sum(ss) / (float)d;
        const float inv = 1.0f / sqrtf(ms + p.eps);
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int c = lane + 64 * t;
            if (c >= nch) continue;
            float wv[8];
            ld_params<8>(p.w, p.wdt, (size_t)c * 8, wv);
#pragma unroll
            for (int e = 0; e < 8; e++) v[t][e] = v[t][e] * inv * wv[e];
        }
    }
    const size_t hh = p.hd / 2;
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int c = lane + 64 * t;
        if (c >= nch) continue;
        const size_t col = (size_t)c * 8, h = col / p.hd, j = col % p.hd;
        if (p.cs) {
            float cv[4], sv[4];
            ld_params<4>(p.cs, p.rdt, row * hh + j / 2, cv);
            ld_params<4>(p.sn, p.rdt, row * hh + j / 2, sv);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float a = v[t][2 * e], b = v[t][2 * e + 1];
                v[t][2 * e] = a * cv[e] - b * sv[e];
                v[t][2 * e + 1] = a * sv[e] + b * cv[e];
            }
        }
        u32x4 w[2];
        pack8(v[t], w, OD);
        u32x4 *o = (u32x4 *)((char *)p.out + ((h * p.rows + row) * p.hd + j) * (OD == LX2V_DTYPE_BF16 ? 2 : 4));
        o[0] = w[0];
        if (OD == LX2V_DTYPE_F32) o[1] = w[1];
    }
}

// Any head size (and rows too wide for the register kernel): one wave per
// row, columns strided over the lanes, the row read twice.
template <int DT, int OD>
__global__ __launch_bounds__(kNThreads) void k_head_split_any(HeadSplitArgs p) {
    const int lane = threadIdx.x & 63;
    const size_t row = blockIdx.x * (size_t)(kNThreads / 64) + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const size_t d = p.heads * p.hd, base = row * p.stride + p.col_off;
    auto ld = [&](size_t col) {
        return DT == LX2V_DTYPE_BF16 ? bf16_bits_to_f32(((const uint16_t *)p.src)[base + col])
                                     : ((const float *)p.src)[base + col];
    };
    float inv = 1.0f;
    if (p.w) {
        float ss = 0.0f;
        for (size_t col = lane; col < d; col += 64) {
            const float x = ld(col);
            ss += x * x;
        }
        inv = 1.0f / sqrtf(wave_sum(ss) / (float)d + p.eps);
    }
    auto val = [&](size_t col) { return p.w ? ld(col) * inv * ld_param(p.w, p.wdt, col) : ld(col); };
    auto st = [&](size_t col, float x) {
        const size_t h = col / p.hd, j = col % p.hd, o = (h * p.rows + row) * p.hd + j;
        if (OD == LX2V_DTYPE_BF16)
            ((uint16_t *)p.out)[o] = f32_to_bf16_bits(x);
        else
            ((float *)p.out)[o] = x;
    };
    const size_t hh = p.hd / 2;
    // lane-strided over pairs of each head (an odd head's last element alone)
    const size_t per = hh + (p.hd & 1);
    for (size_t u = lane; u < p.heads * per; u += 64) {
        const size_t h = u / per, i = u % per, col = h * p.hd + 2 * i;
        if (i == hh) {  // odd hd: the unpaired last element
            st(col, val(col));
            continue;
        }
        const float a = val(col), b = val(col + 1);
        if (p.cs) {
            const float cv = ld_param(p.cs, p.rdt, row * hh + i), sv = ld_param(p.sn, p.rdt, row * hh + i);
            st(col, a * cv - b * sv);
            st(col + 1, a * sv + b * cv);
        } else {
            st(col, a);
            st(col + 1, b);
        }
    }
}

template <int DT, int OD>
void head_split_launch(hipStream_t s, const HeadSplitArgs &p) {
    const dim3 block(kNThreads), grid((unsigned)((p.rows + kNThreads / 64 - 1) / (kNThreads / 64)));
    const size_t d = p.heads * p.hd, per = (d / 8 + 63) / 64;
    const bool vec = p.hd % 8 == 0 && p.stride % 8 == 0 && p.col_off % 8 == 0 && per <= 12;
    if (!vec)
        hipLaunchKernelGGL((k_head_split_any<DT, OD>), grid, block, 0, s, p);
    else if (per <= 2)
        hipLaunchKernelGGL((k_head_split<DT, OD, 2>), grid, block, 0, s, p);
    else if (per == 3)  // 1536 columns: no chunk past the row
        hipLaunchKernelGGL((k_head_split<DT, OD, 3>), grid, block, 0, s, p);
    else if (per <= 4)
        hipLaunchKernelGGL((k_head_split<DT, OD, 4>), grid, block, 0, s, p);
    else if (per <= 8)
        hipLaunchKernelGGL((k_head_split<DT, OD, 8>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((k_head_split<DT, OD, 12>), grid, block, 0, s, p);
}

}  // namespace

void launch_norm(hipStream_t s, void *x, const void *a, int dt, const float *gate, const float *pm, const float *pa,
                 int mod, float eps, size_t rows, size_t dim, void *out, int od, float *oscale, uint8_t *omx,
                 size_t srows) {
    if (rows == 0 || dim == 0) return;
    NormArgs p;
    p.x = x;
    p.a = a;
    p.gate = gate;
    p.pm = pm;
    p.pa = pa;
    p.mod = mod;
    p.eps = eps;
    p.rows = rows;
    p.dim = dim;
    p.out = out;
    p.oscale = oscale;
    p.omx = omx;
    p.srows = srows;
    const bool res = a != nullptr;
    if (dt == LX2V_DTYPE_BF16) {
        if (res)
            norm_launch_od<LX2V_DTYPE_BF16, true>(s, p, od);
        else
            norm_launch_od<LX2V_DTYPE_BF16, false>(s, p, od);
    } else {
        if (res)
            norm_launch_od<LX2V_DTYPE_F32, true>(s, p, od);
        else
            norm_launch_od<LX2V_DTYPE_F32, false>(s, p, od);
    }
}

void launch_head_split(hipStream_t s, const void *src, int dt, size_t rows, size_t stride, size_t col_off,
                       size_t heads, size_t hd, const void *w, int wdt, const void *cs, const void *sn, int rdt,
                       float eps, void *out, int od) {
    if (rows == 0 || heads * hd == 0) return;
    HeadSplitArgs p{src, rows, stride, col_off, heads, hd, w, cs, sn, wdt, rdt, eps, out};
    if (dt == LX2V_DTYPE_BF16) {
        if (od == LX2V_DTYPE_BF16)
            head_split_launch<LX2V_DTYPE_BF16, LX2V_DTYPE_BF16>(s, p);
        else
            head_split_launch<LX2V_DTYPE_BF16, LX2V_DTYPE_F32>(s, p);
    } else {
        if (od == LX2V_DTYPE_BF16)
            head_split_launch<LX2V_DTYPE_F32, LX2V_DTYPE_BF16>(s, p);
        else
            head_split_launch<LX2V_DTYPE_F32, LX2V_DTYPE_F32>(s, p);
    }
}

void launch_gate_residual(hipStream_t s, void *h, const void *a, int dt, const float *g, size_t rows, size_t dim) {
    const size_t n = rows * dim;
    if (n == 0) return;
    const bool v8 = dim % 8 == 0;
    const size_t threads = v8 ? n / 8 : n;
    const dim3 grid((unsigned)((threads + kNThreads - 1) / kNThreads)), block(kNThreads);
    if (dt == LX2V_DTYPE_BF16) {
        if (v8)
            hipLaunchKernelGGL((k_gate_residual<LX2V_DTYPE_BF16, true>), grid, block, 0, s, h, a, g, n, dim);
        else
            hipLaunchKernelGGL((k_gate_residual<LX2V_DTYPE_BF16, false>), grid, block, 0, s, h, a, g, n, dim);
    } else {
        if (v8)
            hipLaunchKernelGGL((k_gate_residual<LX2V_DTYPE_F32, true>), grid, block, 0, s, h, a, g, n, dim);
        else
            hipLaunchKernelGGL((k_gate_residual<LX2V_DTYPE_F32, false>), grid, block, 0, s, h, a, g, n, dim);
    }
}

}  // namespace lx2v

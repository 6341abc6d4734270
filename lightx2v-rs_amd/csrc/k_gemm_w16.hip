// k_gemm_w16.hip -- weight-only quantized linear on the gfx950 bf16 MFMA
// (v_mfma_f32_32x32x16_bf16): Q8 (quant.rs:142-205), Q4 (quant.rs:207-356)
// and FP8 with any group (quant.rs:358-460).
//
//   Y[m, n] = act( sum_k bf16(X[m,k]) * bf16(dequant(W)[n,k]) + bias[n] )
//
// The packed codes stream from HBM in the reference's byte layout (int8
// row-major; nibbles two per byte, element 2i low; e4m3 row-major) with
// their f32 per-group scales.  The tile loader dequantizes each 16/32-code
// chunk in registers exactly as the reference's dequantize() (q*s,
// (c-z)*s, e4m3(c)*s in f32), rounds to bf16 and writes the K-major tile to
// LDS; activations (f32 or bf16) are rounded to bf16 on the same path.
// Tile shape, swizzle, XCD mapping, the two-register-stage pipeline and the
// operand roles (weights = MFMA A operand, so the epilogue writes four
// consecutive channels per lane) follow k_gemm_fp8.hip, with a 64-element K
// stage (128 bytes of bf16 per row).
#include "device_common.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

constexpr int BK = 64;        // K elements per stage
constexpr int ROWB = BK * 2;  // bytes per LDS tile row (bf16)

__device__ __forceinline__ uint32_t lds_off(uint32_t row, uint32_t c) {
    return row * ROWB + ((c ^ ((row >> 1) & 7u)) << 4);
}

// Source chunks per weight row per K stage, and K elements per source chunk.
template <int WF>
struct WTraits;
template <>
struct WTraits<LX2V_WFMT_Q8> {
    static constexpr int kPerChunk = 16, kChunksPerRow = BK / 16;
};
template <>
struct WTraits<LX2V_WFMT_FP8> {
    static constexpr int kPerChunk = 16, kChunksPerRow = BK / 16;
};
template <>
struct WTraits<LX2V_WFMT_Q4> {
    static constexpr int kPerChunk = 32, kChunksPerRow = BK / 32;
};

// Dequantize one 16-byte source chunk into LDS chunks (8 bf16 each).
template <int WF>
__device__ __forceinline__ void dequant_store(uint8_t *s, uint32_t row, uint32_t sc, u32x4 raw,
                                              float scale, float zero) {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    if (WF == LX2V_WFMT_Q4) {
        // 32 nibbles, element 2i in the low nibble of byte i (quant.rs:305-311).
#pragma unroll
        for (int q = 0; q < 4; q++) {  // 4 LDS chunks of 8 elements
            uint32_t word = w[q];
            u32x4 o;
            uint32_t ov[4];
#pragma unroll
            for (int p = 0; p < 4; p++) {
                float a = ((float)((word >> (8 * p)) & 15u) - zero) * scale;
                float b = ((float)((word >> (8 * p + 4)) & 15u) - zero) * scale;
                ov[p] = pack_bf16x2(a, b);
            }
            o.x = ov[0], o.y = ov[1], o.z = ov[2], o.w = ov[3];
            *(u32x4 *)(s + lds_off(row, sc * 4 + q)) = o;
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; h++) {  // 2 LDS chunks of 8 elements
            uint32_t ov[4];
#pragma unroll
            for (int p = 0; p < 2; p++) {
                uint32_t word = w[2 * h + p];
                float f[4];
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    if (WF == LX2V_WFMT_Q8)
                        f[b] = (float)(int)(int8_t)(word >> (8 * b)) * scale;
                    else
                        f[b] = e4m3_ref_decode((word >> (8 * b)) & 0xFFu) * scale;
                }
                ov[2 * p] = pack_bf16x2(f[0], f[1]);
                ov[2 * p + 1] = pack_bf16x2(f[2], f[3]);
            }
            u32x4 o;
            o.x = ov[0], o.y = ov[1], o.z = ov[2], o.w = ov[3];
            *(u32x4 *)(s + lds_off(row, sc * 2 + h)) = o;
        }
    }
}

template <int BM, int BN, int WF, int XT, typename TY>
__global__ __launch_bounds__(256, 1) void k_gemm_w16(const void *__restrict__ X,
                                                     const uint8_t *__restrict__ Wc,
                                                     const float *__restrict__ Ws,
                                                     const float *__restrict__ Wz, int group,
                                                     const float *__restrict__ bias,
                                                     TY *__restrict__ Y, int M, int N, int K,
                                                     int act, int tiles_m, int tiles_n) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int XB = XT == LX2V_DTYPE_BF16 ? 2 : 4;    // bytes per activation
    constexpr int XLD = XT == LX2V_DTYPE_BF16 ? 1 : 2;   // 16B loads per LDS chunk
    constexpr int ACH = BM * 8 / 256;                     // LDS chunks of X per thread
    constexpr int CPR = WTraits<WF>::kChunksPerRow;
    constexpr int KPC = WTraits<WF>::kPerChunk;
    constexpr int BCH = BN * CPR / 256;                   // weight source chunks per thread
    constexpr uint32_t WB_DEN = WF == LX2V_WFMT_Q4 ? 2 : 1;  // code bytes per element = 1/DEN
    static_assert(BCH >= 1, "tile too small for the weight loader");
    constexpr int STAGE = (BM + BN) * ROWB;
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KG = K / group;  // scale columns
    const int KT = (K + BK - 1) / BK;

    const auto rx = make_rsrc((const uint8_t *)X + (size_t)m0 * K * XB, (uint32_t)(M - m0) * (uint32_t)K * XB);
    const uint32_t wrow_bytes = (uint32_t)K / WB_DEN;
    const auto rw = make_rsrc(Wc + (size_t)n0 * wrow_bytes, (uint32_t)(N - n0) * wrow_bytes);

    // X chunk j of this thread: tile row j * 32 + tid / 8, LDS chunk tid % 8
    // (K elements [8c, 8c+8) of the stage); one LDS offset up to j * 32 rows.
    const uint32_t crow = (uint32_t)tid >> 3, cc = (uint32_t)tid & 7u;
    const uint32_t x_goff = (crow * (uint32_t)K + cc * 8) * XB;
    const uint32_t x_gstep = 32u * (uint32_t)K * XB;
    const uint32_t x_loff = lds_off(crow, cc);
    // Weight source chunks.
    uint32_t w_goff[BCH], w_row[BCH], w_sc[BCH], w_srow[BCH];
#pragma unroll
    for (int j = 0; j < BCH; j++) {
        uint32_t id = j * 256 + tid, row = id / CPR, sc = id % CPR;
        w_row[j] = row;
        w_sc[j] = sc;
        w_goff[j] = row * wrow_bytes + sc * 16;
        uint32_t n = (uint32_t)n0 + row;
        w_srow[j] = (n < (uint32_t)N ? n : (uint32_t)N - 1) * (uint32_t)KG;
    }

    struct Regs {
        u32x4 x[ACH][XLD];
        u32x4 w[BCH];
        float sc[BCH], ze[BCH];
    };
    // Stage `kt` into registers; stages past the end load zeros.
    auto gload = [&](Regs &r, int kt) {
        const uint32_t k0 = (uint32_t)kt * BK;
        const bool xin = kt < KT && k0 + cc * 8 < (uint32_t)K;
#pragma unroll
        for (int j = 0; j < ACH; j++)
#pragma unroll
            for (int h = 0; h < XLD; h++)
                r.x[j][h] = buffer_load_x4(rx, xin ? x_goff + j * x_gstep + k0 * XB + h * 16 : kOob);
#pragma unroll
        for (int j = 0; j < BCH; j++) {
            uint32_t kk = k0 + w_sc[j] * KPC;
            bool kin = kt < KT && kk < (uint32_t)K;
            r.w[j] = buffer_load_x4(rw, kin ? w_goff[j] + k0 / WB_DEN : kOob);
            uint32_t g = w_srow[j] + (kin ? kk : 0) / (uint32_t)group;
            r.sc[j] = Ws[g];
            if (WF == LX2V_WFMT_Q4) r.ze[j] = Wz[g];
        }
    };
    auto sstore = [&](const Regs &r, int buf) {
        uint8_t *s = smem + buf * STAGE;
#pragma unroll
        for (int j = 0; j < ACH; j++) {
            u32x4 o;
            if (XT == LX2V_DTYPE_BF16) {
                o = r.x[j][0];
            } else {
                f32x4 lo = __builtin_bit_cast(f32x4, r.x[j][0]);
                f32x4 hi = __builtin_bit_cast(f32x4, r.x[j][1]);
                o.x = pack_bf16x2(lo.x, lo.y);
                o.y = pack_bf16x2(lo.z, lo.w);
                o.z = pack_bf16x2(hi.x, hi.y);
                o.w = pack_bf16x2(hi.z, hi.w);
            }
            *(u32x4 *)(s + x_loff + j * 32 * ROWB) = o;
        }
        uint8_t *sb = s + BM * ROWB;
#pragma unroll
        for (int j = 0; j < BCH; j++)
            dequant_store<WF>(sb, w_row[j], w_sc[j], r.w[j], r.sc[j], WF == LX2V_WFMT_Q4 ? r.ze[j] : 0.0f);
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int i = 0; i < TM; i++) acc[j][i] = (f32x16){};

    const uint32_t frow = lane & 31, fhalf = lane >> 5;
    auto compute = [&](int buf) {
        const uint8_t *s = smem + buf * STAGE;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            bf16x8 af[TM], bfr[TN];
            const uint32_t c = kk * 2 + fhalf;
#pragma unroll
            for (int i = 0; i < TM; i++)
                af[i] = __builtin_bit_cast(bf16x8, *(const u32x4 *)(s + lds_off(wm * WM + i * 32 + frow, c)));
#pragma unroll
            for (int j = 0; j < TN; j++)
                bfr[j] = __builtin_bit_cast(
                    bf16x8, *(const u32x4 *)(s + lds_off(BM + wn * WN + j * 32 + frow, c)));
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int i = 0; i < TM; i++)
                    acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[j][i], 0, 0, 0);
        }
    };

    // Same pipeline as k_gemm_fp8: LDS buffer 0 holds stage kt, r1 stage
    // kt + 1, r0 stage kt + 2 on entry; the scheduling barriers pin the
    // load issue points.
    Regs r0, r1;
    gload(r0, 0);
    gload(r1, 1);
    sstore(r0, 0);
    __syncthreads();
    gload(r0, 2);
    for (int kt = 0; kt < KT; kt += 2) {
        compute(0);
        sstore(r1, 1);
        __syncthreads();
        gload(r1, kt + 3);
        __builtin_amdgcn_sched_barrier(0);
        compute(1);
        sstore(r0, 0);
        __syncthreads();
        gload(r0, kt + 4);
        __builtin_amdgcn_sched_barrier(0);
    }

    // Epilogue: D[n][m] blocks, four consecutive channels per register group.
    const bool vec = (N & 3) == 0;
    int mrow[TM];
#pragma unroll
    for (int i = 0; i < TM; i++) mrow[i] = m0 + wm * WM + i * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < TN; j++) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int nb = n0 + wn * WN + j * 32 + 8 * g + 4 * (lane >> 5);
            if (nb >= N) continue;
            const bool full = vec && nb + 3 < N;
            float b4[4];
            if (full) {
                f32x4 u = bias ? *(const f32x4 *)(bias + nb) : (f32x4){};
                b4[0] = u.x, b4[1] = u.y, b4[2] = u.z, b4[3] = u.w;
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) b4[q] = (nb + q < N && bias) ? bias[nb + q] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < TM; i++) {
                if (mrow[i] >= M) continue;
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    v[q] = acc[j][i][4 * g + q] + b4[q];
                    if (act == LX2V_ACT_GELU_TANH) v[q] = gelu_tanh_fast(v[q]);
                }
                TY *yp = Y + (size_t)mrow[i] * N + nb;
                if (full) {
                    store4(yp, v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        if (nb + q < N) store1(yp + q, v[q]);
                }
            }
        }
    }
}

template <int BM, int BN, int WF>
void launch_fmt(hipStream_t s, const void *x, int x_dtype, const lx2v_hip_weight *w,
                const float *bias, int act, void *y, int y_dtype, int M) {
    int N = (int)w->rows, K = (int)w->cols;
    int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    dim3 grid(tiles_m * tiles_n);
    const uint8_t *c = (const uint8_t *)w->codes;
    int g = (int)w->group;
#define LX2V_W16_LAUNCH(XT, TY)                                                                     \
    hipLaunchKernelGGL((k_gemm_w16<BM, BN, WF, XT, TY>), grid, dim3(256), 0, s, x, c, w->scales,    \
                       w->zeros, g, bias, (TY *)y, M, N, K, act, tiles_m, tiles_n)
    if (x_dtype == LX2V_DTYPE_BF16) {
        if (y_dtype == LX2V_DTYPE_BF16)
            LX2V_W16_LAUNCH(LX2V_DTYPE_BF16, uint16_t);
        else
            LX2V_W16_LAUNCH(LX2V_DTYPE_BF16, float);
    } else {
        if (y_dtype == LX2V_DTYPE_BF16)
            LX2V_W16_LAUNCH(LX2V_DTYPE_F32, uint16_t);
        else
            LX2V_W16_LAUNCH(LX2V_DTYPE_F32, float);
    }
#undef LX2V_W16_LAUNCH
}

template <int BM, int BN>
void launch_tile(hipStream_t s, const void *x, int x_dtype, const lx2v_hip_weight *w,
                 const float *bias, int act, void *y, int y_dtype, int M) {
    switch (w->fmt) {
        case LX2V_WFMT_Q8: launch_fmt<BM, BN, LX2V_WFMT_Q8>(s, x, x_dtype, w, bias, act, y, y_dtype, M); break;
        case LX2V_WFMT_Q4: launch_fmt<BM, BN, LX2V_WFMT_Q4>(s, x, x_dtype, w, bias, act, y, y_dtype, M); break;
        default: launch_fmt<BM, BN, LX2V_WFMT_FP8>(s, x, x_dtype, w, bias, act, y, y_dtype, M); break;
    }
}

}  // namespace

bool gemm_w16_supported(const lx2v_hip_weight *w) {
    size_t N = w->rows, K = w->cols, g = w->group;
    if (w->fmt != LX2V_WFMT_Q8 && w->fmt != LX2V_WFMT_Q4 && w->fmt != LX2V_WFMT_FP8) return false;
    size_t kpc = w->fmt == LX2V_WFMT_Q4 ? 32 : 16;
    return N > 0 && K >= kpc && K % kpc == 0 && g % kpc == 0 && K % g == 0 && N * K < (1ull << 31) &&
           N < (1u << 30);
}

void launch_gemm_w16(hipStream_t s, int num_cu, const void *x, int x_dtype, const lx2v_hip_weight *w,
                     const float *bias, int act, void *y, int y_dtype, size_t M) {
    size_t N = w->rows;
    struct Cfg {
        int bm, bn;
    };
    const Cfg cfgs[] = {{256, 128}, {128, 256}, {128, 128}};
    double best = -1.0;
    int pick = 0;
    for (int i = 0; i < 3; i++) {
        size_t tiles = ((M + cfgs[i].bm - 1) / cfgs[i].bm) * ((N + cfgs[i].bn - 1) / cfgs[i].bn);
        size_t waves = (tiles + num_cu - 1) / num_cu;
        double eff = (double)M * N / ((double)waves * num_cu * cfgs[i].bm * cfgs[i].bn);
        if (eff > best * 1.0001) {
            best = eff;
            pick = i;
        }
    }
    int m = (int)M;
    switch (pick) {
        case 0: launch_tile<256, 128>(s, x, x_dtype, w, bias, act, y, y_dtype, m); break;
        case 1: launch_tile<128, 256>(s, x, x_dtype, w, bias, act, y, y_dtype, m); break;
        default: launch_tile<128, 128>(s, x, x_dtype, w, bias, act, y, y_dtype, m); break;
    }
}

}  // namespace lx2v

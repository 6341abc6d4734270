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
#include <utility>

#include "gemm_common.hpp"

// Cache-policy bits of the LDS-staged epilogue's stores (buffer_store: 1 =
// sc0, 2 = nt, 16 = sc1; the values written are the same for every policy):
// sc1, as k_gemm_fp8.hip's staged epilogues (measured: Q4 FFN down and the
// native 4680 x 64 -> 1536 linear 1-10% faster, Q8 FFN up unchanged).
#ifndef LX2V_W16_CP
#define LX2V_W16_CP 16
#endif

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

// ---- direct-to-LDS kernel (bf16 activations, K a multiple of 64) --------------------
//
// Every operand of a 64-column stage travels HBM -> LDS with the 16-byte
// buffer_load ... lds into NS-slot rings: the activation tile, the weight's
// packed codes (in the reference's byte layout) and its group scales (and
// Q4 zeros) from the stage-major copy (lx2v_hip_weight::sscale).  One stage
// ahead of the contraction every thread dequantizes its 16-element units
// exactly as the reference's dequantize() and writes them, rounded to bf16,
// into a two-slot bf16 weight ring, so each weight element is decoded once
// per workgroup and the MFMAs read both operands as bf16 fragments.  With
// no load into registers in the main loop, explicit vmcnt waits carry every
// dependency (see dma16).
//
// Stage kt (one barrier):
//   wait for this wave's loads of X(kt) and of the weight stage kt + 1 (one
//   batch, issued NS - 1 stages earlier) and for its bf16 stores of kt;
//   barrier (publishes them, retires every read of kt - 1);
//   load X(kt + NS - 1) and the weight stage kt + NS into the slots kt - 1
//   and kt freed; read the fragments of kt; dequantize kt + 1 into the bf16
//   slot kt - 1 used; MFMAs.

constexpr int BKE = 64;        // K elements per stage
// Q4 with every zero 8 (lx2v_hip_weight::zero8): the same codes and scales,
// no zeros loaded (a format id of this file only)
constexpr int kWfmtQ4Sym = 100;
constexpr int XRB = BKE * 2;   // bytes per LDS tile row (bf16)

// 16 consecutive K elements of one weight row, as 8 packed bf16 pairs
// (element 2i low), each rounded from the reference's f32 dequantization
// (quant.rs:183-191, 279-289, 432-440): c = 16 code bytes (Q8, FP8) or 8
// (Q4, in c.x, c.y), s / z = the group's scale / zero.
template <int WF>
__device__ __forceinline__ void unit_dequant(u32x4 c, float s, float z, uint32_t (&o)[8]) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
    if constexpr (WF == LX2V_WFMT_Q8) {
        // byte ^ 0x80 reads as q + 128 unsigned, and fma(q + 128, s, -128 s)
        // rounds the exact q * s once (128 s is exact): the reference's q * s.
        const float nb = -128.0f * s;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t b = w[q] ^ 0x80808080u;
            const float f0 = __builtin_fmaf((float)(b & 0xFFu), s, nb);
            const float f1 = __builtin_fmaf((float)((b >> 8) & 0xFFu), s, nb);
            const float f2 = __builtin_fmaf((float)((b >> 16) & 0xFFu), s, nb);
            const float f3 = __builtin_fmaf((float)(b >> 24), s, nb);
            o[2 * q] = pack_bf16x2(f0, f1);
            o[2 * q + 1] = pack_bf16x2(f2, f3);
        }
    } else if constexpr (WF == kWfmtQ4Sym) {
        // zero 8: (c - 8) s is exact before its one rounding, and so is
        // fma(c, s, -8 s) (8 s is exact): the same f32 value
        const float nb = -8.0f * s;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const uint32_t lo = w[q] & 0x0F0F0F0Fu, hi = (w[q] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const float e0 = __builtin_fmaf((float)((lo >> (8 * b)) & 0xFFu), s, nb);
                const float e1 = __builtin_fmaf((float)((hi >> (8 * b)) & 0xFFu), s, nb);
                o[4 * q + b] = pack_bf16x2(e0, e1);
            }
        }
        (void)z;
    } else if constexpr (WF == LX2V_WFMT_Q4) {
        // element 2i in the low nibble of byte i (quant.rs:305-311)
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const uint32_t lo = w[q] & 0x0F0F0F0Fu, hi = (w[q] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const float e0 = ((float)((lo >> (8 * b)) & 0xFFu) - z) * s;
                const float e1 = ((float)((hi >> (8 * b)) & 0xFFu) - z) * s;
                o[4 * q + b] = pack_bf16x2(e0, e1);
            }
        }
    } else {
        // e4m3 through the hardware OCP decode; the reference decodes
        // exponent field 0 as m * 2^-12, an eighth of OCP's m * 2^-9.
#pragma unroll
        for (int q = 0; q < 4; q++) {
            typedef float f32x2_t __attribute__((ext_vector_type(2)));
            const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[q], false);
            const f32x2_t b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[q], true);
            float f[4] = {a.x, a.y, b.x, b.y};
            const uint32_t e = w[q] & 0x78787878u;
            if ((e - 0x01010101u) & ~e & 0x80808080u) {  // some byte has exponent field 0
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (((e >> (8 * k)) & 0xFFu) == 0) f[k] *= 0.125f;
            }
            o[2 * q] = pack_bf16x2(f[0] * s, f[1] * s);
            o[2 * q + 1] = pack_bf16x2(f[2] * s, f[3] * s);
        }
    }
}

template <int BM, int BN, int WGM, int WGN, int NS, int WF, typename TY, int KE>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void k_gemm_w16_dma(const uint16_t *__restrict__ X,
                                                                 const uint8_t *__restrict__ Wc,
                                                                 const float *__restrict__ Wss,
                                                                 const float *__restrict__ Wsz, int spr,
                                                                 const float *__restrict__ bias,
                                                                 TY *__restrict__ Y, int M, int N, int K,
                                                                 int act, int tiles_m, int tiles_n) {
    constexpr int NW = WGM * WGN, NT = 64 * NW;
    constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
    // KE K elements per stage (64, or 32 for the 256 x 256 tile, whose
    // 64-element rings would not fit the LDS); KB bytes per bf16 LDS row
    constexpr int KB = KE * 2, CPR = KB / 16, RPL = 1024 / KB, SPS = 64 / KE;
    static_assert(KE == 32 || KE == 64, "32- or 64-element K stages");
    constexpr bool Q4 = WF == LX2V_WFMT_Q4 || WF == kWfmtQ4Sym;
    constexpr bool ZL = WF == LX2V_WFMT_Q4;  // zeros loaded with the scales
    constexpr int DEN = Q4 ? 2 : 1;          // elements per code byte
    constexpr int CBS = KE / DEN;            // code bytes per weight row per stage
    constexpr int XS = BM * KB;              // activation slot
    constexpr int CS = BN * CBS;             // code slot
    constexpr int SS = BN * 16;              // scale (zero) slot: up to 4 per row (one 64-element stage's)
    constexpr int WSL = BN * KB;             // bf16 weight slot
    constexpr int RING = XS + CS + SS * (ZL ? 2 : 1);  // one stage of every ring
    constexpr int XJ = XS / 1024, CJ = CS / 1024, SJ = SS / 1024, ZJ = ZL ? SJ : 0;
    constexpr int ALD = XJ / NW;             // activation loads per wave per stage
    constexpr int EJ = CJ + SJ + ZJ;         // weight loads per stage, spread over the waves
    constexpr int EPW = (EJ + NW - 1) / NW;  // ... at most this many per wave
    constexpr int UPT = BN * (KE / 16) / NT;  // 16-element units per thread per stage
    using Ops = TileOps<BM, BN, NT>;
    static_assert(ALD * NW == XJ && CS % 1024 == 0 && SS % 1024 == 0 && UPT * NT == BN * (KE / 16),
                  "tile loads must split over the waves");
    static_assert(NS >= 2 && (NS - 1) * (ALD + EPW) < 64, "vmcnt range");
    static_assert(NS * RING + 2 * WSL + Ops::NV * 4 <= 160 * 1024, "LDS");
    static_assert(XJ % NW == 0, "activation loads split over the waves");
    static_assert((XS & (XS - 1)) == 0 && (WSL & (WSL - 1)) == 0, "slot sizes are powers of two");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * RING + 2 * WSL];
    __shared__ __attribute__((aligned(16))) float sc[Ops::NV];
    uint8_t *const xr = smem;                      // NS activation slots
    uint8_t *const cr = smem + NS * XS;            // NS code slots
    uint8_t *const sr = cr + NS * CS;              // NS scale slots
    uint8_t *const zr = sr + NS * SS;              // NS zero slots (Q4 with zeros)
    uint8_t *const wr = smem + NS * RING;          // 2 bf16 weight slots

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    const int wid_u = __builtin_amdgcn_readfirstlane(wid);  // DMA addresses and job choice (scalar)
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KT = K / KE;
    Ops ops;
    ops.load(tid, m0, n0, M, N, nullptr, nullptr, bias);

    // Rows past the matrix read zero (codes) or another row's scales: they
    // only feed outputs that are never stored.
    const uint32_t cbrow = (uint32_t)K / DEN;  // code bytes per weight row
    // bytes of one 64-element stage of scales (the stage-major copy's rows;
    // a 32-element stage loads its 64-element stage's)
    const uint32_t sstage = (uint32_t)N * (uint32_t)spr * 4u;
    const auto rx = make_rsrc(X + (size_t)m0 * K, (uint32_t)(M - m0) * (uint32_t)K * 2u);
    const auto rw = make_rsrc(Wc + (size_t)n0 * cbrow, (uint32_t)(N - n0) * cbrow);
    const auto rs = make_rsrc(Wss, (uint32_t)(KT / SPS) * sstage);
    const auto rz = make_rsrc(ZL ? Wsz : Wss, ZL ? (uint32_t)(KT / SPS) * sstage : 0u);

    // Activation load i of this wave: tile rows [(i NW + wid) RPL, +RPL),
    // lane l fills slot l % CPR of row l / CPR.
    const uint32_t lrow = (uint32_t)lane / CPR, lslot = (uint32_t)lane % CPR;
    uint32_t x_off[ALD];
#pragma unroll
    for (int i = 0; i < ALD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * RPL + lrow;
        x_off[i] = row * (uint32_t)K * 2u + dma_slot<KB>(row, lslot) * 16u;
    }
    // Weight load x of this wave: job e = x NW + wid of [CJ code KBs, SJ
    // scale KBs, ZJ zero KBs]; its lane offset without the stage term.
    uint32_t e_off[EPW];
#pragma unroll
    for (int x = 0; x < EPW; x++) {
        const int e = x * NW + wid;
        const uint32_t b = (uint32_t)(e < CJ ? e : (e < CJ + SJ ? e - CJ : e - CJ - SJ)) * 1024u + lane * 16u;
        if (e < CJ)
            e_off[x] = (b / CBS) * cbrow + b % CBS;
        else
            e_off[x] = b < (uint32_t)BN * (uint32_t)spr * 4u ? (uint32_t)n0 * (uint32_t)spr * 4u + b : kOob;
    }

    // Activation stage kt into X slot slot_x and weight stage kt + 1 into
    // code / scale slot slot_w: one batch of this wave's loads, load n of
    // which is piece(n) (n < ALD: activation rows; then this wave's weight
    // jobs, if it has one at that index).
    auto piece = [&](int n, int kt, int slot_x, int slot_w) {
        if (n < ALD) {
            const bool in_x = kt >= 0 && kt < KT;
            dma16(rx, xr + slot_x * XS + (n * NW + wid_u) * 1024,
                  in_x ? x_off[n < ALD ? n : 0] + (uint32_t)kt * KB : kOob);
            return;
        }
        const int x = n - ALD, e = x * NW + wid_u, xe = x < EPW ? x : 0;
        const int kw = kt + 1;
        const bool in = kw < KT;
        if (e < CJ) {
            dma16(rw, cr + slot_w * CS + e * 1024, in ? e_off[xe] + (uint32_t)kw * CBS : kOob);
        } else if (e < CJ + SJ) {
            dma16(rs, sr + slot_w * SS + (e - CJ) * 1024,
                  in && e_off[xe] != kOob ? e_off[xe] + (uint32_t)(kw / SPS) * sstage : kOob);
        } else if (e < EJ) {
            dma16(rz, zr + slot_w * SS + (e - CJ - SJ) * 1024,
                  in && e_off[xe] != kOob ? e_off[xe] + (uint32_t)(kw / SPS) * sstage : kOob);
        }
    };
    auto issue = [&](int kt, int slot_x, int slot_w) {
#pragma unroll
        for (int n = 0; n < ALD + EPW; n++) piece(n, kt, slot_x, slot_w);
    };
    // Weight stage kw from its code / scale slot into bf16 weight slot `ws`.
    // ... in three parts, so that a stage can spread them between its MFMAs:
    // the codes and scales into registers, the conversion, the bf16 stores.
    u32x4 dqc[UPT];
    float dqs[UPT], dqz[UPT];
    uint32_t dqo[UPT][8];
    auto dq_load = [&](int slot_w, int kw) {
        const uint8_t *cs = cr + slot_w * CS;
        const float *ss = (const float *)(sr + slot_w * SS);
        const float *zs = (const float *)(zr + slot_w * SS);
#pragma unroll
        for (int u = 0; u < UPT; u++) {
            const uint32_t id = (uint32_t)(u * NT + tid), row = id / (KE / 16), k16 = id % (KE / 16);
            if constexpr (Q4) {
                const u32x2 h = *(const u32x2 *)(cs + row * CBS + k16 * 8u);
                dqc[u] = (u32x4){h.x, h.y, 0u, 0u};
            } else {
                dqc[u] = *(const u32x4 *)(cs + row * CBS + k16 * 16u);
            }
            // the unit's 16 elements within their 64-element scale stage
            const uint32_t u64 = (uint32_t)(kw % SPS) * (KE / 16) + k16;
            const uint32_t si = row * (uint32_t)spr + ((u64 * (uint32_t)spr) >> 2);
            dqs[u] = ss[si];
            dqz[u] = ZL ? zs[si] : 0.0f;
        }
    };
    auto dq_math = [&]() {
#pragma unroll
        for (int u = 0; u < UPT; u++) unit_dequant<WF>(dqc[u], dqs[u], dqz[u], dqo[u]);
    };
    auto dq_store = [&](int ws) {
        uint8_t *d = wr + ws * WSL;
#pragma unroll
        for (int u = 0; u < UPT; u++) {
            const uint32_t id = (uint32_t)(u * NT + tid), row = id / (KE / 16), k16 = id % (KE / 16);
            const uint32_t cc = k16 * 2u;
            *(u32x4 *)(d + ((row * KB + (dma_slot<KB>(row, cc) << 4)) & (WSL - 1))) =
                (u32x4){dqo[u][0], dqo[u][1], dqo[u][2], dqo[u][3]};
            *(u32x4 *)(d + ((row * KB + (dma_slot<KB>(row, cc + 1) << 4)) & (WSL - 1))) =
                (u32x4){dqo[u][4], dqo[u][5], dqo[u][6], dqo[u][7]};
        }
    };
    auto dequant = [&](int slot_w, int ws, int kw) {
        dq_load(slot_w, kw);
        dq_math();
        dq_store(ws);
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int i = 0; i < TM; i++) acc[j][i] = (f32x16){};

    // Loads per wave per stage batch: ALD activation loads and this wave's
    // share of the weight loads (waves below EJ % NW take one more).
    const bool extra = wid_u < EJ % NW;
    const uint32_t frow = lane & 31, fhalf = lane >> 5;
    // One 16-element K slice's fragments: the wave's TM activation and TN
    // weight row blocks.
    struct Frag {
        u32x4 x[TM], w[TN];
    };
    // read_one(j, kk, f, m): fragment m (activation blocks, then weight
    // blocks) of slice kk of the stage in ring position j.
    auto read_one = [&](int j, int kk, Frag &f, int m) {
        const uint32_t c = (uint32_t)kk * 2u + fhalf;
        if (m < TM) {
            const uint8_t *xs = xr + (j % NS) * XS;
            const uint32_t row = (uint32_t)(wm * WM + m * 32) + frow;
            f.x[m] = *(const u32x4 *)(xs + ((row * KB + (dma_slot<KB>(row, c) << 4)) & (XS - 1)));
        } else {
            const uint8_t *ws = wr + (j & 1) * WSL;
            const uint32_t row = (uint32_t)(wn * WN + (m - TM) * 32) + frow;
            f.w[m - TM] = *(const u32x4 *)(ws + ((row * KB + (dma_slot<KB>(row, c) << 4)) & (WSL - 1)));
        }
    };
    // The K loop is skewed by one slice: after barrier kt a wave contracts
    // the previous stage's last slice (from registers, read before the
    // barrier) while it reads this stage's first, then each slice while
    // reading the next, so no MFMA waits for LDS after a barrier (with
    // every read of a stage issued before its first MFMA, the reads' return
    // held both waves of a SIMD off the matrix core).  fb holds the slice
    // carried across the barrier; zero before the first stage, whose
    // carried MFMAs then add +0.
    Frag fa, fb;
#pragma unroll
    for (int i = 0; i < TM; i++) fb.x[i] = (u32x4){};
#pragma unroll
    for (int jj = 0; jj < TN; jj++) fb.w[jj] = (u32x4){};
    constexpr int MPS = TN * TM, NSL = KE / 16;  // MFMAs per slice, slices per stage
    static_assert(MPS >= TM + TN && NSL % 2 == 0, "at most one fragment read per MFMA; the carried set is fb");
    // Stage kt = (multiple of U) + J, U = lcm(NS, 2): ring slots are
    // compile-time offsets.
    auto stage = [&](auto J, int kt) {
        constexpr int j = decltype(J)::value;
        constexpr int LB = ALD + EJ / NW, VM0 = (NS - 2) * LB, VM1 = (NS - 2) * (LB + 1);
        if (EJ % NW && extra)
            __builtin_amdgcn_s_waitcnt((VM1 & 15) | ((VM1 >> 4) << 14) | (7 << 4));  // lgkmcnt(0) too
        else
            __builtin_amdgcn_s_waitcnt((VM0 & 15) | ((VM0 >> 4) << 14) | (7 << 4));
        asm volatile("s_barrier" ::: "memory");
        // MFMAs: slice p - 1 of this stage (p = 0: the previous stage's last
        // slice) from one fragment set while slice p is read into the other.
        // After each of the first ALD + EPW MFMAs, one load of the batch of
        // X(kt + NS - 1) (into the slot X(kt - 1) used) and weight stage kt
        // + NS (into the slot of stage kt, dequantized in stage kt - 1):
        // issued back to back, the loads held both waves of a SIMD off the
        // MFMA pipe.  The dequantization of weight stage kt + 1 (its codes
        // landed before this stage's barrier) goes between later MFMAs: the
        // reads after MFMA DQL, the conversion after DQM (the reads have had
        // the MFMAs between to return), the stores after DQS.
        constexpr int NMF = NSL * MPS, DQL = NMF / 4, DQM = NMF / 2, DQS = 3 * NMF / 4;
        static_assert(ALD + EPW <= NMF, "a stage's loads interleave with its MFMAs");
        static_for<NSL>([&](auto P) {
            constexpr int p = decltype(P)::value;
            Frag &fc = p % 2 ? fa : fb;  // contracted (p = 0: carried)
            Frag &fn = p % 2 ? fb : fa;  // read: slice p of this stage
#pragma unroll
            for (int jj = 0; jj < TN; jj++)
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    acc[jj][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fc.w[jj]),
                                                                       __builtin_bit_cast(bf16x8, fc.x[i]),
                                                                       acc[jj][i], 0, 0, 0);
                    const int m = jj * TM + i, n = p * MPS + m;
                    __builtin_amdgcn_sched_barrier(0);
                    if (n < ALD + EPW) piece(n, kt + NS - 1, (j + NS - 1) % NS, j % NS);
                    if (n == DQL) dq_load((j + 1) % NS, kt + 1);
                    if (n == DQM) dq_math();
                    if (n == DQS) dq_store((j + 1) & 1);
                    if (m < TM + TN) read_one(j, p, fn, m);
                    __builtin_amdgcn_sched_barrier(0);
                }
        });
    };

    // Prologue: weight stage 0 alone, then as stages -NS+1 .. -1 would:
    // X(s) and weight stage s + 1 for s = 0 .. NS - 2; wait for weight
    // stage 0 (everything but those NS - 1 batches), publish it, dequantize.
    issue(-1, NS - 1, 0);  // X(-1) loads nothing (kOob)
#pragma unroll
    for (int st = 0; st < NS - 1; st++) issue(st, st, (st + 1) % NS);
    {
        constexpr int LB = ALD + EJ / NW, VM0 = (NS - 1) * LB, VM1 = (NS - 1) * (LB + 1);
        if (EJ % NW && extra)
            __builtin_amdgcn_s_waitcnt((VM1 & 15) | ((VM1 >> 4) << 14) | (7 << 4) | (15 << 8));
        else
            __builtin_amdgcn_s_waitcnt((VM0 & 15) | ((VM0 >> 4) << 14) | (7 << 4) | (15 << 8));
    }
    asm volatile("s_barrier" ::: "memory");
    dequant(0, 0, 0);
    constexpr int U = NS % 2 ? 2 * NS : NS;
    for (int kt = 0; kt < KT; kt += U) {
        static_for<U>([&](auto J) {
            if (kt + decltype(J)::value < KT) stage(J, kt + decltype(J)::value);
        });
    }
    // the last stage's last slice, from registers
#pragma unroll
    for (int jj = 0; jj < TN; jj++)
#pragma unroll
        for (int i = 0; i < TM; i++)
            acc[jj][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fb.w[jj]),
                                                               __builtin_bit_cast(bf16x8, fb.x[i]), acc[jj][i], 0,
                                                               0, 0);
    ops.park(sc, tid, m0, n0, M, N, nullptr, nullptr);
    staged_epilogue<BM, BN, NT, NS * RING + 2 * WSL, TM, TN, TY, true, -1, true, LX2V_W16_CP>(
        acc, smem, sc, wm * WM, wn * WN, tid, lane, m0, n0, M, N, act, Y);
}

template <int BM, int BN, int WGM, int WGN, int NS, int WF, int KE>
void launch_dma_fmt(hipStream_t s, const uint16_t *x, const lx2v_hip_weight *w, const float *bias, int act, void *y,
                    int y_dtype, int M) {
    const int N = (int)w->rows, K = (int)w->cols;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const dim3 grid(tiles_m * tiles_n), block(64 * WGM * WGN);
    const uint8_t *c = (const uint8_t *)w->codes;
    if (y_dtype == LX2V_DTYPE_BF16)
        hipLaunchKernelGGL((k_gemm_w16_dma<BM, BN, WGM, WGN, NS, WF, uint16_t, KE>), grid, block, 0, s, x, c, w->sscale,
                           w->szero, w->spr, bias, (uint16_t *)y, M, N, K, act, tiles_m, tiles_n);
    else
        hipLaunchKernelGGL((k_gemm_w16_dma<BM, BN, WGM, WGN, NS, WF, float, KE>), grid, block, 0, s, x, c, w->sscale,
                           w->szero, w->spr, bias, (float *)y, M, N, K, act, tiles_m, tiles_n);
}

template <int BM, int BN, int WGM, int WGN, int NS, int KE = 64>
void launch_dma_cfg(hipStream_t s, const uint16_t *x, const lx2v_hip_weight *w, const float *bias, int act, void *y,
                    int y_dtype, int M) {
    switch (w->fmt) {
        case LX2V_WFMT_Q8:
            launch_dma_fmt<BM, BN, WGM, WGN, NS, LX2V_WFMT_Q8, KE>(s, x, w, bias, act, y, y_dtype, M);
            break;
        case LX2V_WFMT_Q4:
            if (w->zero8)
                launch_dma_fmt<BM, BN, WGM, WGN, NS, kWfmtQ4Sym, KE>(s, x, w, bias, act, y, y_dtype, M);
            else
                launch_dma_fmt<BM, BN, WGM, WGN, NS, LX2V_WFMT_Q4, KE>(s, x, w, bias, act, y, y_dtype, M);
            break;
        default:
            launch_dma_fmt<BM, BN, WGM, WGN, NS, LX2V_WFMT_FP8, KE>(s, x, w, bias, act, y, y_dtype, M);
            break;
    }
}

// Direct-to-LDS configurations: tile, waves, ring depth (one workgroup per CU).
struct DmaCfg {
    int bm, bn, wgm, wgn, ns;
};
constexpr DmaCfg kDmaW16[] = {
    {256, 128, 4, 2, 3},
    {128, 256, 2, 4, 2},
    {256, 256, 4, 2, 4},  // 32-element K stages: half the activation bytes per MFMA of the 256 x 128 tile
};
constexpr int kNumDmaW16 = sizeof(kDmaW16) / sizeof(kDmaW16[0]);

void launch_dma_idx(int idx, hipStream_t s, const uint16_t *x, const lx2v_hip_weight *w, const float *bias, int act,
                    void *y, int y_dtype, int M) {
    switch (idx) {
        case 0: launch_dma_cfg<256, 128, 4, 2, 3>(s, x, w, bias, act, y, y_dtype, M); break;
        case 1: launch_dma_cfg<128, 256, 2, 4, 2>(s, x, w, bias, act, y, y_dtype, M); break;
        default: launch_dma_cfg<256, 256, 4, 2, 4, 32>(s, x, w, bias, act, y, y_dtype, M); break;
    }
}

// LIGHTX2V_HIP_W16_CFG=<index> forces a configuration (for sweeps and
// tests; read on every plan).
int forced_w16_cfg() {
    const char *e = getenv("LIGHTX2V_HIP_W16_CFG");
    if (!e || !*e) return -1;
    const int i = atoi(e);
    return (i >= 0 && i < kNumDmaW16) ? i : -1;
}

// ---- bf16 x bf16: native f32 weights rounded to bf16 at upload ------------------
//
// Backend::weight's f32 weights (WeightQuant::Native, quant.rs:28-30) on
// the bf16 MFMA: the weight's bf16 copy (RNE from f32, made once at upload)
// and the bf16 activations both travel HBM -> LDS by the 16-byte
// buffer_load ... lds into an NS-stage ring of 64-element K stages, laid
// out and read like k_gemm_w16_dma's activation tiles; four 32x32x16 MFMAs
// per block per stage; the staged epilogue adds the bias and applies GELU.
template <int BM, int BN, int WGM, int WGN, int NS, typename TY>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void k_gemm_bf16_dma(const uint16_t *__restrict__ X,
                                                                  const uint16_t *__restrict__ W,
                                                                  const float *__restrict__ bias,
                                                                  TY *__restrict__ Y, int M, int N, int K, int act,
                                                                  int tiles_m, int tiles_n) {
    constexpr int NW = WGM * WGN, NT = 64 * NW;
    constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
    constexpr int XS = BM * XRB, WS = BN * XRB, STAGE = XS + WS;
    constexpr int ALD = BM / 8 / NW, BLD = BN / 8 / NW, LPS = ALD + BLD;
    using Ops = TileOps<BM, BN, NT>;
    static_assert(ALD * 8 * NW == BM && BLD * 8 * NW == BN, "tile rows must split over the waves");
    static_assert(NS >= 2 && (NS - 2) * LPS < 64, "vmcnt range");
    static_assert(NS * STAGE + Ops::NV * 4 <= 160 * 1024, "LDS");
    static_assert((XS & (XS - 1)) == 0 && (WS & (WS - 1)) == 0, "slot sizes are powers of two");
    static_assert(4 * TN * TM >= LPS, "a stage's loads interleave with its MFMAs");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE];
    __shared__ __attribute__((aligned(16))) float sc[Ops::NV];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    const int wid_u = __builtin_amdgcn_readfirstlane(wid);
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KT = K / BKE;
    Ops ops;
    ops.load(tid, m0, n0, M, N, nullptr, nullptr, bias);

    // Rows past either matrix read zero: they feed outputs that are never stored.
    const auto rx = make_rsrc(X + (size_t)m0 * K, (uint32_t)(M - m0) * (uint32_t)K * 2u);
    const auto rw = make_rsrc(W + (size_t)n0 * K, (uint32_t)(N - n0) * (uint32_t)K * 2u);
    // Load i of this wave covers tile rows [(i NW + wid) 8, +8); lane l
    // fills slot l % 8 of row l / 8 with the chunk the swizzle puts there.
    const uint32_t lrow = (uint32_t)lane / 8u, lslot = (uint32_t)lane % 8u;
    uint32_t x_off[ALD], w_off[BLD];
#pragma unroll
    for (int i = 0; i < ALD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * 8u + lrow;
        x_off[i] = row * (uint32_t)K * 2u + dma_slot<XRB>(row, lslot) * 16u;
    }
#pragma unroll
    for (int i = 0; i < BLD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * 8u + lrow;
        w_off[i] = row * (uint32_t)K * 2u + dma_slot<XRB>(row, lslot) * 16u;
    }
    auto piece = [&](int n, int kt, int buf) {
        const bool in = kt < KT;
        uint8_t *sb = smem + buf * STAGE;
        if (n < ALD)
            dma16(rx, sb + (n * NW + wid_u) * 1024, in ? x_off[n < ALD ? n : 0] + (uint32_t)kt * XRB : kOob);
        else
            dma16(rw, sb + XS + ((n - ALD) * NW + wid_u) * 1024,
                  in ? w_off[n >= ALD ? n - ALD : 0] + (uint32_t)kt * XRB : kOob);
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int i = 0; i < TM; i++) acc[j][i] = (f32x16){};
    // One stage's MFMAs from slot buf, the loads of stage dkt (slot dbuf)
    // one after each of its first MFMAs.  Lanes 0..31 supply K elements
    // 8 c .. 8 c + 7 of their row, lanes 32..63 the next 8 (chunk 2 kk + h).
    const uint32_t frow = lane & 31, fhalf = lane >> 5;
    auto compute = [&](int buf, int dkt, int dbuf) {
        const uint8_t *xs = smem + buf * STAGE, *ws = xs + XS;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const uint32_t c = (uint32_t)kk * 2u + fhalf;
            u32x4 xf[TM], wf[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint32_t row = (uint32_t)(wm * WM + i * 32) + frow;
                xf[i] = *(const u32x4 *)(xs + ((row * XRB + (dma_slot<XRB>(row, c) << 4)) & (XS - 1)));
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint32_t row = (uint32_t)(wn * WN + j * 32) + frow;
                wf[j] = *(const u32x4 *)(ws + ((row * XRB + (dma_slot<XRB>(row, c) << 4)) & (WS - 1)));
            }
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wf[j]),
                                                                      __builtin_bit_cast(bf16x8, xf[i]), acc[j][i],
                                                                      0, 0, 0);
                    const int n = (kk * TN + j) * TM + i;
                    if (n < LPS) {
                        __builtin_amdgcn_sched_barrier(0);
                        piece(n, dkt, dbuf);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
        }
    };
    // Entering stage kt: stages kt .. kt + NS - 2 are in flight, so waiting
    // until NS - 2 stages' loads remain leaves stage kt complete for this
    // wave; the barrier publishes every wave's part and retires the reads
    // of stage kt - 1, whose slot this stage's loads refill.
#pragma unroll
    for (int st = 0; st < NS - 1; st++)
#pragma unroll
        for (int n = 0; n < LPS; n++) piece(n, st, st);
    for (int kt = 0; kt < KT; kt += NS) {
#pragma unroll
        for (int j = 0; j < NS; j++) {
            if (kt + j < KT) {
                wait_vmcnt<(NS - 2) * LPS>();
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                compute(j, kt + j + NS - 1, (j + NS - 1) % NS);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    ops.park(sc, tid, m0, n0, M, N, nullptr, nullptr);
    staged_epilogue<BM, BN, NT, NS * STAGE, TM, TN, TY, true, -1, true, LX2V_W16_CP>(
        acc, smem, sc, wm * WM, wn * WN, tid, lane, m0, n0, M, N, act, Y);
}

template <int BM, int BN, int WGM, int WGN, int NS>
void launch_bf16_cfg(hipStream_t s, const uint16_t *x, const uint16_t *w, const float *bias, int act, void *y,
                     int y_dtype, int M, int N, int K) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const dim3 grid(tiles_m * tiles_n), block(64 * WGM * WGN);
    if (y_dtype == LX2V_DTYPE_BF16)
        hipLaunchKernelGGL((k_gemm_bf16_dma<BM, BN, WGM, WGN, NS, uint16_t>), grid, block, 0, s, x, w, bias,
                           (uint16_t *)y, M, N, K, act, tiles_m, tiles_n);
    else
        hipLaunchKernelGGL((k_gemm_bf16_dma<BM, BN, WGM, WGN, NS, float>), grid, block, 0, s, x, w, bias, (float *)y,
                           M, N, K, act, tiles_m, tiles_n);
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

bool gemm_w16_dma_supported(const lx2v_hip_weight *w, size_t M) {
    const size_t N = w->rows, K = w->cols, g = w->group;
    if (w->fmt != LX2V_WFMT_Q8 && w->fmt != LX2V_WFMT_Q4 && w->fmt != LX2V_WFMT_FP8) return false;
    const size_t cb = w->fmt == LX2V_WFMT_Q4 ? K / 2 : K;
    return w->sscale && M > 0 && N > 0 && K >= BKE && K % BKE == 0 && g % 16 == 0 && K % g == 0 &&
           M * K * 2 < (1ull << 31) && N * cb < (1ull << 31) && (K / BKE) * N * (size_t)w->spr * 4 < (1ull << 31) &&
           M < (1u << 30) && N < (1u << 30);
}

// Fill efficiency of each configuration (useful tiles over tile slots of
// the rounds the grid takes), the larger workgroup tile on ties (it moves
// fewer activation bytes per MFMA: Q8 4680 x 1536 -> 8960 takes 159 us on
// the 256 x 256 tile against 184 on 256 x 128, at the same fill).
int plan_gemm_w16_dma(int num_cu, size_t M, size_t N) {
    if (forced_w16_cfg() >= 0) return forced_w16_cfg();
    double best = -1.0;
    int pick = 0;
    for (int i = 0; i < kNumDmaW16; i++) {
        const DmaCfg &c = kDmaW16[i];
        const size_t tiles = ((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
        const size_t slots = (size_t)num_cu;
        const size_t rounds = (tiles + slots - 1) / slots;
        const double eff = (double)M * N / ((double)rounds * slots * c.bm * c.bn);
        const bool tie = eff <= best * 1.0001 && eff >= best * 0.9999;
        if (eff > best * 1.0001 || (tie && c.bm * c.bn > kDmaW16[pick].bm * kDmaW16[pick].bn)) {
            best = eff;
            pick = i;
        }
    }
    return pick;
}

void launch_gemm_w16_dma(hipStream_t s, int cfg, const uint16_t *x, const lx2v_hip_weight *w, const float *bias,
                         int act, void *y, int y_dtype, size_t M) {
    launch_dma_idx(cfg, s, x, w, bias, act, y, y_dtype, (int)M);
}

bool gemm_bf16_supported(size_t M, size_t N, size_t K) {
    return M > 0 && N > 0 && K >= BKE && K % BKE == 0 && M * K * 2 < (1ull << 31) && N * K * 2 < (1ull << 31) &&
           M < (1u << 30) && N < (1u << 30);
}

// 256 x 128 (8 waves), 128 x 256 (8 waves) or 128 x 128 (4 waves): the one
// that leaves the fewest idle tile slots over the rounds the grid takes, the
// larger tile on ties.
void launch_gemm_bf16(hipStream_t s, int num_cu, const uint16_t *x, const uint16_t *w, const float *bias, int act,
                      void *y, int y_dtype, size_t M, size_t N, size_t K) {
    struct Cfg {
        int bm, bn;
    };
    const Cfg cfgs[] = {{256, 128}, {128, 256}, {128, 128}};
    double best = -1.0;
    int pick = 0;
    for (int i = 0; i < 3; i++) {
        const size_t tiles = ((M + cfgs[i].bm - 1) / cfgs[i].bm) * ((N + cfgs[i].bn - 1) / cfgs[i].bn);
        const size_t rounds = (tiles + num_cu - 1) / num_cu;
        const double eff = (double)M * N / ((double)rounds * num_cu * cfgs[i].bm * cfgs[i].bn);
        if (eff > best * 1.0001) {
            best = eff;
            pick = i;
        }
    }
    const int m = (int)M, n = (int)N, k = (int)K;
    switch (pick) {
        case 0: launch_bf16_cfg<256, 128, 4, 2, 3>(s, x, w, bias, act, y, y_dtype, m, n, k); break;
        case 1: launch_bf16_cfg<128, 256, 2, 4, 3>(s, x, w, bias, act, y, y_dtype, m, n, k); break;
        default: launch_bf16_cfg<128, 128, 2, 2, 3>(s, x, w, bias, act, y, y_dtype, m, n, k); break;
    }
}

}  // namespace lx2v

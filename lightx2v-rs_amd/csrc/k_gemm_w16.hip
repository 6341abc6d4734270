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
// Tile shape, swizzle and XCD mapping follow k_gemm_fp8.hip with a 64-
// element K stage (128 bytes of bf16 per row).
#include "device_common.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

constexpr int BK = 64;        // K elements per stage
constexpr int ROWB = BK * 2;  // bytes per LDS tile row (bf16)

__device__ __forceinline__ uint32_t lds_off(uint32_t row, uint32_t c) {
    return row * ROWB + ((c ^ ((row >> 1) & 7u)) << 4);
}

__device__ __forceinline__ void tile_of(int bid, int nb, int tiles_m, int tiles_n, int *tm, int *tn) {
    const int per = nb / 8, rem = nb % 8;
    const int x = bid % 8, j = bid / 8;
    const int id = x * per + (x < rem ? x : rem) + j;
    const int G = tiles_m < 4 ? tiles_m : 4;
    const int group = id / (G * tiles_n);
    const int first = group * G;
    const int gsz = (tiles_m - first) < G ? (tiles_m - first) : G;
    const int in = id - first * tiles_n;
    *tm = first + in % gsz;
    *tn = in / gsz;
}

template <typename TY>
__device__ __forceinline__ void store_y(TY *y, size_t idx, float v);
template <>
__device__ __forceinline__ void store_y<float>(float *y, size_t idx, float v) {
    y[idx] = v;
}
template <>
__device__ __forceinline__ void store_y<uint16_t>(uint16_t *y, size_t idx, float v) {
    y[idx] = f32_to_bf16_bits(v);
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
    constexpr int ACH = BM * 8 / 256;                     // LDS chunks of A per thread
    constexpr int CPR = WTraits<WF>::kChunksPerRow;
    constexpr int KPC = WTraits<WF>::kPerChunk;
    constexpr int BCH = BN * CPR / 256;                   // weight source chunks per thread
    constexpr int WB_NUM = WF == LX2V_WFMT_Q4 ? 1 : 1;
    constexpr int WB_DEN = WF == LX2V_WFMT_Q4 ? 2 : 1;    // code bytes per element = NUM/DEN
    static_assert(BCH >= 1, "tile too small for the weight loader");
    constexpr int STAGE = (BM + BN) * ROWB;
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KG = K / group;  // scale columns

    const auto rx = make_rsrc((const uint8_t *)X + (size_t)m0 * K * XB, (uint32_t)(M - m0) * (uint32_t)K * XB);
    const uint32_t wrow_bytes = (uint32_t)K * WB_NUM / WB_DEN;
    const auto rw = make_rsrc(Wc + (size_t)n0 * wrow_bytes, (uint32_t)(N - n0) * wrow_bytes);

    // A chunk coordinates: LDS chunk c of row r holds K elements [8c, 8c+8).
    uint32_t a_goff[ACH], a_loff[ACH], a_kc[ACH];
#pragma unroll
    for (int j = 0; j < ACH; j++) {
        uint32_t id = j * 256 + tid, row = id >> 3, c = id & 7;
        a_goff[j] = (row * (uint32_t)K + c * 8) * XB;
        a_loff[j] = lds_off(row, c);
        a_kc[j] = c * 8;
    }
    // Weight source chunk coordinates.
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

    u32x4 ra[ACH][XLD], rw_[BCH];
    float wsc[BCH], wze[BCH];
    auto gload = [&](int k0) {
#pragma unroll
        for (int j = 0; j < ACH; j++) {
            bool kin = (uint32_t)k0 + a_kc[j] < (uint32_t)K;
#pragma unroll
            for (int h = 0; h < XLD; h++)
                ra[j][h] = buffer_load_x4(rx, kin ? a_goff[j] + (uint32_t)k0 * XB + h * 16 : kOob);
        }
#pragma unroll
        for (int j = 0; j < BCH; j++) {
            uint32_t kk = (uint32_t)k0 + w_sc[j] * KPC;
            bool kin = kk < (uint32_t)K;
            rw_[j] = buffer_load_x4(rw, kin ? w_goff[j] + (uint32_t)k0 * WB_NUM / WB_DEN : kOob);
            uint32_t g = w_srow[j] + (kin ? kk : 0) / (uint32_t)group;
            wsc[j] = Ws[g];
            if (WF == LX2V_WFMT_Q4) wze[j] = Wz[g];
        }
    };
    auto sstore = [&](int buf) {
        uint8_t *s = smem + buf * STAGE;
#pragma unroll
        for (int j = 0; j < ACH; j++) {
            u32x4 o;
            if (XT == LX2V_DTYPE_BF16) {
                o = ra[j][0];
            } else {
                f32x4 lo = __builtin_bit_cast(f32x4, ra[j][0]);
                f32x4 hi = __builtin_bit_cast(f32x4, ra[j][1]);
                o.x = pack_bf16x2(lo.x, lo.y);
                o.y = pack_bf16x2(lo.z, lo.w);
                o.z = pack_bf16x2(hi.x, hi.y);
                o.w = pack_bf16x2(hi.z, hi.w);
            }
            *(u32x4 *)(s + a_loff[j]) = o;
        }
        uint8_t *sb = s + BM * ROWB;
#pragma unroll
        for (int j = 0; j < BCH; j++)
            dequant_store<WF>(sb, w_row[j], w_sc[j], rw_[j], wsc[j], WF == LX2V_WFMT_Q4 ? wze[j] : 0.0f);
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (f32x16){};

    const uint32_t frow = lane & 31, fhalf = lane >> 5;
    const int KT = (K + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * BK);
        const uint8_t *s = smem + cur * STAGE;
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
                    bf16x8, *(const u32x4 *)(s + BM * ROWB + lds_off(wn * WN + j * 32 + frow, c)));
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

    float bn[TN];
    int ncol[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        int n = n0 + wn * WN + j * 32 + (lane & 31);
        ncol[j] = n;
        bn[j] = (n < N && bias) ? bias[n] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if (ncol[j] >= N) continue;
                float v = acc[i][j][r] + bn[j];
                if (act == LX2V_ACT_GELU_TANH) v = gelu_tanh(v);
                store_y<TY>(Y, (size_t)m * N + ncol[j], v);
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
    const Cfg cfgs[] = {{256, 256}, {256, 128}, {128, 256}, {128, 128}};
    double best = -1.0;
    int pick = 0;
    for (int i = 0; i < 4; i++) {
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
        case 0: launch_tile<256, 256>(s, x, x_dtype, w, bias, act, y, y_dtype, m); break;
        case 1: launch_tile<256, 128>(s, x, x_dtype, w, bias, act, y, y_dtype, m); break;
        case 2: launch_tile<128, 256>(s, x, x_dtype, w, bias, act, y, y_dtype, m); break;
        default: launch_tile<128, 128>(s, x, x_dtype, w, bias, act, y, y_dtype, m); break;
    }
}

}  // namespace lx2v

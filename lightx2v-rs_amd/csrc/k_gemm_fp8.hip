// k_gemm_fp8.hip -- FP8-e4m3 weight x per-token e4m3 activation GEMM on the
// gfx950 fp8 MFMA (v_mfma_f32_32x32x64_f8f6f4), for weights with one scale
// per output channel (Fp8E4M3 with group == cols, quant.rs:364-373,
// 425-429).
//
//   Y[m, n] = act( (sum_k e4m3(A[m,k]) * e4m3(B[n,k])) * sa[m] * sb[n] + bias[n] )
//
// A = per-token quantized activations [M, K], B = the weight's e4m3 codes
// [N, K] exactly as the reference lays them out (row-major, K contiguous);
// both are "K-major", which is the layout the MFMA operands want, so codes
// go from HBM to LDS to the matrix cores untouched.
//
// Work decomposition: one workgroup (4 waves, 2x2) per BM x BN output tile,
// K stepped 128 bytes at a time through a double-buffered LDS stage with an
// XOR swizzle on 16-byte chunks; each wave owns a (BM/2) x (BN/2) sub-tile of
// 32x32 MFMA blocks whose accumulators stay in registers for the whole K
// loop; the epilogue applies both scales, bias, GELU and the store.
#include "device_common.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

constexpr int BK = 128;  // bytes (= e4m3 elements) of K per LDS stage

// 16-byte chunk `c` (0..7) of tile row `row` lives at this LDS byte offset.
__device__ __forceinline__ uint32_t lds_off(uint32_t row, uint32_t c) {
    return row * BK + ((c ^ ((row >> 1) & 7u)) << 4);
}

// Map a linear workgroup id to an output tile so that the workgroups one
// XCD runs (ids congruent mod 8 are dispatched to the same XCD) form a
// compact block of tiles sharing A rows and B columns in that XCD's L2.
__device__ __forceinline__ void tile_of(int bid, int nb, int tiles_m, int tiles_n, int *tm, int *tn) {
    const int per = nb / 8, rem = nb % 8;
    const int x = bid % 8, j = bid / 8;
    const int id = x * per + (x < rem ? x : rem) + j;
    const int G = tiles_m < 4 ? tiles_m : 4;  // tile-rows per group
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

template <int BM, int BN, typename TY>
__global__ __launch_bounds__(256, 1) void k_gemm_fp8(const uint8_t *__restrict__ A,
                                                     const float *__restrict__ sa,
                                                     const uint8_t *__restrict__ B,
                                                     const float *__restrict__ sb,
                                                     const float *__restrict__ bias, TY *__restrict__ Y,
                                                     int M, int N, int K, int act, int tiles_m,
                                                     int tiles_n) {
    constexpr int WM = BM / 2, WN = BN / 2;     // wave sub-tile
    constexpr int TM = WM / 32, TN = WN / 32;   // 32x32 MFMA blocks per wave
    constexpr int ACH = BM * BK / 16 / 256;     // 16-byte chunks per thread per stage
    constexpr int BCH = BN * BK / 16 / 256;
    constexpr int STAGE = (BM + BN) * BK;
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const uint32_t a_bytes = (uint32_t)(M - m0) * (uint32_t)K;
    const uint32_t b_bytes = (uint32_t)(N - n0) * (uint32_t)K;
    const auto ra_src = make_rsrc(A + (size_t)m0 * K, a_bytes);
    const auto rb_src = make_rsrc(B + (size_t)n0 * K, b_bytes);

    // Per-thread chunk coordinates (fixed across the K loop).
    uint32_t a_goff[ACH], a_loff[ACH], b_goff[BCH], b_loff[BCH];
#pragma unroll
    for (int j = 0; j < ACH; j++) {
        uint32_t id = j * 256 + tid, row = id >> 3, c = id & 7;
        a_goff[j] = row * (uint32_t)K + c * 16;
        a_loff[j] = lds_off(row, c);
    }
#pragma unroll
    for (int j = 0; j < BCH; j++) {
        uint32_t id = j * 256 + tid, row = id >> 3, c = id & 7;
        b_goff[j] = row * (uint32_t)K + c * 16;
        b_loff[j] = BM * BK + lds_off(row, c);
    }

    // Every chunk of this thread sits at the same column (tid & 7) * 16 of
    // its row, so one compare masks the ragged last K stage (a chunk past
    // K would otherwise read the start of the next row).
    const uint32_t kcol = (uint32_t)(tid & 7) * 16;
    u32x4 ra[ACH], rb[BCH];
    auto gload = [&](int k0) {
        const bool kin = (uint32_t)k0 + kcol < (uint32_t)K;
#pragma unroll
        for (int j = 0; j < ACH; j++) ra[j] = buffer_load_x4(ra_src, kin ? a_goff[j] + k0 : kOob);
#pragma unroll
        for (int j = 0; j < BCH; j++) rb[j] = buffer_load_x4(rb_src, kin ? b_goff[j] + k0 : kOob);
    };
    auto sstore = [&](int buf) {
        uint8_t *s = smem + buf * STAGE;
#pragma unroll
        for (int j = 0; j < ACH; j++) *(u32x4 *)(s + a_loff[j]) = ra[j];
#pragma unroll
        for (int j = 0; j < BCH; j++) *(u32x4 *)(s + b_loff[j]) = rb[j];
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (f32x16){};

    // Fragment rows / chunk halves of this lane.
    const uint32_t frow = lane & 31, fhalf = (lane >> 5) * 2;

    const int KT = (K + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * BK);
        const uint8_t *s = smem + cur * STAGE;
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            i32x8 af[TM], bf[TN];
            const uint32_t c0 = kk * 4 + fhalf;
#pragma unroll
            for (int i = 0; i < TM; i++) {
                uint32_t row = wm * WM + i * 32 + frow;
                u32x4 lo = *(const u32x4 *)(s + lds_off(row, c0));
                u32x4 hi = *(const u32x4 *)(s + lds_off(row, c0 + 1));
                af[i] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                uint32_t row = wn * WN + j * 32 + frow;
                u32x4 lo = *(const u32x4 *)(s + BM * BK + lds_off(row, c0));
                u32x4 hi = *(const u32x4 *)(s + BM * BK + lds_off(row, c0 + 1));
                bf[j] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        af[i], bf[j], acc[i][j], 0, 0, 0, 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

    // Epilogue.  D layout of a 32x32 MFMA block: lane l holds column l%32,
    // rows 8*(r/4) + 4*(l/32) + r%4 for r = 0..15.
    float sbn[TN], bn[TN];
    int ncol[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        int n = n0 + wn * WN + j * 32 + (lane & 31);
        ncol[j] = n;
        bool ok = n < N;
        sbn[j] = ok ? sb[n] : 0.0f;
        bn[j] = (ok && bias) ? bias[n] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m >= M) continue;
            float sam = sa[m];
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if (ncol[j] >= N) continue;
                float v = acc[i][j][r] * sam * sbn[j] + bn[j];
                if (act == LX2V_ACT_GELU_TANH) v = gelu_tanh(v);
                store_y<TY>(Y, (size_t)m * N + ncol[j], v);
            }
        }
    }
}

template <int BM, int BN>
void launch_cfg(hipStream_t s, const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
                const float *bias, int act, void *y, int y_dtype, int M, int N, int K) {
    int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    dim3 grid(tiles_m * tiles_n);
    if (y_dtype == LX2V_DTYPE_BF16)
        hipLaunchKernelGGL((k_gemm_fp8<BM, BN, uint16_t>), grid, dim3(256), 0, s, a, sa, b, sb, bias,
                           (uint16_t *)y, M, N, K, act, tiles_m, tiles_n);
    else
        hipLaunchKernelGGL((k_gemm_fp8<BM, BN, float>), grid, dim3(256), 0, s, a, sa, b, sb, bias,
                           (float *)y, M, N, K, act, tiles_m, tiles_n);
}

}  // namespace

bool gemm_fp8_supported(size_t M, size_t N, size_t K) {
    // 32-bit buffer offsets; K a multiple of 16 (the 16-byte chunk loads).
    return M > 0 && N > 0 && K >= 16 && K % 16 == 0 && M * K < (1ull << 31) &&
           N * K < (1ull << 31) && M < (1u << 30) && N < (1u << 30);
}

void launch_gemm_fp8(hipStream_t s, int num_cu, const uint8_t *a, const float *a_scale,
                     const uint8_t *b, const float *b_scale, const float *bias, int act, void *y,
                     int y_dtype, size_t M, size_t N, size_t K) {
    // Pick the tile that fills the chip best: fraction of issued MFMA work
    // that is useful, over whole waves of workgroups; ties go to the larger
    // tile (more reuse per LDS byte).
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
    int m = (int)M, n = (int)N, k = (int)K;
    switch (pick) {
        case 0: launch_cfg<256, 256>(s, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k); break;
        case 1: launch_cfg<256, 128>(s, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k); break;
        case 2: launch_cfg<128, 256>(s, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k); break;
        default: launch_cfg<128, 128>(s, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k); break;
    }
}

}  // namespace lx2v

// k_gemm_fp8.hip -- FP8-e4m3 weight x per-token e4m3 activation GEMM on the
// gfx950 fp8 MFMA (v_mfma_f32_32x32x64_f8f6f4), for weights with one scale
// per output channel (Fp8E4M3 with group == cols, quant.rs:364-373,
// 425-429).
//
//   Y[m, n] = act( (sum_k e4m3(A[m,k]) * e4m3(B[n,k])) * sa[m] * sb[n] + bias[n] )
//
// A = per-token quantized activations [M, K], B = the weight's e4m3 codes
// [N, K] exactly as the reference lays them out (row-major, K contiguous);
// both are K-major, the layout the MFMA operands want, so codes go from HBM
// to LDS to the matrix cores untouched.
//
// Work decomposition.  One workgroup (4 waves, 2 x 2) per BM x BN output
// tile; each wave owns a (BM/2) x (BN/2) sub-tile of 32 x 32 MFMA blocks
// whose accumulators stay in AGPRs for the whole K loop.  K advances 128
// bytes per stage through two LDS buffers (16-byte chunks XOR-swizzled so
// the fragment reads are bank-conflict free) fed from two register stages:
// the global loads of stage k+2 are in flight while stage k is contracted
// and stage k+1 waits in registers, which gives the loads two stages of
// MFMA time to arrive.
//
// Operand roles: the weight tile is the MFMA's A operand and the activation
// tile its B operand, so the 32 x 32 result block D[n][m] leaves each lane
// one activation row m and, per group of four accumulator registers, four
// consecutive output channels n -- the epilogue applies both scales, bias
// and GELU and writes those four outputs with one 16-byte (f32) or 8-byte
// (bf16) store.
#include "device_common.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

constexpr int BK = 128;  // bytes (= e4m3 elements) of K per stage

// 16-byte chunk `c` (0..7) of tile row `row` lives at this LDS byte offset.
__device__ __forceinline__ uint32_t lds_off(uint32_t row, uint32_t c) {
    return row * BK + ((c ^ ((row >> 1) & 7u)) << 4);
}

// Epilogue shared by both fp8 kernels.  Block D[n][m] (32 x 32) of
// acc[j][i]: lane l holds m = mbase + 32 i + l % 32 and, in registers
// 4g .. 4g+3, n = nbase + 32 j + 8g + 4 (l / 32) + 0..3.  Applies the token
// scale, channel scale and bias, then GELU, and stores four channels at once
// where the row stays 16-byte aligned (N % 4 == 0).
template <int TM, int TN, typename TY>
__device__ __forceinline__ void epilogue_fp8(const f32x16 (&acc)[TN][TM], int mbase, int nbase, int lane, int M,
                                             int N, const float *__restrict__ sa,
                                             const float *__restrict__ sb,
                                             const float *__restrict__ bias, int act, TY *__restrict__ Y) {
    const bool vec = (N & 3) == 0;
    float sam[TM];
    int mrow[TM];
#pragma unroll
    for (int i = 0; i < TM; i++) {
        mrow[i] = mbase + i * 32 + (lane & 31);
        sam[i] = mrow[i] < M ? sa[mrow[i]] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int nb = nbase + j * 32 + 8 * g + 4 * (lane >> 5);
            if (nb >= N) continue;
            const bool full = vec && nb + 3 < N;
            float s4[4], b4[4];
            if (full) {
                f32x4 t = *(const f32x4 *)(sb + nb);
                s4[0] = t.x, s4[1] = t.y, s4[2] = t.z, s4[3] = t.w;
                f32x4 u = bias ? *(const f32x4 *)(bias + nb) : (f32x4){};
                b4[0] = u.x, b4[1] = u.y, b4[2] = u.z, b4[3] = u.w;
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    bool ok = nb + q < N;
                    s4[q] = ok ? sb[nb + q] : 0.0f;
                    b4[q] = (ok && bias) ? bias[nb + q] : 0.0f;
                }
            }
#pragma unroll
            for (int i = 0; i < TM; i++) {
                if (mrow[i] >= M) continue;
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    v[q] = acc[j][i][4 * g + q] * sam[i] * s4[q] + b4[q];
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

// ---- register-staged kernel (any K that is a multiple of 16) ----------------------

template <int BM, int BN, typename TY>
__global__ __launch_bounds__(256, 1) void k_gemm_fp8(const uint8_t *__restrict__ A,
                                                     const float *__restrict__ sa,
                                                     const uint8_t *__restrict__ B,
                                                     const float *__restrict__ sb,
                                                     const float *__restrict__ bias, TY *__restrict__ Y,
                                                     int M, int N, int K, int act, int tiles_m,
                                                     int tiles_n) {
    constexpr int WM = BM / 2, WN = BN / 2;     // wave sub-tile (activation rows, channels)
    constexpr int TM = WM / 32, TN = WN / 32;   // 32x32 MFMA blocks per wave
    constexpr int ACH = BM * BK / 16 / 256;     // 16-byte chunks per thread per stage
    constexpr int BCH = BN * BK / 16 / 256;
    constexpr int STAGE = (BM + BN) * BK;
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;

    // Loads past a matrix's last row read zero (buffer range check).
    const auto ra_src = make_rsrc(A + (size_t)m0 * K, (uint32_t)(M - m0) * (uint32_t)K);
    const auto rb_src = make_rsrc(B + (size_t)n0 * K, (uint32_t)(N - n0) * (uint32_t)K);

    // Chunk j of this thread: tile row j * 32 + tid / 8, chunk tid % 8.  The
    // swizzle depends on row bits 1..3 only, so every j shares one LDS
    // offset up to j * 32 rows.
    const uint32_t crow = (uint32_t)tid >> 3, cc = (uint32_t)tid & 7u;
    const uint32_t g_base = crow * (uint32_t)K + cc * 16;
    const uint32_t g_step = 32u * (uint32_t)K;
    const uint32_t l_base = lds_off(crow, cc);
    const uint32_t kcol = cc * 16;
    const int KT = (K + BK - 1) / BK;

    // Stage `kt` into registers; stages past the end (and the ragged K tail
    // of a 16-byte chunk column) load zeros.
    auto gload = [&](u32x4(&ra)[ACH], u32x4(&rb)[BCH], int kt) {
        const uint32_t k0 = (uint32_t)kt * BK;
        const bool kin = kt < KT && k0 + kcol < (uint32_t)K;
        const uint32_t off = kin ? g_base + k0 : kOob;
#pragma unroll
        for (int j = 0; j < ACH; j++) ra[j] = buffer_load_x4(ra_src, kin ? off + j * g_step : kOob);
#pragma unroll
        for (int j = 0; j < BCH; j++) rb[j] = buffer_load_x4(rb_src, kin ? off + j * g_step : kOob);
    };
    auto sstore = [&](const u32x4(&ra)[ACH], const u32x4(&rb)[BCH], int buf) {
        uint8_t *s = smem + buf * STAGE + l_base;
#pragma unroll
        for (int j = 0; j < ACH; j++) *(u32x4 *)(s + j * 32 * BK) = ra[j];
#pragma unroll
        for (int j = 0; j < BCH; j++) *(u32x4 *)(s + (BM + j * 32) * BK) = rb[j];
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int i = 0; i < TM; i++) acc[j][i] = (f32x16){};

    // Fragment row of this lane and the chunk pair (0/1 or 2/3 of each 64-
    // byte half stage) its half-wave supplies.
    const uint32_t frow = lane & 31, fhalf = (lane >> 5) * 2;
    auto compute = [&](int buf) {
        const uint8_t *s = smem + buf * STAGE;
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            i32x8 af[TM], bf[TN];
            const uint32_t c0 = kk * 4 + fhalf;
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint32_t row = wm * WM + i * 32 + frow;
                u32x4 lo = *(const u32x4 *)(s + lds_off(row, c0));
                u32x4 hi = *(const u32x4 *)(s + lds_off(row, c0 + 1));
                af[i] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint32_t row = BM + wn * WN + j * 32 + frow;
                u32x4 lo = *(const u32x4 *)(s + lds_off(row, c0));
                u32x4 hi = *(const u32x4 *)(s + lds_off(row, c0 + 1));
                bf[j] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
            // Scale operands 0 with format 0 (e4m3) on both sides select the
            // unscaled fp8 MFMA.
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int i = 0; i < TM; i++)
                    acc[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        bf[j], af[i], acc[j][i], 0, 0, 0, 0, 0, 0);
        }
    };

    // Pipeline: two register stages (r0, r1), two LDS buffers.  Entering
    // an iteration: LDS buffer 0 holds stage kt, r1 stage kt + 1 and r0
    // stage kt + 2 (both in flight).  Stages past KT are zeros, so an odd
    // KT costs one zero stage and no branch.
    u32x4 ra0[ACH], rb0[BCH], ra1[ACH], rb1[BCH];
    gload(ra0, rb0, 0);
    gload(ra1, rb1, 1);
    sstore(ra0, rb0, 0);
    __syncthreads();
    gload(ra0, rb0, 2);
    // The scheduling barriers keep each stage's loads where they are
    // issued here; left alone, the compiler sinks them below the next
    // LDS stores and the prefetch distance shrinks to one stage.
    for (int kt = 0; kt < KT; kt += 2) {
        compute(0);
        sstore(ra1, rb1, 1);  // buffer 1 was last read before the previous barrier
        __syncthreads();
        gload(ra1, rb1, kt + 3);
        __builtin_amdgcn_sched_barrier(0);
        compute(1);
        sstore(ra0, rb0, 0);
        __syncthreads();
        gload(ra0, rb0, kt + 4);
        __builtin_amdgcn_sched_barrier(0);
    }

    epilogue_fp8<TM, TN, TY>(acc, m0 + wm * WM, n0 + wn * WN, lane, M, N, sa, sb, bias, act, Y);
}

// ---- direct-to-LDS kernel (K a multiple of BK) ----------------------------------------
//
// Same contraction and epilogue; the tiles travel HBM -> LDS with the
// gfx950 16-byte buffer_load ... lds, which writes lane l's 16 bytes at the
// wave-uniform LDS address + 16 l, so the XOR swizzle is applied on the
// global side (lane l of a 1 KB block fetches the chunk that belongs in its
// slot).  NS LDS stages form a ring: stage kt + NS - 1 is in flight while
// stage kt is contracted, with one barrier per stage and no register
// staging or LDS store instructions.  WGM x WGN waves (4 or 8: two waves per
// SIMD let one wave's MFMAs run while the other waits).

// Chunk slot of 16-byte chunk `c` in row `row` of a BK-byte-row tile:
// consecutive rows of one 256-byte LDS bank window keep their chunks in
// distinct banks, and a 16-lane read of one chunk column is conflict free.
template <int BKB>
__device__ __forceinline__ uint32_t dma_slot(uint32_t row, uint32_t c) {
    constexpr uint32_t CPR = BKB / 16, RW = 256 / BKB;
    return c ^ ((row / RW) % CPR);
}

// One 16-byte-per-lane buffer load straight into LDS at `lds` + 16 * lane.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff) {
    typedef __attribute__((address_space(3))) void *lds_ptr;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)lds, 16, voff, 0, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    // gfx9 s_waitcnt: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8.
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int BM, int BN, int WGM, int WGN, int BKB, int NS, typename TY>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void k_gemm_fp8_dma(const uint8_t *__restrict__ A,
                                                                   const float *__restrict__ sa,
                                                                   const uint8_t *__restrict__ B,
                                                                   const float *__restrict__ sb,
                                                                   const float *__restrict__ bias,
                                                                   TY *__restrict__ Y, int M, int N, int K,
                                                                   int act, int tiles_m, int tiles_n) {
    constexpr int NW = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int CPR = BKB / 16;                 // 16-byte chunks per tile row
    constexpr int RPI = 64 / CPR;                 // tile rows per 1 KB load
    constexpr int ALD = BM / RPI / NW, BLD = BN / RPI / NW;  // loads per wave per stage
    constexpr int STAGE = (BM + BN) * BKB;
    static_assert(ALD * RPI * NW == BM && BLD * RPI * NW == BN, "tile rows must split over the waves");
    static_assert(NS >= 2 && NS * STAGE <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KT = K / BKB;

    // Rows past the matrix read zero (or leave LDS as it was): they only
    // feed output rows / channels that are never stored.
    const auto ra_src = make_rsrc(A + (size_t)m0 * K, (uint32_t)(M - m0) * (uint32_t)K);
    const auto rb_src = make_rsrc(B + (size_t)n0 * K, (uint32_t)(N - n0) * (uint32_t)K);

    // Load i of this wave covers tile rows [(i NW + wid) RPI, +RPI); lane l
    // fills slot l % CPR of row l / CPR.
    const uint32_t lrow = (uint32_t)lane / CPR, lslot = (uint32_t)lane % CPR;
    uint32_t a_off[ALD], b_off[BLD];
#pragma unroll
    for (int i = 0; i < ALD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * RPI + lrow;
        a_off[i] = row * (uint32_t)K + dma_slot<BKB>(row, lslot) * 16;
    }
#pragma unroll
    for (int i = 0; i < BLD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * RPI + lrow;  // swizzle rows counted from B's first row
        b_off[i] = row * (uint32_t)K + dma_slot<BKB>(BM + row, lslot) * 16;
    }
    auto issue = [&](int kt, int buf) {
        const uint32_t k0 = (uint32_t)kt * BKB;
        const bool in = kt < KT;
        uint8_t *sbuf = smem + buf * STAGE;
#pragma unroll
        for (int i = 0; i < ALD; i++)
            dma16(ra_src, sbuf + (i * NW + wid) * RPI * BKB, in ? a_off[i] + k0 : kOob);
#pragma unroll
        for (int i = 0; i < BLD; i++)
            dma16(rb_src, sbuf + (BM + (i * NW + wid) * RPI) * BKB, in ? b_off[i] + k0 : kOob);
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int i = 0; i < TM; i++) acc[j][i] = (f32x16){};

    const uint32_t frow = lane & 31, fhalf = (lane >> 5) * 2;
    auto compute = [&](int buf) {
        const uint8_t *s = smem + buf * STAGE;
#pragma unroll
        for (int kk = 0; kk < BKB / 64; kk++) {
            i32x8 af[TM], bf[TN];
            const uint32_t c0 = kk * 4 + fhalf;
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint32_t row = wm * WM + i * 32 + frow;
                u32x4 lo = *(const u32x4 *)(s + row * BKB + (dma_slot<BKB>(row, c0) << 4));
                u32x4 hi = *(const u32x4 *)(s + row * BKB + (dma_slot<BKB>(row, c0 + 1) << 4));
                af[i] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint32_t row = BM + wn * WN + j * 32 + frow;
                u32x4 lo = *(const u32x4 *)(s + row * BKB + (dma_slot<BKB>(row, c0) << 4));
                u32x4 hi = *(const u32x4 *)(s + row * BKB + (dma_slot<BKB>(row, c0 + 1) << 4));
                bf[j] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int i = 0; i < TM; i++)
                    acc[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        bf[j], af[i], acc[j][i], 0, 0, 0, 0, 0, 0);
        }
    };

    // Entering stage kt: stages kt .. kt + NS - 2 are in flight (stages past
    // KT load nothing), so waiting until (NS - 2) stages' loads remain
    // leaves stage kt complete for this wave; the barrier then publishes
    // every wave's part of it and retires the reads of stage kt - 1, whose
    // buffer the next issue overwrites.
    constexpr int LPS = ALD + BLD;
#pragma unroll
    for (int st = 0; st < NS - 1; st++) issue(st, st);
    for (int kt = 0; kt < KT; kt += NS) {
#pragma unroll
        for (int j = 0; j < NS; j++) {
            if (kt + j < KT) {
                wait_vmcnt<(NS - 2) * LPS>();
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                issue(kt + j + NS - 1, (j + NS - 1) % NS);
                compute(j);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    epilogue_fp8<TM, TN, TY>(acc, m0 + wm * WM, n0 + wn * WN, lane, M, N, sa, sb, bias, act, Y);
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

template <int BM, int BN, int WGM, int WGN, int BKB, int NS>
void launch_dma(hipStream_t s, const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
                const float *bias, int act, void *y, int y_dtype, int M, int N, int K) {
    int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    dim3 grid(tiles_m * tiles_n), block(64 * WGM * WGN);
    if (y_dtype == LX2V_DTYPE_BF16)
        hipLaunchKernelGGL((k_gemm_fp8_dma<BM, BN, WGM, WGN, BKB, NS, uint16_t>), grid, block, 0, s, a, sa, b, sb,
                           bias, (uint16_t *)y, M, N, K, act, tiles_m, tiles_n);
    else
        hipLaunchKernelGGL((k_gemm_fp8_dma<BM, BN, WGM, WGN, BKB, NS, float>), grid, block, 0, s, a, sa, b, sb, bias,
                           (float *)y, M, N, K, act, tiles_m, tiles_n);
}

// Direct-to-LDS configurations: tile (activation rows x channels), wave
// grid, K bytes per stage, stages.
struct DmaCfg {
    int bm, bn, wgm, wgn, bk, ns;
};
constexpr DmaCfg kDma[] = {
    {256, 128, 2, 2, 128, 3},  // 0
    {128, 256, 2, 2, 128, 3},  // 1
    {128, 128, 2, 2, 128, 4},  // 2
    {256, 128, 4, 2, 128, 3},  // 3  (8 waves)
    {128, 256, 2, 4, 128, 3},  // 4  (8 waves)
    {256, 256, 2, 4, 64, 4},   // 5  (8 waves)
    {256, 256, 2, 2, 64, 4},   // 6
};

void launch_dma_idx(int idx, hipStream_t s, const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
                    const float *bias, int act, void *y, int y_dtype, int M, int N, int K) {
    switch (idx) {
        case 0: launch_dma<256, 128, 2, 2, 128, 3>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K); break;
        case 1: launch_dma<128, 256, 2, 2, 128, 3>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K); break;
        case 2: launch_dma<128, 128, 2, 2, 128, 4>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K); break;
        case 3: launch_dma<256, 128, 4, 2, 128, 3>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K); break;
        case 4: launch_dma<128, 256, 2, 4, 128, 3>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K); break;
        case 5: launch_dma<256, 256, 2, 4, 64, 4>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K); break;
        default: launch_dma<256, 256, 2, 2, 64, 4>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K); break;
    }
}

// Tuning override: LIGHTX2V_HIP_FP8_CFG=<index into kDma> forces one
// direct-to-LDS configuration (-1 or unset: automatic).
int forced_cfg() {
    static int v = [] {
        const char *e = getenv("LIGHTX2V_HIP_FP8_CFG");
        return e ? atoi(e) : -1;
    }();
    return v;
}

}  // namespace

bool gemm_fp8_supported(size_t M, size_t N, size_t K) {
    // 32-bit buffer offsets (the out-of-range offset 2^31 must stay past
    // the end); K a multiple of 16 (the 16-byte chunk loads).
    return M > 0 && N > 0 && K >= 16 && K % 16 == 0 && M * K < (1ull << 31) &&
           N * K < (1ull << 31) && M < (1u << 30) && N < (1u << 30);
}

void launch_gemm_fp8(hipStream_t s, int num_cu, const uint8_t *a, const float *a_scale,
                     const uint8_t *b, const float *b_scale, const float *bias, int act, void *y,
                     int y_dtype, size_t M, size_t N, size_t K) {
    int m = (int)M, n = (int)N, k = (int)K;
    const int nd = (int)(sizeof(kDma) / sizeof(kDma[0]));
    if (K % 128 == 0) {
        int pick = forced_cfg();
        if (pick < 0 || pick >= nd) {
            // The 8-wave tiles (measured fastest at every Wan shape); of
            // those, the one that fills the chip best: fraction of issued
            // MFMA work that is useful over whole waves of workgroups; ties
            // keep the earlier.
            double best = -1.0;
            pick = 3;
            for (int i = 3; i < 5; i++) {
                size_t tiles = ((M + kDma[i].bm - 1) / kDma[i].bm) * ((N + kDma[i].bn - 1) / kDma[i].bn);
                size_t waves = (tiles + num_cu - 1) / num_cu;
                double eff = (double)M * N / ((double)waves * num_cu * kDma[i].bm * kDma[i].bn);
                if (eff > best * 1.0001) {
                    best = eff;
                    pick = i;
                }
            }
        }
        launch_dma_idx(pick, s, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k);
        return;
    }
    // K not a multiple of 128: the register-staged kernel.
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
    switch (pick) {
        case 0: launch_cfg<256, 128>(s, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k); break;
        case 1: launch_cfg<128, 256>(s, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k); break;
        default: launch_cfg<128, 128>(s, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k); break;
    }
}

}  // namespace lx2v

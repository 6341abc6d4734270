// k_gemm_fp8.hip -- FP8-e4m3 weight x per-token (or MX) e4m3 activation GEMM
// on the gfx950 fp8 MFMA (v_mfma_f32_32x32x64_f8f6f4), for weights with one
// scale per output channel (Fp8E4M3 with group == cols, quant.rs:364-373,
// 425-429) or one per 128 columns of K (group 128, quant.rs:21).
//
//   Y[m, n] = act( (sum_k e4m3(A[m,k]) * e4m3(B[n,k])) * sa[m] * sb[n] + bias[n] )
//
// With group 128 the running sums are rescaled by s[n][g-1] / s[n][g] at
// each group boundary and sb is the last group's scale (k_gemm_fp8_dma's
// notes on GS).
//
// A = per-token quantized activations [M, K], B = the weight's e4m3 codes
// [N, K] exactly as the reference lays them out (row-major, K contiguous);
// both are K-major, the layout the MFMA operands want, so codes go from HBM
// to LDS to the matrix cores untouched.
//
// Kernels (one workgroup per BM x BN output tile, waves of 64 x 64 or 128 x
// 64 sub-tiles of 32 x 32 MFMA blocks, K-major operands from HBM to LDS):
//   k_gemm_fp8_dma -- the main kernel: 16-byte buffer_load ... lds straight
//     into an NS-stage LDS ring (K % 128 == 0), one to three workgroups per
//     CU, an LDS-staged epilogue, per-token or MX e4m3 activations, bf16 /
//     f32 / MX e4m3 output;
//   k_gemm_fp8_pp  -- 256 x 256 tiles whose two wave groups alternate MFMA
//     and LDS phases (ping-pong);
//   k_gemm_fp8     -- register-staged, for K a multiple of 16 but not 128.
// plan_gemm_fp8 picks the configuration per shape from a fitted time model.
//
// Operand roles: the weight tile is the MFMA's A operand and the activation
// tile its B operand, so the 32 x 32 result block D[n][m] leaves each lane
// one activation row m and, per group of four accumulator registers, four
// consecutive output channels n.
#include "gemm_common.hpp"

// The skewed K loop of k_gemm_fp8_dma (on unless built with -DLX2V_FP8_SKEW=0).
#ifndef LX2V_FP8_SKEW
#define LX2V_FP8_SKEW 1
#endif
// ... with the second slice's fragment reads between the first slice's
// MFMAs (on unless built with -DLX2V_FP8_EARLY=0).
#ifndef LX2V_FP8_EARLY
#define LX2V_FP8_EARLY 1
#endif
// Cache-policy bits of the output stores (buffer_store: 1 = sc0, 2 = nt,
// 16 = sc1): of the LDS-staged epilogues (k_gemm_fp8_dma, _pt, _pp), of
// k_gemm_fp8_w4's register epilogue with MX e4m3 / bf16 output and of
// k_gemm_fp8_ov's.  The values written are the same for every policy; the
// choice is by measured time at the Wan shapes: sc1 made the one-round
// 4680 x 1536 -> 1536 tiles about 1.3 us faster per launch and FFN up's MX
// output about 4 us, and made the bf16 256 x 256 stores (the 30-layer K/V
// call) and the overlapped epilogue's (QKV) slower: 0.1 and 1.3 ms per
// chunk; nt was slower wherever a tile stores from registers.
#ifndef LX2V_STAGED_CP
#define LX2V_STAGED_CP 16
#endif
#ifndef LX2V_W4MX_CP
#define LX2V_W4MX_CP 16
#endif
#ifndef LX2V_W4BF_CP
#define LX2V_W4BF_CP 0
#endif
#ifndef LX2V_OV_CP
#define LX2V_OV_CP 0
#endif

namespace lx2v {

namespace {

constexpr int BK = 128;  // bytes (= e4m3 elements) of K per stage
constexpr int kStagedCP = LX2V_STAGED_CP;

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
            // One channel group at a time: keeps the accumulators in AGPRs
            // instead of moving them all to VGPRs up front.
            __builtin_amdgcn_sched_barrier(0);
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
// SIMD let one wave's MFMAs run while the other waits); dma_slot gives the
// LDS swizzle.

// MX activations (AM = 1): A's E8M0 block scales (mx_sidx layout, amx_rows
// rows per 128-column group, amx_len bytes readable from amx) travel with
// each stage -- wave 0 adds one 16-byte DMA of the stage's 128-column group,
// BM rows x 4 bytes -- and feed the block-scaled MFMA: each lane reads its
// row's 4 bytes once per stage and shifts the one its K block needs into
// byte 0 (the byte the MFMA's scale operand reads); the weight's scale
// operand is 2^0.  TY = uint8_t writes MX e4m3 output (codes to Y, scales
// to ymx).
//
// Grouped weight scales (GS = 1): one scale per 128 columns of K per channel
// (Fp8E4M3 with group 128, quant.rs:21, 425-429), BKB = 128 so that a stage
// is exactly one scale group.  Wave 0 adds one DMA per stage: the stage's
// BN channel ratios s_{kt-1} / s_kt from the weight's ratio table (row kt
// of gsc, N floats a row; row 0 all ones).  Before the stage's first MFMA on
// a block, the block's sums are multiplied by its channels' ratios, so the
// accumulator always holds the sum in units of the current group's scale;
// sb holds the last group's scales, which the epilogue applies as a
// per-channel scale, and sa still scales each token.
//
// ACT: the epilogue activation (LX2V_ACT_*), a template parameter so that the
// epilogue holds one copy of its staging code.
template <int BM, int BN, int WGM, int WGN, int BKB, int NS, int OCC, int AM, int GS, int ACT, typename TY>
__global__ __launch_bounds__(64 * WGM * WGN, OCC) void k_gemm_fp8_dma(const uint8_t *__restrict__ A,
                                                                   const float *__restrict__ sa,
                                                                   const uint8_t *__restrict__ B,
                                                                   const float *__restrict__ sb,
                                                                   const float *__restrict__ bias,
                                                                   TY *__restrict__ Y, int M, int N, int K,
                                                                   int act, int tiles_m, int tiles_n,
                                                                   const uint8_t *__restrict__ amx,
                                                                   uint32_t amx_len, int amx_rows,
                                                                   uint8_t *__restrict__ ymx, int ymx_rows,
                                                                   const float *__restrict__ gate,
                                                                   const float *__restrict__ gsc) {
    constexpr int NW = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int CPR = BKB / 16;                 // 16-byte chunks per tile row
    constexpr int RPI = 64 / CPR;                 // tile rows per 1 KB load
    constexpr int ALD = BM / RPI / NW, BLD = BN / RPI / NW;  // loads per wave per stage
    constexpr int STAGE = (BM + BN) * BKB;
    // Fragment-read offsets inside a stage's A rows / B rows, masked (no-op
    // masks: the regions are powers of two) so that the compiler can bound
    // them: it then sees a read never touches a slot a pending DMA writes
    // and waits only for the loads the read needs, not for every load.
    constexpr uint32_t AMASK = BM * BKB - 1, BMASK = BN * BKB - 1;
    static_assert(((BM * BKB) & AMASK) == 0 && ((BN * BKB) & BMASK) == 0, "tile regions are powers of two");
    static_assert(ALD * RPI * NW == BM && BLD * RPI * NW == BN, "tile rows must split over the waves");
    using Ops = TileOps<BM, BN, 64 * NW>;
    // per-stage LDS for A's block scales (BM rows x 4 bytes) or the weight's
    // group scales (BN floats): a whole wave's 16-byte DMA (lanes whose
    // offset is out of range still write their zeros)
    constexpr int ASL = AM ? 1024 : 16, GSL = GS ? 1024 : 16;
    static_assert(!AM || BM * 4 <= ASL, "A scale slot");
    static_assert(!GS || (BKB == 128 && BN * 4 <= 64 * 16), "grouped scales: one 128-column group per stage");
    constexpr bool XS = AM || GS;       // wave 0 issues more loads per stage
    constexpr int XN = (AM ? 1 : 0) + (GS ? 1 : 0);  // ... this many
    static_assert(NS >= 2 && OCC * (NS * STAGE + Ops::NV * 4 + NS * (ASL + GSL)) <= 160 * 1024,
                  "LDS for OCC workgroups per CU");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE];
    __shared__ __attribute__((aligned(16))) float sc[Ops::NV];
    __shared__ __attribute__((aligned(16))) uint8_t asl[NS * ASL];
    __shared__ __attribute__((aligned(16))) uint8_t gsl[NS * GSL];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    const int wid_u = __builtin_amdgcn_readfirstlane(wid);  // DMA LDS addresses only (scalar)
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;
    // Split K (gridDim.y > 1; per-token / per-channel scales only, which the
    // host leaves to the reduction): part blockIdx.y of the stages, its sums
    // to its own M x N slice of Y.
    const int kts = K / BKB, kt0 = (int)((long long)blockIdx.y * kts / gridDim.y);
    const int KT = (int)((long long)(blockIdx.y + 1) * kts / gridDim.y) - kt0;
    Y += (size_t)blockIdx.y * (size_t)M * (size_t)N;
    Ops ops;
    ops.load(tid, m0, n0, M, N, sa, sb, bias);

    // Rows past the matrix read zero (or leave LDS as it was): they only
    // feed output rows / channels that are never stored.
    const uint32_t k0b = (uint32_t)kt0 * BKB;
    const auto ra_src = make_rsrc(A + (size_t)m0 * K + k0b, (uint32_t)(M - m0) * (uint32_t)K - k0b);
    const auto rb_src = make_rsrc(B + (size_t)n0 * K + k0b, (uint32_t)(N - n0) * (uint32_t)K - k0b);
    // (readfirstlane: the saturating length would otherwise be computed on
    // the VALU and take the descriptor out of SGPRs)
    const auto rs_src = make_rsrc(
        AM ? amx + 4 * m0 : A, __builtin_amdgcn_readfirstlane(AM ? (amx_len > 4u * m0 ? amx_len - 4u * (uint32_t)m0 : 0u)
                                                                : 0u));
    const auto rg_src = make_rsrc(
        GS ? (const uint8_t *)(gsc + n0) : A,
        __builtin_amdgcn_readfirstlane(GS ? ((uint32_t)KT * (uint32_t)N - (uint32_t)n0) * 4u : 0u));

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
    // Load n (< ALD: A rows, then B rows) of this wave's share of stage kt.
    auto piece = [&](int n, int kt, int buf) {
        const uint32_t k0 = (uint32_t)kt * BKB;
        const bool in = kt < KT;
        uint8_t *sbuf = smem + buf * STAGE;
        if (n < ALD)
            dma16(ra_src, sbuf + (n * NW + wid_u) * RPI * BKB, in ? a_off[n < ALD ? n : 0] + k0 : kOob);
        else
            dma16(rb_src, sbuf + (BM + ((n - ALD) * NW + wid_u) * RPI) * BKB,
                  in ? b_off[n >= ALD ? n - ALD : 0] + k0 : kOob);
    };
    // Wave 0's MX scale load of stage kt (slot buf) and / or its group-scale load.
    auto issue_scales = [&](int kt, int buf) {
        if constexpr (GS) {
            // lane l: the ratios of channels n0 + 4 l .. + 3 at stage kt; past
            // the last channel the next row (or zeros at the end) is read, for
            // channels that are never stored
            if (wid_u == 0) {
                const bool ok = kt < KT && lane < BN / 4;
                dma16(rg_src, gsl + buf * GSL, ok ? (uint32_t)kt * (uint32_t)N * 4u + (uint32_t)lane * 16u : kOob);
            }
        }
        if constexpr (AM) {
            const bool in = kt < KT;
            // First in the stage's issue order: issued after the A / B
            // loads, this load's return gated wave 0's stage waits (measured
            // ~15% on the K-heavy shapes).  Wave 0; lane l: rows 4 l .. 4 l
            // + 3 of the stage's 128-column group.
            if (wid_u == 0) {
                const bool ok = in && lane < BM / 4;
                dma16(rs_src, asl + buf * ASL,
                      ok ? (uint32_t)(kt * BKB / 128) * (uint32_t)amx_rows * 4u + (uint32_t)lane * 16u : kOob);
            }
        }
    };
    auto issue = [&](int kt, int buf) {
        issue_scales(kt, buf);
#pragma unroll
        for (int n = 0; n < ALD + BLD; n++) piece(n, kt, buf);
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int i = 0; i < TM; i++) acc[j][i] = (f32x16){};

    const uint32_t frow = lane & 31, fhalf = (lane >> 5) * 2;
    constexpr int LPS = ALD + BLD;
    // The K loop skewed by one slice (below): 128-byte stages, per-stage
    // scales not folded per stage.
    constexpr bool SKEW = LX2V_FP8_SKEW && BKB == 128;
    // One 64-byte K slice's fragments: the wave's TM A row blocks and TN B
    // column blocks.
    struct Frag {
        i32x8 a[TM], b[TN];
    };
    // read_half(buf, kk, f): slice kk of the stage in slot buf.  16-byte
    // chunks of the 64-byte K slice each lane supplies: the block-scaled MFMA
    // reads a lane's bytes 0..15 as K [16 h, 16 h + 16) and bytes 16..31 as
    // K [32 + 16 h, +16) of the slice (h = lane / 32) and scales K [0, 32)
    // with the lanes-0..31 scale and K [32, 64) with the lanes-32..63 one
    // (probed on gfx950), so with MX activations lane half h takes chunks h
    // and h + 2 and each MX block is one hardware scale block.  Unscaled, any
    // K order shared by both operands is the same product.
    // read_frag(buf, kk, f, i): fragment i of slice kk (the wave's A row
    // blocks 0 .. TM - 1, then its B column blocks).
    auto read_frag = [&](int buf, int kk, Frag &f, int i) {
        const uint8_t *s = smem + buf * STAGE;
        const uint32_t c0 = AM ? kk * 4 + (lane >> 5) : kk * 4 + fhalf;
        const uint32_t c1 = AM ? c0 + 2 : c0 + 1;
        if (i < TM) {
            const uint32_t row = wm * WM + i * 32 + frow;
            u32x4 lo = *(const u32x4 *)(s + ((row * BKB + (dma_slot<BKB>(row, c0) << 4)) & AMASK));
            u32x4 hi = *(const u32x4 *)(s + ((row * BKB + (dma_slot<BKB>(row, c1) << 4)) & AMASK));
            f.a[i] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        } else {
            const int j = i - TM;
            const uint32_t row = BM + wn * WN + j * 32 + frow;
            const uint32_t rb = row - BM;
            u32x4 lo = *(const u32x4 *)(s + BM * BKB + ((rb * BKB + (dma_slot<BKB>(row, c0) << 4)) & BMASK));
            u32x4 hi = *(const u32x4 *)(s + BM * BKB + ((rb * BKB + (dma_slot<BKB>(row, c1) << 4)) & BMASK));
            f.b[j] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
    };
    auto read_half = [&](int buf, int kk, Frag &f) {
#pragma unroll
        for (int i = 0; i < TM + TN; i++) read_frag(buf, kk, f, i);
    };
    // MX activations: each of the wave's rows' 4 scale bytes of the stage in
    // slot buf, and the scale operand of slice kk (lane l holds block 2 s +
    // l / 32 of its row's 128-column group, s the 64-column slice: that
    // block's scale shifted into byte 0).
    typedef uint32_t SRaw[AM ? TM : 1];
    typedef int SOp[AM ? TM : 1];
    auto read_sraw = [&](int buf, SRaw &sr) {
        if constexpr (AM) {
#pragma unroll
            for (int i = 0; i < TM; i++) sr[i] = *(const uint32_t *)(asl + buf * ASL + (wm * WM + i * 32 + frow) * 4);
        }
    };
    auto scale_op = [&](const SRaw &sr, int kk, int stage, SOp &as) {
        if constexpr (AM) {
            const int sh = 8 * (int)(lane >> 5) + 16 * (BKB == 128 ? kk : (stage & 1));
#pragma unroll
            for (int i = 0; i < TM; i++) as[i] = (int)(sr[i] >> sh);
        }
    };
    // mfma_half(f, as, nbase, dkt, dbuf): the slice's TN x TM MFMAs into acc,
    // with load nbase + (j TM + i) of stage dkt (slot dbuf) issued after MFMA
    // (j, i) while it is below LPS -- issued back to back right after the
    // barrier, the loads held both waves of a SIMD off the MFMA pipe (7-9%
    // at one workgroup per CU).  dkt < 0: no loads.  RS (grouped scales, a
    // stage's first slice): block m is rescaled (rescale(m)) right before its
    // MFMA.
    // after(m): called after the half's MFMA m (0 .. TN TM - 1), behind the
    // load it may issue -- the skewed loop reads the next slice's fragments
    // there, so that they land while the half's later MFMAs run.
    // Grouped scales (GS, one scale per 128 columns of K per channel, a
    // stage being one group): the accumulator holds the sum so far in units
    // of the current group's scale.  Before stage g's first MFMA on a block
    // its sums are multiplied by s_{g-1} / s_g of each of the lane's
    // channels (the weight's ratio table, row g, loaded by wave 0 with each
    // stage; row 0 is all ones), and the epilogue's channel scale is the
    // last group's: every tile shape and kernel applies the same operations
    // to a block in the same order.
    // TR (grouped scales, bf16 / f32 output): the blocks are transposed --
    // the MFMA takes the activations as its first operand, so lane l holds
    // channel l % 32 of a block (and the block's rows 8 g + 4 (l / 32) + q)
    // and needs one ratio per block, one 4-byte LDS read, where the plain
    // layout needs 16 channels' ratios, four 16-byte reads: measured, those
    // reads were most of the grouped kernels' cost over the per-channel
    // ones.  The swapped MFMA gives exactly the transposed sums (checked bit
    // for bit on gfx950), so the results are the plain layout's.
    constexpr bool TR = GS && sizeof(TY) != 1;
    f32x4 rg[GS && !TR ? TN : 1][4];
    float rt[TR ? TN : 1];
    auto read_r = [&](int buf) {
        if constexpr (TR) {
#pragma unroll
            for (int j = 0; j < TN; j++) rt[j] = *(const float *)(gsl + buf * GSL + (wn * WN + j * 32 + (lane & 31)) * 4);
        } else if constexpr (GS) {
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    rg[j][g] = *(const f32x4 *)(gsl + buf * GSL + (wn * WN + j * 32 + 8 * g + 4 * (lane >> 5)) * 4);
        }
    };
    auto rescale = [&](int m) {
        if constexpr (TR) {
            const int j = m / TM, i = m % TM;
#pragma unroll
            for (int e = 0; e < 16; e++) acc[j][i][e] *= rt[j];
        } else if constexpr (GS) {
            const int j = m / TM, i = m % TM;
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
                for (int q = 0; q < 4; q++) acc[j][i][4 * g + q] *= rg[j][g][q];
        }
    };
    auto mfma_half_then = [&](auto RS, const Frag &f, const SOp &as, int kk, int nbase, int dkt, int dbuf,
                              auto &&after) {
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int i = 0; i < TM; i++) {
                if constexpr (decltype(RS)::value) rescale(j * TM + i);
                if constexpr (AM && TR)
                    acc[j][i] =
                        __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[i], f.b[j], acc[j][i], 0, 0, 0, as[i], 0, 127);
                else if constexpr (AM)
                    acc[j][i] =
                        __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b[j], f.a[i], acc[j][i], 0, 0, 0, 127, 0, as[i]);
                else if constexpr (TR)
                    acc[j][i] =
                        __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[i], f.b[j], acc[j][i], 0, 0, 0, 0, 0, 0);
                else
                    acc[j][i] =
                        __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b[j], f.a[i], acc[j][i], 0, 0, 0, 0, 0, 0);
                const int n = nbase + j * TM + i;
                if (n < LPS && dkt >= 0) {
                    __builtin_amdgcn_sched_barrier(0);
                    piece(n, dkt, dbuf);
                    __builtin_amdgcn_sched_barrier(0);
                }
                after(j * TM + i);
            }
    };
    using RsNo = std::false_type;
    using RsYes = std::integral_constant<bool, GS != 0>;
    auto mfma_half = [&](const Frag &f, const SOp &as, int kk, int nbase, int dkt, int dbuf) {
        mfma_half_then(RsNo{}, f, as, kk, nbase, dkt, dbuf, [](int) {});
    };
    // compute(buf, stage, dkt, dbuf): the MFMAs of `stage` from slot buf,
    // slice by slice (each slice's reads, then its MFMAs), with the loads of
    // stage dkt interleaved.
    auto compute = [&](int buf, int stage, int dkt, int dbuf) {
        SRaw sraw;
        read_sraw(buf, sraw);
        read_r(buf);
#pragma unroll
        for (int kk = 0; kk < BKB / 64; kk++) {
            Frag f;
            read_half(buf, kk, f);
            SOp as;
            scale_op(sraw, kk, stage, as);
            if (kk == 0)
                mfma_half_then(RsYes{}, f, as, kk, kk * TN * TM, dkt, dbuf, [](int) {});
            else
                mfma_half(f, as, kk, kk * TN * TM, dkt, dbuf);
        }
    };
    static_assert((BKB / 64) * TN * TM >= ALD + BLD, "a stage's loads interleave with its MFMAs");

    // Entering stage kt: stages kt .. kt + NS - 2 are in flight (stages past
    // KT load nothing), so waiting until (NS - 2) stages' loads remain
    // leaves stage kt complete for this wave; the barrier then publishes
    // every wave's part of it and retires the reads of stage kt - 1, whose
    // buffer the next issue overwrites.
#pragma unroll
    for (int st = 0; st < NS - 1; st++) issue(st, st);
    if constexpr (SKEW) {
        // Skewed by one 64-byte slice: a wave reads stage kt's second slice
        // at the end of iteration kt and contracts it after the next barrier,
        // while stage kt + 1's first slice is being read, so the MFMAs that
        // follow a barrier never wait for LDS.  Each wait before a barrier
        // also retires the wave's reads (lgkmcnt 0): the loads issued after
        // the barrier overwrite the slot those reads came from.
        Frag f0, f1;
        SRaw sr;
        SOp as1;
        auto wait_stage = [&]() {
            if (XS && wid_u == 0)  // wave 0 also loads each stage's A scales
                wait_vmcnt_lds0<(NS - 2) * (LPS + XN)>();
            else
                wait_vmcnt_lds0<(NS - 2) * LPS>();
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        };
        // stage 0: its first slice, then the second slice's reads
        wait_stage();
        if constexpr (XS) issue_scales(NS - 1, NS - 1);
        read_sraw(0, sr);
        read_half(0, 0, f0);
        {
            SOp as0;
            scale_op(sr, 0, 0, as0);
            mfma_half(f0, as0, 0, 0, NS - 1, NS - 1);
        }
#pragma unroll
        for (int n = TN * TM; n < LPS; n++) piece(n, NS - 1, NS - 1);
        read_half(0, 1, f1);
        scale_op(sr, 1, 0, as1);
        __builtin_amdgcn_sched_barrier(0);
        // stage kt (kt = 1 mod NS at the top): slot (kt + j) % NS, the loads
        // of stage kt + j + NS - 1 into slot j
        for (int kt = 1; kt < KT; kt += NS) {
#pragma unroll
            for (int j = 0; j < NS; j++) {
                if (kt + j < KT) {
                    const int buf = (1 + j) % NS;
                    wait_stage();
                    if constexpr (XS) issue_scales(kt + j + NS - 1, j);
                    read_sraw(buf, sr);
                    read_r(buf);
                    read_half(buf, 0, f0);
                    __builtin_amdgcn_sched_barrier(0);
                    mfma_half(f1, as1, 1, 0, kt + j + NS - 1, j);  // stage kt + j - 1, second slice
                    SOp as0;
                    scale_op(sr, 0, kt + j, as0);
#if LX2V_FP8_EARLY
                    // the second slice's fragments read between the first
                    // slice's MFMAs (RPM reads per MFMA), so that they have
                    // landed when the next barrier's wait retires them
                    mfma_half_then(RsYes{}, f0, as0, 0, TN * TM, kt + j + NS - 1, j, [&](int m) {
                        constexpr int RPM = (TM + TN + TN * TM - 1) / (TN * TM);
#pragma unroll
                        for (int r = 0; r < RPM; r++)
                            if (m * RPM + r < TM + TN) {
                                __builtin_amdgcn_sched_barrier(0);
                                read_frag(buf, 1, f1, m * RPM + r);
                                __builtin_amdgcn_sched_barrier(0);
                            }
                    });
#else
                    mfma_half_then(RsYes{}, f0, as0, 0, TN * TM, kt + j + NS - 1, j, [](int) {});
                    read_half(buf, 1, f1);
#endif
                    scale_op(sr, 1, kt + j, as1);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        mfma_half(f1, as1, 1, 0, -1, 0);
    } else {
        for (int kt = 0; kt < KT; kt += NS) {
#pragma unroll
            for (int j = 0; j < NS; j++) {
                if (kt + j < KT) {
                    if (XS && wid_u == 0)  // wave 0 also loads each stage's A and / or group scales
                        wait_vmcnt<(NS - 2) * (LPS + XN)>();
                    else
                        wait_vmcnt<(NS - 2) * LPS>();
                    __builtin_amdgcn_s_barrier();
                    __builtin_amdgcn_sched_barrier(0);
                    if constexpr (XS) issue_scales(kt + j + NS - 1, (j + NS - 1) % NS);
                    compute(j, kt + j, kt + j + NS - 1, (j + NS - 1) % NS);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }
    ops.park(sc, tid, m0, n0, M, N, sa, sb);
    MxOut mx;
    mx.scales = ymx;
    mx.rows = ymx_rows;
    mx.gate = gate;
    staged_epilogue<BM, BN, 64 * NW, NS * STAGE, TM, TN, TY, true, ACT, true, kStagedCP, TR>(
        acc, smem, sc, wm * WM, wn * WN, tid, lane, m0, n0, M, N, act, Y, mx);
}

// ---- persistent direct-to-LDS kernel ---------------------------------------------
//
// k_gemm_fp8_dma's 256 x 128 tile (8 waves of 64 x 64 sub-tiles, 128-byte
// stages in a 3-stage ring, per-token e4m3 activations) as one workgroup per
// CU that walks a list of tiles: pass i of workgroup w computes tile
// xcd_tile(w + i G) for a grid of G = min(tiles, CUs) workgroups, G a
// multiple of 8 whenever the tiles outnumber the CUs, so every tile of a
// workgroup lies in its XCD's band.  The ring runs on across
// tiles: while a tile's last two stages are contracted, the next tile's
// first two are already loading, and the epilogue stages its outputs
// through the slot the last stage freed.  A tile's token scales, channel
// scales and bias travel into LDS by DMA too (issued with its first stage),
// so no compiler-tracked load is ever waited for -- such a wait would also
// wait for the next tile's stages.  Null scales read a table of ones.
//
// Constraints (checked by the host): K % 128 == 0 and K >= 256; no MX
// activations, no residual mode.  GS: group-128 weight scales (wave 0 adds
// the stage's BN scales to each stage, as in k_gemm_fp8_dma).

__device__ const float k_ones[256] = {
#define LX2V_1x16 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f
    LX2V_1x16, LX2V_1x16, LX2V_1x16, LX2V_1x16, LX2V_1x16, LX2V_1x16, LX2V_1x16, LX2V_1x16,
    LX2V_1x16, LX2V_1x16, LX2V_1x16, LX2V_1x16, LX2V_1x16, LX2V_1x16, LX2V_1x16, LX2V_1x16
#undef LX2V_1x16
};

template <int GS, int ACT, typename TY>
__global__ __launch_bounds__(512, 1) void k_gemm_fp8_pt(const uint8_t *__restrict__ A, const float *__restrict__ sa,
                                                       const uint8_t *__restrict__ B, const float *__restrict__ sb,
                                                       const float *__restrict__ bias, TY *__restrict__ Y, int M,
                                                       int N, int K, int act, int tiles_m, int tiles_n,
                                                       uint8_t *__restrict__ ymx, int ymx_rows,
                                                       const float *__restrict__ gsc) {
    constexpr int BM = 256, BN = 128, WGM = 4, WGN = 2, BKB = 128, NS = 3;
    constexpr int NW = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int CPR = BKB / 16, RPI = 64 / CPR;
    constexpr int ALD = BM / RPI / NW, BLD = BN / RPI / NW;
    constexpr int STAGE = (BM + BN) * BKB;
    constexpr uint32_t AMASK = BM * BKB - 1, BMASK = BN * BKB - 1;
    constexpr int GSL = 1024;  // per-stage slot for the group scales (a whole wave's DMA)
    constexpr int NV = BM + 2 * BN;
    static_assert(NS * STAGE + NV * 4 + 1024 + (GS ? NS * GSL : 0) <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE];
    // [BM token scales][BN channel scales][BN bias] + a 1 KB pad that the
    // partial DMAs of the last region never reach (lane-masked)
    __shared__ __attribute__((aligned(16))) float sc[NV + 256];
    __shared__ __attribute__((aligned(16))) uint8_t gsl[GS ? NS * GSL : 16];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    const int wid_u = __builtin_amdgcn_readfirstlane(wid);
    const int G = gridDim.x, w = blockIdx.x, ntiles = tiles_m * tiles_n;
    const int my_n = w < ntiles ? (ntiles - w + G - 1) / G : 0;
    if (my_n == 0) return;  // (uniform) no tile: no descriptor may be built
    const int KT = K / BKB;
    auto tile_of = [&](int i, int *m0, int *n0) {
        int tm, tn;
        xcd_tile(w + i * G, ntiles, tiles_m, tiles_n, &tm, &tn);
        *m0 = tm * BM;
        *n0 = tn * BN;
    };

    // Issue side: the (pass, stage) whose loads go out next, and its tile's
    // descriptors.
    int is_i = 0, is_kt = 0, is_m0 = 0, is_n0 = 0;
    tile_of(0, &is_m0, &is_n0);
    __amdgpu_buffer_rsrc_t ra_src, rb_src, rg_src;
    auto set_issue_tile = [&]() {
        ra_src = make_rsrc(A + (size_t)is_m0 * K, __builtin_amdgcn_readfirstlane((uint32_t)(M - is_m0) * (uint32_t)K));
        rb_src = make_rsrc(B + (size_t)is_n0 * K, __builtin_amdgcn_readfirstlane((uint32_t)(N - is_n0) * (uint32_t)K));
        if constexpr (GS)
            rg_src = make_rsrc(gsc + is_n0, __builtin_amdgcn_readfirstlane(
                                                ((uint32_t)KT * (uint32_t)N - (uint32_t)is_n0) * 4u));
    };
    set_issue_tile();

    const uint32_t lrow = (uint32_t)lane / CPR, lslot = (uint32_t)lane % CPR;
    uint32_t a_off[ALD], b_off[BLD];
#pragma unroll
    for (int i = 0; i < ALD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * RPI + lrow;
        a_off[i] = row * (uint32_t)K + dma_slot<BKB>(row, lslot) * 16;
    }
#pragma unroll
    for (int i = 0; i < BLD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * RPI + lrow;
        b_off[i] = row * (uint32_t)K + dma_slot<BKB>(BM + row, lslot) * 16;
    }
    // Load n of this wave's share of the issue stage into slot buf.
    auto piece = [&](int n, int buf) {
        const bool in = is_i < my_n;
        const uint32_t k0 = (uint32_t)is_kt * BKB;
        uint8_t *sbuf = smem + buf * STAGE;
        if (n < ALD)
            dma16(ra_src, sbuf + (n * NW + wid_u) * RPI * BKB, in ? a_off[n < ALD ? n : 0] + k0 : kOob);
        else
            dma16(rb_src, sbuf + (BM + ((n - ALD) * NW + wid_u) * RPI) * BKB,
                  in ? b_off[n >= ALD ? n - ALD : 0] + k0 : kOob);
    };
    auto issue_scales = [&](int buf) {
        if constexpr (GS) {
            if (wid_u == 0) {
                const bool ok = is_i < my_n && lane < BN / 4;
                dma16(rg_src, gsl + buf * GSL, ok ? (uint32_t)is_kt * (uint32_t)N * 4u + (uint32_t)lane * 16u : kOob);
            }
        }
    };
    auto advance_issue = [&]() {
        if (++is_kt == KT) {
            is_kt = 0;
            if (++is_i < my_n) {
                tile_of(is_i, &is_m0, &is_n0);
                set_issue_tile();
            }
        }
    };
    // The tile's epilogue operands into sc (wave 1: token scales, wave 2:
    // channel scales, wave 3: bias; lanes past the region masked off).
    // A null scale reads the ones table; a null bias reads nothing (zeros).
    auto issue_ops = [&](int m0, int n0) {
        if (wid_u == 1) {
            const auto r = sa ? make_rsrc(sa + m0, __builtin_amdgcn_readfirstlane((uint32_t)(M - m0) * 4u))
                              : make_rsrc(k_ones, 1024u);
            dma16(r, (uint8_t *)sc, (uint32_t)lane * 16u);
        } else if (wid_u == 2) {
            const auto r = sb ? make_rsrc(sb + n0, __builtin_amdgcn_readfirstlane((uint32_t)(N - n0) * 4u))
                              : make_rsrc(k_ones, 1024u);
            if (lane < BN / 4) dma16(r, (uint8_t *)(sc + BM), (uint32_t)lane * 16u);
        } else if (wid_u == 3) {
            const auto r = bias ? make_rsrc(bias + n0, __builtin_amdgcn_readfirstlane((uint32_t)(N - n0) * 4u))
                                : make_rsrc(k_ones, 0u);
            if (lane < BN / 4) dma16(r, (uint8_t *)(sc + BM + BN), (uint32_t)lane * 16u);
        }
    };
    constexpr int LPS = ALD + BLD;

    f32x16 acc[TN][TM];
    // Grouped scales: as k_gemm_fp8_dma, each block's sums are rescaled by
    // the stage's ratio s_{g-1} / s_g right before the stage's first MFMA
    // on the block; the epilogue's channel scale is the last group's.  (The
    // transposed blocks of k_gemm_fp8_dma measured slower here: 45.8 ->
    // 47.1 us at QKV; a tile's epilogue comes every 12 stages at the Wan
    // shapes and its 2-byte staging writes cost more than the ratio reads
    // save.)
    f32x4 rg[GS ? TN : 1][4];
    auto read_r = [&](int buf) {
        if constexpr (GS) {
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    rg[j][g] = *(const f32x4 *)(gsl + buf * GSL + (wn * WN + j * 32 + 8 * g + 4 * (lane >> 5)) * 4);
        }
    };
    const uint32_t frow = lane & 31, fhalf = (lane >> 5) * 2;
    auto compute = [&](int buf, bool do_issue, int dbuf) {
        const uint8_t *st = smem + buf * STAGE;
        read_r(buf);
#pragma unroll
        for (int kk = 0; kk < BKB / 64; kk++) {
            i32x8 af[TM], bf[TN];
            const uint32_t c0 = kk * 4 + fhalf, c1 = c0 + 1;
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint32_t row = wm * WM + i * 32 + frow;
                u32x4 lo = *(const u32x4 *)(st + ((row * BKB + (dma_slot<BKB>(row, c0) << 4)) & AMASK));
                u32x4 hi = *(const u32x4 *)(st + ((row * BKB + (dma_slot<BKB>(row, c1) << 4)) & AMASK));
                af[i] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint32_t row = BM + wn * WN + j * 32 + frow;
                const uint32_t rb = row - BM;
                u32x4 lo = *(const u32x4 *)(st + BM * BKB + ((rb * BKB + (dma_slot<BKB>(row, c0) << 4)) & BMASK));
                u32x4 hi = *(const u32x4 *)(st + BM * BKB + ((rb * BKB + (dma_slot<BKB>(row, c1) << 4)) & BMASK));
                bf[j] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    if constexpr (GS) {
                        if (kk == 0) {
#pragma unroll
                            for (int g = 0; g < 4; g++)
#pragma unroll
                                for (int q = 0; q < 4; q++) acc[j][i][4 * g + q] *= rg[j][g][q];
                        }
                    }
                    acc[j][i] =
                        __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], af[i], acc[j][i], 0, 0, 0, 0, 0, 0);
                    const int n = kk * TN * TM + j * TM + i;
                    if (n < LPS && do_issue) {
                        __builtin_amdgcn_sched_barrier(0);
                        piece(n, dbuf);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
        }
    };
    static_assert((BKB / 64) * TN * TM >= LPS, "a stage's loads interleave with its MFMAs");

    // Prologue: the first NS - 1 stages of the walk.
#pragma unroll
    for (int st = 0; st < NS - 1; st++) {
        issue_scales(st);
#pragma unroll
        for (int n = 0; n < LPS; n++) piece(n, st);
        advance_issue();
    }
    int s = 0;  // global stage index of this workgroup's walk
    for (int i = 0; i < my_n; i++) {
        int m0, n0;
        tile_of(i, &m0, &n0);
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int ii = 0; ii < TM; ii++) acc[j][ii] = (f32x16){};
        for (int kt = 0; kt < KT; kt++, s++) {
            // Stage s complete for this wave (stages s + 1 .. s + NS - 2 may
            // still fly); the barrier publishes every wave's part and frees
            // the slot the issue below refills.
            if (GS && wid_u == 0)
                wait_vmcnt<(NS - 2) * (LPS + 1)>();
            else
                wait_vmcnt<(NS - 2) * LPS>();
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            if (kt == 0) issue_ops(m0, n0);  // after the barrier: the last epilogue is done with sc
            const int buf = s % NS, dbuf = (s + NS - 1) % NS;
            issue_scales(dbuf);
            compute(buf, true, dbuf);
            advance_issue();
            __builtin_amdgcn_sched_barrier(0);
        }
        // The ops DMA went out with stage s - KT, before the ring loads that
        // every later wait covered (KT >= 2).
        MxOut mx;
        mx.scales = ymx;
        mx.rows = ymx_rows;
        staged_epilogue<BM, BN, 64 * NW, STAGE, TM, TN, TY, false, ACT, false, kStagedCP>(
            acc, smem + ((s - 1) % NS) * STAGE, sc, wm * WM, wn * WN, tid, lane, m0, n0, M, N, act, Y, mx);
    }
    wait_vmcnt<0>();  // the walk's trailing loads (zeros) land before the workgroup ends
}

// ---- persistent kernel with the epilogue folded into the next tile ----------------
//
// The persistent 256 x 128 walk of k_gemm_fp8_pt (3-stage DMA ring running
// on across tiles, epilogue operands by DMA, a grid of min(tiles, CUs)
// workgroups) with two accumulator sets, one per tile parity: while tile t
// + 1's first EP stages are contracted into one set, each wave finishes
// tile t from the other -- token scale, channel scale, bias, GELU, bf16
// rounding or MX e4m3 quantization -- one 32 x 32 block per stage (two
// stages with GELU), its VALU work placed between the stage's MFMAs so
// that it issues while the matrix core runs.  The tile's operands sit in
// the LDS slot of its parity, so the next tile's DMA does not overwrite them.
//
// The results go straight from registers to memory.  Lanes l and l + 32
// hold one token's channels 8g + 0..3 and 8g + 4..7 (g = 0..3); one
// v_permlane32_swap per register pair leaves lane l with a contiguous half
// of the 32 channels and lane l + 32 with the other, so each 16-byte store
// of a lane pairs with its neighbour's into one 32-byte piece of the row
// (bf16: two stores per block; MX: one 16-byte store of codes and the
// block's scale byte).
//
// vmcnt accounting: every stage issues LPS ring loads, and the stage that
// finishes a block issues PST stores after them (the first tile, which has
// no predecessor, stores to an out-of-range offset so that every count
// holds); the wait for stage s leaves in flight what was issued after its
// loads: the next stage's loads and the stores of the two stages between.
//
// Constraints (host): K % 128 == 0, K / 128 >= EP + 2, N % 128 == 0,
// M N sizeof(TY) < 2^31; bf16 or MX e4m3 output; per-token activations and
// per-channel weight scales; no residual mode.
template <int ACT, typename TY, int GS>
__global__ __launch_bounds__(512, 1) void k_gemm_fp8_ov(const uint8_t *__restrict__ A, const float *__restrict__ sa,
                                                       const uint8_t *__restrict__ B, const float *__restrict__ sb,
                                                       const float *__restrict__ bias, TY *__restrict__ Y, int M,
                                                       int N, int K, int tiles_m, int tiles_n,
                                                       uint8_t *__restrict__ ymx, int ymx_rows,
                                                       const float *__restrict__ gsc) {
    constexpr int BM = 256, BN = 128, WGN = 2, BKB = 128, NS = 3;
    constexpr int NW = 8, WM = 64, WN = 64, TM = 2, TN = 2;
    constexpr int CPR = BKB / 16, RPI = 64 / CPR;
    constexpr int ALD = BM / RPI / NW, BLD = BN / RPI / NW, LPS = ALD + BLD;
    constexpr int STAGE = (BM + BN) * BKB;
    constexpr uint32_t AMASK = BM * BKB - 1, BMASK = BN * BKB - 1;
    constexpr int NV = BM + 2 * BN;
    constexpr int EB = sizeof(TY);
    static_assert(EB == 1 || EB == 2, "bf16 or MX e4m3 output");
    constexpr bool GELU = ACT == LX2V_ACT_GELU_TANH;
    constexpr int NSLOT = 2 * TN * TM;  // MFMA slots per stage
    // A finished block's epilogue spans two stages (16 slots).  Its 16
    // values (channel group g = e / 4) are computed four per slot at slots
    // 1, 2, 9, 10, or with GELU one per slot (slot e), so that no slot's
    // VALU work outlasts an MFMA by much.  bf16: channels 0..15 of the
    // block are swapped and stored in its first stage, 16..31 in its
    // second (one store per stage); MX: codes and scale byte in the second.
    constexpr int SPB = 2;
    constexpr int EP = TM * TN * SPB;  // stages that carry the epilogue
    constexpr int qF01 = GELU ? 7 : 3, qS01 = GELU ? 7 : 6;    // bf16, first half
    constexpr int qF23 = GELU ? 15 : 11, qS23 = GELU ? 15 : 14;  // bf16 second half; MX quantize + store
    static_assert(qS01 % NSLOT >= LPS && qS23 % NSLOT >= LPS, "a block's stores follow its stage's loads");
    // vector-memory stores issued by peeled stage kt
    constexpr auto pst = [](int kt) { return kt < 0 || kt >= EP ? 0 : (EB == 2 ? 1 : (kt % 2 == 1 ? 2 : 0)); };
    // Grouped weight scales (GS): wave 0 loads each stage's channel ratios
    // (one more load per stage: XL) into a slot of the stage's ring index
    constexpr int GSL = 1024, XL = GS ? 1 : 0;
    static_assert(NS * STAGE + (2 * NV + 256) * 4 + (GS ? NS * GSL : 0) <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE];
    // Per parity: [BM token scales][BN channel scales][BN bias], then a pad.
    __shared__ __attribute__((aligned(16))) float sc[2 * NV + 256];
    __shared__ __attribute__((aligned(16))) uint8_t gsl[GS ? NS * GSL : 16];

    const uint32_t smem_at = lds_addr(smem), sc_at = lds_addr(sc), gsl_at = lds_addr(gsl);
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    const int wid_u = __builtin_amdgcn_readfirstlane(wid);
    const int G = gridDim.x, w = blockIdx.x, ntiles = tiles_m * tiles_n;
    const int my_n = w < ntiles ? (ntiles - w + G - 1) / G : 0;
    if (my_n == 0) return;  // (uniform) no tile: no descriptor may be built
    const int KT = K / BKB;
    auto tile_of = [&](int i, int *m0, int *n0) {
        int tm, tn;
        xcd_tile(w + i * G, ntiles, tiles_m, tiles_n, &tm, &tn);
        *m0 = tm * BM;
        *n0 = tn * BN;
    };

    // Issue side: the (pass, stage) whose loads go out next.
    int is_i = 0, is_kt = 0, is_m0 = 0, is_n0 = 0;
    tile_of(0, &is_m0, &is_n0);
    __amdgpu_buffer_rsrc_t ra_src, rb_src, rg_src;
    auto set_issue_tile = [&]() {
        ra_src = make_rsrc(A + (size_t)is_m0 * K, __builtin_amdgcn_readfirstlane((uint32_t)(M - is_m0) * (uint32_t)K));
        rb_src = make_rsrc(B + (size_t)is_n0 * K, __builtin_amdgcn_readfirstlane((uint32_t)(N - is_n0) * (uint32_t)K));
        if constexpr (GS)
            rg_src = make_rsrc(gsc + is_n0, __builtin_amdgcn_readfirstlane(
                                                ((uint32_t)KT * (uint32_t)N - (uint32_t)is_n0) * 4u));
    };
    set_issue_tile();
    const uint32_t lrow = (uint32_t)lane / CPR, lslot = (uint32_t)lane % CPR;
    uint32_t a_off[ALD], b_off[BLD];
#pragma unroll
    for (int i = 0; i < ALD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * RPI + lrow;
        a_off[i] = row * (uint32_t)K + dma_slot<BKB>(row, lslot) * 16;
    }
#pragma unroll
    for (int i = 0; i < BLD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * RPI + lrow;
        b_off[i] = row * (uint32_t)K + dma_slot<BKB>(BM + row, lslot) * 16;
    }
    auto piece = [&](int n, int buf) {
        const bool in = is_i < my_n;
        const uint32_t k0 = (uint32_t)is_kt * BKB;
        const uint32_t sbuf = smem_at + (uint32_t)(buf * STAGE);
        if (n < ALD)
            dma16_at(ra_src, sbuf + (n * NW + wid_u) * RPI * BKB, in ? a_off[n < ALD ? n : 0] + k0 : kOob);
        else
            dma16_at(rb_src, sbuf + (BM + ((n - ALD) * NW + wid_u) * RPI) * BKB,
                     in ? b_off[n >= ALD ? n - ALD : 0] + k0 : kOob);
    };
    // Grouped scales: wave 0's load of the issue stage's channel ratios
    // (lane l: channels 4 l .. 4 l + 3 of the issue tile; lanes past the
    // tile's BN channels read nothing), first in the stage's issue order.
    auto ratios = [&](int buf) {
        if constexpr (GS) {
            if (wid_u == 0) {
                const bool ok = is_i < my_n && lane < BN / 4;
                dma16_at(rg_src, gsl_at + (uint32_t)(buf * GSL),
                         ok ? (uint32_t)is_kt * (uint32_t)N * 4u + (uint32_t)lane * 16u : kOob);
            }
        }
    };
    // Wave 0 also waits for each stage's ratio load.
    auto wait_ring = [&](auto NOUT) {
        constexpr int nout = decltype(NOUT)::value;
        if (GS && wid_u == 0)
            wait_vmcnt<nout + XL>();
        else
            wait_vmcnt<nout>();
    };
    auto advance_issue = [&]() {
        if (++is_kt == KT) {
            is_kt = 0;
            if (++is_i < my_n) {
                tile_of(is_i, &is_m0, &is_n0);
                set_issue_tile();
            }
        }
    };
    // A tile's epilogue operands into its parity's slot (wave 1: token
    // scales, wave 2: channel scales, wave 3: bias).
    auto issue_ops = [&](int m0, int n0, uint32_t dst) {
        if (wid_u == 1) {
            const auto r = sa ? make_rsrc(sa + m0, __builtin_amdgcn_readfirstlane((uint32_t)(M - m0) * 4u))
                              : make_rsrc(k_ones, 1024u);
            dma16_at(r, dst, (uint32_t)lane * 16u);
        } else if (wid_u == 2) {
            const auto r = sb ? make_rsrc(sb + n0, __builtin_amdgcn_readfirstlane((uint32_t)(N - n0) * 4u))
                              : make_rsrc(k_ones, 1024u);
            if (lane < BN / 4) dma16_at(r, dst + BM * 4, (uint32_t)lane * 16u);
        } else if (wid_u == 3) {
            const auto r = bias ? make_rsrc(bias + n0, __builtin_amdgcn_readfirstlane((uint32_t)(N - n0) * 4u))
                                : make_rsrc(k_ones, 0u);
            if (lane < BN / 4) dma16_at(r, dst + (BM + BN) * 4, (uint32_t)lane * 16u);
        }
    };

    // ---- epilogue steps of one 32 x 32 block (jb, ib) of a finished tile ----
    const auto ry = make_rsrc(Y, (uint32_t)M * (uint32_t)N * EB);
    const auto rmx = make_rsrc(ymx, EB == 1 ? ((uint32_t)(N / 128 - 1) * (uint32_t)ymx_rows + (uint32_t)M) * 4u : 0u);
    const int l32 = lane & 31, hf = lane >> 5;
    struct Epi {
        float tsc, amax;
        f32x4 cs[4], bs[4];
        float v[16];
        uint32_t w[8];
        int kx;
    };
    auto epi_step = [&](auto Q, auto BLK, Epi &e, const f32x16 (&pv)[TN][TM], const float *scp, int pm0, int pn0,
                        bool live) {
        constexpr int q = decltype(Q)::value, blk = decltype(BLK)::value;
        constexpr int jb = blk / TM, ib = blk % TM;
        // the values this slot computes: [e0, e0 + ne)
        constexpr int e0 = GELU ? q : (q == 1 ? 0 : q == 2 ? 4 : q == 9 ? 8 : 12);
        constexpr int ne = GELU ? 1 : (q == 1 || q == 2 || q == 9 || q == 10 ? 4 : 0);
        const int cb = wn * WN + jb * 32;  // the block's first tile column
        auto ops = [&](int g) {
            const int c = cb + 8 * g + 4 * hf;
            e.cs[g] = *(const f32x4 *)(scp + BM + c);
            e.bs[g] = *(const f32x4 *)(scp + BM + BN + c);
        };
        if constexpr (q == 0) {
            e.tsc = scp[wm * WM + ib * 32 + l32];
            e.amax = 0.0f;
            ops(0);
            ops(1);
        }
        static_for<ne>([&](auto K_) {
            constexpr int el = e0 + decltype(K_)::value, g = el / 4, k = el % 4;
            if constexpr (k == 0 && g + 2 < 4) ops(g + 2);  // two groups ahead
            float t = pv[jb][ib][el] * e.tsc * e.cs[g][k] + e.bs[g][k];
            if constexpr (GELU) t = gelu_tanh_fast(t);
            e.v[el] = t;
            if constexpr (EB == 2) {
                if constexpr (el % 2 == 1) e.w[el / 2] = pack_bf16x2(e.v[el - 1], t);
            } else {
                e.amax = fmaxf(e.amax, fabsf(t));
            }
        });
        const int m = pm0 + wm * WM + ib * 32 + l32, n = pn0 + cb;
        const bool in = live && m < M;
        const uint32_t row = (uint32_t)m * (uint32_t)N + (uint32_t)n;
        if constexpr (EB == 2) {
            // swap lanes l / l + 32 so that lane l holds channels 0..7 (16..23)
            // in w0..w3 (w4..w7) and lane l + 32 channels 8..15 (24..31)
            if constexpr (q == qF01) {
                swap32(e.w[0], e.w[2]);
                swap32(e.w[1], e.w[3]);
            }
            if constexpr (q == qS01)
                buffer_store_x4<LX2V_OV_CP>((u32x4){e.w[0], e.w[1], e.w[2], e.w[3]}, ry,
                                in ? (row + 8u * (uint32_t)hf) * 2u : kOob);
            if constexpr (q == qF23) {
                swap32(e.w[4], e.w[6]);
                swap32(e.w[5], e.w[7]);
            }
            if constexpr (q == qS23)
                buffer_store_x4<LX2V_OV_CP>((u32x4){e.w[4], e.w[5], e.w[6], e.w[7]}, ry,
                                in ? (row + 16u + 8u * (uint32_t)hf) * 2u : kOob);
        } else {
            if constexpr (q == qF23) {
                const float amax = max_pair32(e.amax);
                e.kx = mx_exponent(amax);
                const float msc = mx_scale(e.kx);
#pragma unroll
                for (int g = 0; g < 4; g++) e.w[g] = quant4_sc(e.v + 4 * g, msc);
                // lane l: channels 0..15 as w0, w2, w1, w3; lane l + 32: 16..31
                swap32(e.w[0], e.w[2]);
                swap32(e.w[1], e.w[3]);
            }
            if constexpr (q == qS23) {
                buffer_store_x4<LX2V_OV_CP>((u32x4){e.w[0], e.w[2], e.w[1], e.w[3]}, ry, in ? row + 16u * (uint32_t)hf : kOob);
                buffer_store_b8<LX2V_OV_CP>((uint8_t)(e.kx + 127), rmx,
                                in && hf == 0 ? (uint32_t)mx_sidx((size_t)m, (size_t)(n / 32), (size_t)ymx_rows)
                                              : kOob);
            }
        }
    };

    // ---- one stage: MFMAs into ac, the issue stage's loads and the
    // epilogue slots between them ----
    const uint32_t frow = lane & 31, fhalf = (lane >> 5) * 2;
    auto stage = [&](auto FIRST, f32x16 (&ac)[TN][TM], int buf, int dbuf, auto &&slot) {
        const uint8_t *st = smem + buf * STAGE;
        ratios(dbuf);
        static_for<BKB / 64>([&](auto KK) {
            constexpr int kk = decltype(KK)::value;
            i32x8 af[TM], bf[TN];
            const uint32_t c0 = kk * 4 + fhalf, c1 = c0 + 1;
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint32_t row = wm * WM + i * 32 + frow;
                u32x4 lo = *(const u32x4 *)(st + ((row * BKB + (dma_slot<BKB>(row, c0) << 4)) & AMASK));
                u32x4 hi = *(const u32x4 *)(st + ((row * BKB + (dma_slot<BKB>(row, c1) << 4)) & AMASK));
                af[i] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint32_t row = BM + wn * WN + j * 32 + frow;
                const uint32_t rb = row - BM;
                u32x4 lo = *(const u32x4 *)(st + BM * BKB + ((rb * BKB + (dma_slot<BKB>(row, c0) << 4)) & BMASK));
                u32x4 hi = *(const u32x4 *)(st + BM * BKB + ((rb * BKB + (dma_slot<BKB>(row, c1) << 4)) & BMASK));
                bf[j] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
            static_for<TN * TM>([&](auto JI) {
                constexpr int j = decltype(JI)::value / TM, i = decltype(JI)::value % TM;
                constexpr int n = kk * TN * TM + j * TM + i;
                if constexpr (GS && kk == 0 && !decltype(FIRST)::value) {
                    // the block's sums in units of this stage's group scale
                    // (s_{g-1} / s_g per channel; as k_gemm_fp8_dma)
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const f32x4 r4 =
                            *(const f32x4 *)(gsl + buf * GSL + (wn * WN + j * 32 + 8 * g + 4 * (lane >> 5)) * 4);
#pragma unroll
                        for (int q = 0; q < 4; q++) ac[j][i][4 * g + q] *= r4[q];
                    }
                }
                if constexpr (decltype(FIRST)::value && kk == 0)
                    ac[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], af[i], (f32x16){}, 0, 0, 0, 0,
                                                                               0, 0);
                else
                    ac[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], af[i], ac[j][i], 0, 0, 0, 0,
                                                                               0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (n < LPS) piece(n, dbuf);
                slot(std::integral_constant<int, n>{});
                __builtin_amdgcn_sched_barrier(0);
            });
        });
    };
    static_assert(NSLOT >= LPS, "a stage's loads interleave with its MFMAs");


    f32x16 acc[2][TN][TM];
    Epi e;
    // Prologue: the first NS - 1 stages of the walk.
#pragma unroll
    for (int st = 0; st < NS - 1; st++) {
        ratios(st);
#pragma unroll
        for (int n = 0; n < LPS; n++) piece(n, st);
        advance_issue();
    }
    int s = 0;  // global stage index of this workgroup's walk
    auto tile = [&](auto P, int i) {
        constexpr int p = decltype(P)::value;
        int m0, n0, pm0 = 0, pn0 = 0;
        tile_of(i, &m0, &n0);
        if (i > 0) tile_of(i - 1, &pm0, &pn0);
        const bool live = i > 0;
        const float *scp = sc + (p ^ 1) * NV;
        static_for<EP + 2>([&](auto KT_) {
            constexpr int kt = decltype(KT_)::value;
            // Stage s complete for this wave; then the barrier publishes
            // every wave's part and frees the slot the issue refills.
            wait_ring(std::integral_constant<int, LPS + pst(kt - 1) + pst(kt - 2)>{});
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kt == 0) issue_ops(m0, n0, sc_at + p * NV * 4);
            const int buf = s % NS, dbuf = (s + NS - 1) % NS;
            auto slot = [&](auto NN) {
                if constexpr (kt < EP) {
                    constexpr int q = (kt % SPB) * NSLOT + decltype(NN)::value;
                    epi_step(std::integral_constant<int, q>{}, std::integral_constant<int, kt / SPB>{}, e,
                             acc[p ^ 1], scp, pm0, pn0, live);
                }
            };
            stage(std::integral_constant<bool, kt == 0>{}, acc[p], buf, dbuf, slot);
            advance_issue();
            s++;
            __builtin_amdgcn_sched_barrier(0);
        });
        for (int kt = EP + 2; kt < KT; kt++, s++) {
            wait_ring(std::integral_constant<int, LPS>{});
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            const int buf = s % NS, dbuf = (s + NS - 1) % NS;
            stage(std::false_type{}, acc[p], buf, dbuf, [](auto) {});
            advance_issue();
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    for (int i = 0; i < my_n; i += 2) {
        tile(std::integral_constant<int, 0>{}, i);
        if (i + 1 < my_n) tile(std::integral_constant<int, 1>{}, i + 1);
    }
    // The last tile's epilogue (its operands' DMA went out with its first
    // stage, before ring loads that later waits covered).
    auto last = [&](auto P) {
        constexpr int p = decltype(P)::value;
        int m0, n0;
        tile_of(my_n - 1, &m0, &n0);
        static_for<TN * TM>([&](auto BLK) {
            static_for<NSLOT * SPB>([&](auto Q) { epi_step(Q, BLK, e, acc[p], sc + p * NV, m0, n0, true); });
        });
    };
    if (my_n & 1)
        last(std::integral_constant<int, 0>{});
    else
        last(std::integral_constant<int, 1>{});
    wait_vmcnt<0>();  // the walk's trailing loads (zeros) land before the workgroup ends
}

// ---- persistent 256 x 256 kernel, one wave per SIMD ---------------------------------
//
// Measured on gfx950: one wave issues independent 32x32x64 fp8 MFMAs at the
// full rate (3.6 PF/s on random operands with 4 accumulators in a wave per
// SIMD), but a wave's ds_read_b128 returns at about one per 40 cycles.  So a
// wave that is alone on its SIMD keeps the matrix core busy only if it
// needs at most about one 1 KB fragment read per 64-cycle MFMA: a 128 x 128
// wave tile (16 MFMAs per 64-byte K slice against 16 reads), four of them
// in a 256 x 256 tile.  Per 64 bytes of K the tile then moves 32 KB into LDS
// and 64 KB out of it for 2 x 256 x 256 x 64 FLOPs: half the LDS bytes per
// FLOP of the 8-wave 256 x 128 tile, whose K loop the LDS bounds.
//
// Structure: a grid of min(tiles, CUs) workgroups walking a strided tile
// list (xcd_tile, as k_gemm_fp8_ov); 64-byte K stages in a 4-slot direct-to-
// LDS ring that runs on across tiles (stage g + 3 is loaded while stage g
// is contracted).  The K loop is skewed by one stage: after barrier g each
// wave contracts stage g - 1 from registers while it reads stage g's
// fragments (one ds_read_b128 after each MFMA) and issues stage g + 3's
// loads, so no MFMA waits for LDS.  A tile's token scales, channel scales
// and bias travel by DMA too (waves 0 / 1 / 2 with the tile's first stage;
// wave 3 loads a dummy into a spare slot so every wave issues the same 9
// loads per stage).  The epilogue (scales, bias, GELU, bf16 or MX e4m3)
// runs from registers after the tile's last MFMAs and stores straight to
// memory, lanes l and l + 32 paired by v_permlane32_swap into 32-byte row
// pieces, while the next tile's first three stages load.
//
// vmcnt accounting: every stage issues LPS = 9 loads and every epilogue
// ST stores (stores past M or N go to an out-of-range offset, so the count
// is the same for every lane and tile; a dummy epilogue of ST out-of-range
// stores follows the prologue loads for the first tile).  At the top of
// stage g the loads of g + 1 and g + 2 may still be in flight, and, for the
// first three stages of a tile, the previous tile's stores issued after
// stage g's loads: the waits allow exactly those.
//
// Constraints (host): K % 64 == 0, K / 64 >= 4, N % 256 == 0, M N sizeof(TY)
// < 2^31; bf16 or MX e4m3 output; per-token activations, per-channel weight
// scales; no residual mode.
template <int BKB, int ACT, typename TY>
__global__ __launch_bounds__(256, 1) void k_gemm_fp8_w4(const uint8_t *__restrict__ A, const float *__restrict__ sa,
                                                       const uint8_t *__restrict__ B, const float *__restrict__ sb,
                                                       const float *__restrict__ bias, TY *__restrict__ Y, int M,
                                                       int N, int K, int tiles_m, int tiles_n,
                                                       uint8_t *__restrict__ ymx, int ymx_rows) {
    constexpr int BM = 256, BN = 256, NW = 4, WGN = 2, WM = 128, WN = 128, TM = 4, TN = 4;
    static_assert(BKB == 64 || BKB == 128, "64- or 128-byte K stages");
    constexpr int KK = BKB / 64;                                    // 64-byte K slices per stage
    constexpr int NS = BKB == 64 ? 4 : 2;                           // ring slots (128 KB)
    constexpr int CPR = BKB / 16, RPI = 64 / CPR;                   // tile rows per 1 KB load
    constexpr int ALD = BM / RPI / NW, BLD = BN / RPI / NW;        // ring loads per wave per stage
    constexpr int LPS = ALD + BLD + 1;                              // + the operand / dummy load
    constexpr int STAGE = (BM + BN) * BKB;                          // 32 or 64 KB
    constexpr uint32_t AMASK = BM * BKB - 1, BMASK = BN * BKB - 1;
    constexpr int NV = BM + 2 * BN;  // token scales, channel scales, bias (one set per tile parity)
    constexpr int EB = sizeof(TY);
    static_assert(EB == 1 || EB == 2, "bf16 or MX e4m3 output");
    constexpr bool GELU = ACT == LX2V_ACT_GELU_TANH;
    // stores per epilogue per lane: bf16 two 16-byte stores per 32 x 32
    // block; MX one 16-byte code store and one scale byte
    constexpr int ST = TM * TN * 2;
    constexpr int W4CP = EB == 1 ? LX2V_W4MX_CP : LX2V_W4BF_CP;  // the stores' cache policy
    static_assert((NS - 2) * LPS + ST < 64, "vmcnt range");
    static_assert(NS * STAGE + 2 * NV * 4 + 1024 <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE];
    __shared__ __attribute__((aligned(16))) float sc[2 * NV];
    __shared__ __attribute__((aligned(16))) uint8_t dummy[1024];

    const uint32_t smem_at = lds_addr(smem), sc_at = lds_addr(sc), dummy_at = lds_addr(dummy);
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WGN, wn = wid % WGN;
    const int wid_u = __builtin_amdgcn_readfirstlane(wid);
    const int G = gridDim.x, w = blockIdx.x, ntiles = tiles_m * tiles_n;
    const int my_n = w < ntiles ? (ntiles - w + G - 1) / G : 0;
    if (my_n == 0) return;  // (uniform) no tile: no descriptor may be built
    const int KT = K / BKB;  // (host: K % 128 == 0, so even for 64-byte stages)
    auto tile_of = [&](int i, int *m0, int *n0) {
        int tm, tn;
        xcd_tile(w + i * G, ntiles, tiles_m, tiles_n, &tm, &tn);
        *m0 = tm * BM;
        *n0 = tn * BN;
    };

    // Issue side: the (tile, stage) whose loads go out next.
    int is_i = 0, is_kt = 0, is_m0 = 0, is_n0 = 0;
    tile_of(0, &is_m0, &is_n0);
    __amdgpu_buffer_rsrc_t ra_src, rb_src;
    auto set_issue_tile = [&]() {
        ra_src = make_rsrc(A + (size_t)is_m0 * K, __builtin_amdgcn_readfirstlane((uint32_t)(M - is_m0) * (uint32_t)K));
        rb_src = make_rsrc(B + (size_t)is_n0 * K, __builtin_amdgcn_readfirstlane((uint32_t)(N - is_n0) * (uint32_t)K));
    };
    set_issue_tile();
    const uint32_t lrow = (uint32_t)lane / CPR, lslot = (uint32_t)lane % CPR;
    uint32_t a_off[ALD], b_off[BLD];
#pragma unroll
    for (int i = 0; i < ALD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * RPI + lrow;
        a_off[i] = row * (uint32_t)K + dma_slot<BKB>(row, lslot) * 16;
    }
#pragma unroll
    for (int i = 0; i < BLD; i++) {
        const uint32_t row = (uint32_t)(i * NW + wid) * RPI + lrow;
        b_off[i] = row * (uint32_t)K + dma_slot<BKB>(row, lslot) * 16;
    }
    // Ring load n (0 .. ALD + BLD - 1) of the issue stage into slot buf.
    auto piece = [&](int n, int buf) {
        const bool in = is_i < my_n;
        const uint32_t k0 = (uint32_t)is_kt * BKB;
        const uint32_t sbuf = smem_at + (uint32_t)(buf * STAGE);
        if (n < ALD)
            dma16_at(ra_src, sbuf + (n * NW + wid_u) * RPI * BKB, in ? a_off[n < ALD ? n : 0] + k0 : kOob);
        else
            dma16_at(rb_src, sbuf + BM * BKB + ((n - ALD) * NW + wid_u) * RPI * BKB,
                     in ? b_off[n >= ALD ? n - ALD : 0] + k0 : kOob);
    };
    // The ninth load of a stage: at the issue tile's first stage (three
    // stages before that tile is contracted), wave 0 / 1 / 2 load its token
    // scales / channel scales / bias into the sc set of its parity (a null
    // bias reads zeros); every other ninth load goes to the dummy slot.
    auto ninth = [&]() {
        const bool ops = is_kt == 0 && is_i < my_n && wid_u < 3;
        if (ops) {
            const uint32_t dst = sc_at + (uint32_t)(is_i & 1) * NV * 4u;
            if (wid_u == 0)
                dma16_at(make_rsrc(sa + is_m0, __builtin_amdgcn_readfirstlane((uint32_t)(M - is_m0) * 4u)), dst,
                         (uint32_t)lane * 16u);
            else if (wid_u == 1)
                dma16_at(make_rsrc(sb + is_n0, __builtin_amdgcn_readfirstlane((uint32_t)(N - is_n0) * 4u)),
                         dst + BM * 4, (uint32_t)lane * 16u);
            else
                dma16_at(make_rsrc(bias ? bias + is_n0 : bias,
                                   bias ? __builtin_amdgcn_readfirstlane((uint32_t)(N - is_n0) * 4u) : 0u),
                         dst + (BM + BN) * 4, (uint32_t)lane * 16u);
        } else {
            dma16_at(ra_src, dummy_at, kOob);
        }
    };
    auto advance_issue = [&]() {
        if (++is_kt == KT) {
            is_kt = 0;
            if (++is_i < my_n) {
                tile_of(is_i, &is_m0, &is_n0);
                set_issue_tile();
            }
        }
    };

    // Fragments of one stage: the wave's TM activation row blocks and TN
    // weight row blocks, each 32 rows x 64 bytes as two 16-byte reads
    // (lane half h: chunks 2 h and 2 h + 1 of the row).
    const uint32_t frow = lane & 31, fhalf = (lane >> 5) * 2;
    struct Frag {
        u32x4 a[TM][2], b[TN][2];
    };
    // read m (0 .. 2 (TM + TN) - 1) of slice kk of the stage in slot buf
    auto read_one = [&](int buf, int kk, Frag &f, int m) {
        const uint8_t *st = smem + buf * STAGE;
        const int fi = m >> 1, h = m & 1;
        const uint32_t c = (uint32_t)kk * 4 + fhalf + (uint32_t)h;
        if (fi < TM) {
            const uint32_t row = wm * WM + fi * 32 + frow;
            f.a[fi][h] = *(const u32x4 *)(st + ((row * BKB + (dma_slot<BKB>(row, c) << 4)) & AMASK));
        } else {
            const uint32_t row = wn * WN + (fi - TM) * 32 + frow;
            f.b[fi - TM][h] = *(const u32x4 *)(st + BM * BKB + ((row * BKB + (dma_slot<BKB>(row, c) << 4)) & BMASK));
        }
    };
    auto as8 = [](const u32x4 (&p)[2]) {
        return (i32x8){(int)p[0].x, (int)p[0].y, (int)p[0].z, (int)p[0].w,
                       (int)p[1].x, (int)p[1].y, (int)p[1].z, (int)p[1].w};
    };

    f32x16 acc[TN][TM];
    Frag fr[2];
    // One slice's MFMAs from fc (zero accumulators first when FIRST); after
    // MFMA m, load L0 + m of the issue stage while below L1 (slot dbuf) and,
    // when RD, read m of slice rkk of the stage in slot rbuf into fn.
    auto load = [&](int n, int dbuf) {
        if (n < ALD + BLD)
            piece(n, dbuf);
        else
            ninth();
    };
    auto step = [&](auto FIRST, auto RD, auto L0, auto L1, const Frag &fc, Frag &fn, int rbuf, int rkk, int dbuf) {
        static_for<TN * TM>([&](auto JI) {
            constexpr int m = decltype(JI)::value, j = m / TM, i = m % TM;
            if constexpr (decltype(FIRST)::value)
                acc[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(as8(fc.b[j]), as8(fc.a[i]), (f32x16){}, 0, 0,
                                                                            0, 0, 0, 0);
            else
                acc[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(as8(fc.b[j]), as8(fc.a[i]), acc[j][i], 0, 0,
                                                                            0, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            constexpr int n = decltype(L0)::value + m;
            if constexpr (n < decltype(L1)::value) load(n, dbuf);
            if constexpr (decltype(RD)::value) read_one(rbuf, rkk, fn, m);
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    static_assert(TN * TM == 2 * (TM + TN) && KK * TN * TM >= LPS, "one read after each MFMA; the loads fit");
    using I0 = std::integral_constant<int, 0>;
    using T = std::true_type;
    using F = std::false_type;

    // ---- epilogue of a finished tile, straight from registers ----
    const auto ry = make_rsrc(Y, (uint32_t)M * (uint32_t)N * EB);
    const auto rmx = make_rsrc(ymx, EB == 1 ? ((uint32_t)(N / 128 - 1) * (uint32_t)ymx_rows + (uint32_t)M) * 4u : 0u);
    const int l32 = lane & 31, hf = lane >> 5;
    auto epilogue = [&](const float *sct, int m0, int n0) {
        static_for<TN>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const int cb = wn * WN + j * 32;  // the block's first tile column
            f32x4 cs[4], bs[4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int c = cb + 8 * g + 4 * hf;
                cs[g] = *(const f32x4 *)(sct + BM + c);
                bs[g] = *(const f32x4 *)(sct + BM + BN + c);
            }
            static_for<TM>([&](auto I) {
                constexpr int i = decltype(I)::value;
                const float tsc = sct[wm * WM + i * 32 + l32];
                float v[16];
                float amax = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    float t = acc[j][i][e] * tsc * cs[e / 4][e % 4] + bs[e / 4][e % 4];
                    if constexpr (GELU) t = gelu_tanh_fast(t);
                    v[e] = t;
                    if constexpr (EB == 1) amax = fmaxf(amax, fabsf(t));
                }
                const int m = m0 + wm * WM + i * 32 + l32, n = n0 + cb;
                const bool in = m < M;
                const uint32_t row = (uint32_t)m * (uint32_t)N + (uint32_t)n;
                uint32_t ww[8];
                if constexpr (EB == 2) {
#pragma unroll
                    for (int k = 0; k < 8; k++) ww[k] = pack_bf16x2(v[2 * k], v[2 * k + 1]);
                    // lane l: channels 0..7 (16..23) of the block, lane l + 32: 8..15 (24..31)
                    swap32(ww[0], ww[2]);
                    swap32(ww[1], ww[3]);
                    swap32(ww[4], ww[6]);
                    swap32(ww[5], ww[7]);
                    buffer_store_x4<W4CP>((u32x4){ww[0], ww[1], ww[2], ww[3]}, ry, in ? (row + 8u * (uint32_t)hf) * 2u : kOob);
                    buffer_store_x4<W4CP>((u32x4){ww[4], ww[5], ww[6], ww[7]}, ry,
                                    in ? (row + 16u + 8u * (uint32_t)hf) * 2u : kOob);
                } else {
                    const int kx = mx_exponent(max_pair32(amax));
                    const float msc = mx_scale(kx);
#pragma unroll
                    for (int g = 0; g < 4; g++) ww[g] = quant4_sc(v + 4 * g, msc);
                    // lane l: channels 0..15 as w0, w2, w1, w3; lane l + 32: 16..31
                    swap32(ww[0], ww[2]);
                    swap32(ww[1], ww[3]);
                    buffer_store_x4<W4CP>((u32x4){ww[0], ww[2], ww[1], ww[3]}, ry, in ? row + 16u * (uint32_t)hf : kOob);
                    buffer_store_b8<W4CP>((uint8_t)(kx + 127), rmx,
                                    in && hf == 0 ? (uint32_t)mx_sidx((size_t)m, (size_t)(n / 32), (size_t)ymx_rows)
                                                  : kOob);
                }
            });
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    // Prologue: the first NS - 1 stages, then the dummy epilogue's stores.
#pragma unroll
    for (int st = 0; st < NS - 1; st++) {
#pragma unroll
        for (int n = 0; n < LPS; n++) load(n, st);
        advance_issue();
    }
#pragma unroll
    for (int q = 0; q < ST; q++) buffer_store_b8(0, ry, kOob);

    int g = 0;  // global stage index of this workgroup's walk
    // One stage of the K loop.  The loop is skewed by one 64-byte slice:
    // after barrier g a wave contracts the slice before stage g's first
    // (none at a tile's first stage) while it reads that first slice, then
    // each next slice while reading the one after it.  64-byte stages use
    // the two fragment sets by stage parity P (KT is even), 128-byte stages
    // by slice.
    auto iter = [&](auto P, int kt) {
        constexpr int p = decltype(P)::value;
        if (kt < NS - 1)
            wait_vmcnt_lds0<(NS - 2) * LPS + ST>();
        else
            wait_vmcnt_lds0<(NS - 2) * LPS>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const int buf = g % NS, dbuf = (g + NS - 1) % NS;
        if constexpr (KK == 1) {
            if (kt == 0) {
                // nothing to contract yet: the loads and reads back to back
#pragma unroll
                for (int n = 0; n < LPS; n++) load(n, dbuf);
#pragma unroll
                for (int m = 0; m < 2 * (TM + TN); m++) read_one(buf, 0, fr[p], m);
            } else if (kt == 1) {
                step(T{}, T{}, I0{}, std::integral_constant<int, LPS>{}, fr[p ^ 1], fr[p], buf, 0, dbuf);
            } else {
                step(F{}, T{}, I0{}, std::integral_constant<int, LPS>{}, fr[p ^ 1], fr[p], buf, 0, dbuf);
            }
        } else {
            constexpr int H1 = TN * TM;  // loads of the first slice step
            if (kt == 0) {
#pragma unroll
                for (int n = 0; n < H1; n++) load(n, dbuf);
#pragma unroll
                for (int m = 0; m < 2 * (TM + TN); m++) read_one(buf, 0, fr[0], m);
                step(T{}, T{}, std::integral_constant<int, H1>{}, std::integral_constant<int, LPS>{}, fr[0], fr[1],
                     buf, 1, dbuf);
            } else {
                step(F{}, T{}, I0{}, std::integral_constant<int, H1>{}, fr[1], fr[0], buf, 0, dbuf);
                step(F{}, T{}, std::integral_constant<int, H1>{}, std::integral_constant<int, LPS>{}, fr[0], fr[1],
                     buf, 1, dbuf);
            }
        }
        advance_issue();
        g++;
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int t = 0; t < my_n; t++) {
        int m0, n0;
        tile_of(t, &m0, &n0);
        if constexpr (KK == 1) {
            for (int kt = 0; kt < KT; kt += 2) {
                iter(std::integral_constant<int, 0>{}, kt);
                iter(std::integral_constant<int, 1>{}, kt + 1);
            }
        } else {
            for (int kt = 0; kt < KT; kt++) iter(I0{}, kt);
        }
        // the tile's last slice (set 1), from registers, then its epilogue
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): its fragments
        step(F{}, F{}, I0{}, I0{}, fr[1], fr[0], 0, 0, 0);
        epilogue(sc + (t & 1) * NV, m0, n0);
    }
    wait_vmcnt<0>();  // the walk's trailing loads (zeros) land before the workgroup ends
}

// ---- ping-pong kernel: two wave groups alternate MFMA and LDS phases ---------------
//
// Measured on gfx950: a ds_read_b128 costs its own wave ~25 MFMA cycles of
// issue, but does not slow the MFMAs of the other wave on the same SIMD.
// So the 8 waves of a 256 x BN tile form two groups of four (waves w and
// w + 4 share a SIMD); every phase one group issues the MFMAs of one LDS
// stage (BKB bytes of K) for its 128 x BN half while the other group reads
// its fragments of the next stage, and a barrier swaps the roles.  Group 0
// also issues the direct-to-LDS loads of stage S + NS - 1 in its read phase
// of stage S (an NS-stage ring), and waits for stage S + 1 at the end of its
// following MFMA phase:
//
//   phase 2S:   group 0 reads stage S (+ loads S + NS - 1);  group 1 computes S - 1
//   phase 2S+1: group 0 computes S (then waits for S + 1);   group 1 reads S
//
// so a load has 2 NS - 2 phases to land.  Group g owns tile rows
// 128 g .. 128 g + 127, split GM x GN over its four waves.

template <int BN, int GM, int GN, int BKB, int NS, typename TY>
__global__ __launch_bounds__(512, 1) void k_gemm_fp8_pp(const uint8_t *__restrict__ A,
                                                       const float *__restrict__ sa,
                                                       const uint8_t *__restrict__ B,
                                                       const float *__restrict__ sb,
                                                       const float *__restrict__ bias,
                                                       TY *__restrict__ Y, int M, int N, int K, int act,
                                                       int tiles_m, int tiles_n) {
    constexpr int BM = 256;
    static_assert(GM * GN == 4, "four waves per group");
    constexpr int WM = BM / 2 / GM, WN = BN / GN, TM = WM / 32, TN = WN / 32, KK = BKB / 64;
    constexpr int NF = KK * (TM + TN);        // fragments per read phase
    constexpr int STAGE = (BM + BN) * BKB;
    constexpr int CPR = BKB / 16;             // 16-byte chunks per tile row
    constexpr int RPI = 64 / CPR;             // tile rows per 1 KB load
    constexpr int LPW = (BM + BN) / RPI / 4;  // loads per group-0 wave per stage
    constexpr int AJ = BM / RPI / 4;          // the first AJ of them are activation rows
    static_assert(AJ * RPI * 4 == BM && LPW * RPI * 4 == BM + BN, "stage rows must split over four waves");
    using Ops = TileOps<BM, BN, 512>;
    static_assert(NS >= 2 && NS * STAGE + Ops::NV * 4 <= 160 * 1024 && (NS - 2) * LPW < 64, "LDS ring / vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE];
    __shared__ __attribute__((aligned(16))) float sc[Ops::NV];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wid >> 2, q = wid & 3, wm = q / GN, wn = q % GN;
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KT = K / BKB;
    Ops ops;
    ops.load(tid, m0, n0, M, N, sa, sb, bias);

    const auto ra_src = make_rsrc(A + (size_t)m0 * K, (uint32_t)(M - m0) * (uint32_t)K);
    const auto rb_src = make_rsrc(B + (size_t)n0 * K, (uint32_t)(N - n0) * (uint32_t)K);

    // Load j of a group-0 wave fills 1 KB block b = 4 j + q of the stage
    // (activation rows for j < AJ, weight rows after).  The swizzle repeats
    // every 16 rows and 4 RPI is a multiple of 16, so one lane offset serves
    // every j.
    const uint32_t lrow = (uint32_t)lane / CPR, lslot = (uint32_t)lane % CPR;
    const uint32_t g_lane = ((uint32_t)q * RPI + lrow) * (uint32_t)K + dma_slot<BKB>((uint32_t)q * RPI + lrow, lslot) * 16;
    const uint32_t g_step = 4u * RPI * (uint32_t)K;
    auto load_stage = [&](int ss) {
        uint8_t *base = smem + (ss % NS) * STAGE;
        const bool in = ss < KT;
        const uint32_t k0 = (uint32_t)ss * BKB;
#pragma unroll
        for (int j = 0; j < LPW; j++) {
            const bool isa = j < AJ;
            const uint32_t off = in ? g_lane + (uint32_t)(isa ? j : j - AJ) * g_step + k0 : kOob;
            dma16(isa ? ra_src : rb_src, base + (j * 4 + q) * RPI * BKB, off);
        }
    };

    // Fragment rows are (multiple of 32) + lane % 32, so their swizzle bits
    // depend on the lane only: one byte offset per chunk pair and kk.
    const uint32_t frow = lane & 31, fhalf = (lane >> 5) * 2;
    uint32_t f_lane[KK][2];
#pragma unroll
    for (int kk = 0; kk < KK; kk++)
#pragma unroll
        for (int h = 0; h < 2; h++)
            f_lane[kk][h] = frow * BKB + (dma_slot<BKB>(frow, (uint32_t)kk * 4 + fhalf + h) << 4);
    i32x8 fr[NF];
    auto read_frags = [&](int ss) {
        const uint8_t *base = smem + (ss % NS) * STAGE;
#pragma unroll
        for (int f = 0; f < NF; f++) {
            const int kk = f / (TM + TN), blk = f % (TM + TN);
            const int row0 = blk < TM ? grp * (BM / 2) + wm * WM + blk * 32 : BM + wn * WN + (blk - TM) * 32;
            const uint8_t *rp = base + row0 * BKB;
            const u32x4 lo = *(const u32x4 *)(rp + f_lane[kk][0]);
            const u32x4 hi = *(const u32x4 *)(rp + f_lane[kk][1]);
            fr[f] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int i = 0; i < TM; i++) acc[j][i] = (f32x16){};

    // Prologue: stages 0 .. NS - 2 issued, stage 0 in LDS.
    if (grp == 0) {
#pragma unroll
        for (int st = 0; st < NS - 1; st++) load_stage(st);
        wait_vmcnt<(NS - 2) * LPW>();
    }
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // Phases 0 .. 2 KT, each closed by a barrier; group 1 runs one phase
    // behind (an idle phase 0 first).  The loop body is the same straight
    // line for both groups, so the accumulators never cross a branch.
    if (grp == 1) {
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int ss = 0; ss < KT; ss++) {
        if (grp == 0) load_stage(ss + NS - 1);  // its buffer held stage ss - 1: read by both groups already
        read_frags(ss);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): fragments in registers
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < KK; kk++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int i = 0; i < TM; i++)
                    acc[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        fr[kk * (TM + TN) + TM + j], fr[kk * (TM + TN) + i], acc[j][i], 0, 0, 0, 0, 0, 0);
        if (grp == 0) wait_vmcnt<(NS - 2) * LPW>();  // stage ss + 1 landed (group 0 issues every load)
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }
    if (grp == 0) __builtin_amdgcn_s_barrier();
    ops.park(sc, tid, m0, n0, M, N, sa, sb);
    // no residual mode here: its prefetch registers would spill this tile
    staged_epilogue<BM, BN, 512, NS * STAGE, TM, TN, TY, false, -1, true, kStagedCP>(
        acc, smem, sc, grp * (BM / 2) + wm * WM, wn * WN, tid, lane, m0, n0, M, N, act, Y);
}

template <int BN, int GM, int GN, int BKB, int NS>
void launch_pp(hipStream_t s, const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
               const float *bias, int act, void *y, int y_dtype, int M, int N, int K) {
    int tiles_m = (M + 255) / 256, tiles_n = (N + BN - 1) / BN;
    dim3 grid(tiles_m * tiles_n), block(512);
    if (y_dtype == LX2V_DTYPE_BF16)
        hipLaunchKernelGGL((k_gemm_fp8_pp<BN, GM, GN, BKB, NS, uint16_t>), grid, block, 0, s, a, sa, b, sb, bias,
                           (uint16_t *)y, M, N, K, act, tiles_m, tiles_n);
    else
        hipLaunchKernelGGL((k_gemm_fp8_pp<BN, GM, GN, BKB, NS, float>), grid, block, 0, s, a, sa, b, sb, bias,
                           (float *)y, M, N, K, act, tiles_m, tiles_n);
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

// MXOUT / MXIN: also instantiate the MX-output / MX-activation kernels (only
// for the configurations the planner offers such shapes to).
template <int BM, int BN, int WGM, int WGN, int BKB, int NS, int OCC = 1, bool MXOUT = false, bool MXIN = false,
          bool GSC = false>
void launch_dma(hipStream_t s, const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
                const float *bias, int act, void *y, int y_dtype, int M, int N, int K, const Fp8Mx &mx,
                int splits = 1) {
    int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    dim3 grid(tiles_m * tiles_n, splits), block(64 * WGM * WGN);
    const uint32_t alen = (uint32_t)mx.a_len;
    const int arows = (int)mx.a_rows, yrows = (int)mx.y_rows;
#define LX2V_DMA_A(AMV, GSV, ACTV, T)                                                                           \
    hipLaunchKernelGGL((k_gemm_fp8_dma<BM, BN, WGM, WGN, BKB, NS, OCC, AMV, GSV, ACTV, T>), grid, block, 0, s, a, sa, \
                       b, sb, bias, (T *)y, M, N, K, act, tiles_m, tiles_n, mx.a, alen, arows, mx.y,             \
                       yrows, mx.gate, mx.wgs)
#define LX2V_DMA_G(AMV, GSV, T)                       \
    do {                                              \
        if (act == LX2V_ACT_GELU_TANH)                \
            LX2V_DMA_A(AMV, GSV, LX2V_ACT_GELU_TANH, T); \
        else                                          \
            LX2V_DMA_A(AMV, GSV, LX2V_ACT_NONE, T);      \
    } while (0)
#define LX2V_DMA(AMV, T) LX2V_DMA_G(AMV, 0, T)
    if constexpr (GSC && MXIN) {
        if (mx.wgs && mx.a) {
            if (y_dtype == LX2V_DTYPE_BF16)
                LX2V_DMA_G(1, 1, uint16_t);
            else if (y_dtype == LX2V_DTYPE_F32)
                LX2V_DMA_G(1, 1, float);
            else
                LX2V_DMA_G(1, 1, uint8_t);
            return;
        }
    }
    if constexpr (GSC) {
        if (mx.wgs) {
            if (y_dtype == LX2V_DTYPE_BF16)
                LX2V_DMA_G(0, 1, uint16_t);
            else if (y_dtype == LX2V_DTYPE_F32)
                LX2V_DMA_G(0, 1, float);
            else if constexpr (MXOUT)
                LX2V_DMA_G(0, 1, uint8_t);
            return;
        }
    }
    if constexpr (MXIN) {
        if (mx.a) {
            if (y_dtype == LX2V_DTYPE_BF16)
                LX2V_DMA(1, uint16_t);
            else if (y_dtype == LX2V_DTYPE_F32)
                LX2V_DMA(1, float);
            else
                LX2V_DMA(1, uint8_t);
            return;
        }
    }
    if constexpr (MXOUT) {
        if (y_dtype == LX2V_DTYPE_MXE4M3) {
            LX2V_DMA(0, uint8_t);
            return;
        }
    }
    if (y_dtype == LX2V_DTYPE_BF16)
        LX2V_DMA(0, uint16_t);
    else
        LX2V_DMA(0, float);
#undef LX2V_DMA
#undef LX2V_DMA_G
#undef LX2V_DMA_A
}


// The persistent 256 x 128 kernel: min(tiles, CUs) workgroups (a multiple
// of 8 whenever the tiles outnumber the CUs) walking the tiles.
void launch_pt(hipStream_t s, int num_cu, const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
               const float *bias, int act, void *y, int y_dtype, int M, int N, int K, const Fp8Mx &mx) {
    const int tiles_m = (M + 255) / 256, tiles_n = (N + 127) / 128, nt = tiles_m * tiles_n;
    int g = nt < num_cu ? nt : num_cu;
    if (g < nt && g >= 8) g = g / 8 * 8;
    const dim3 grid(g), block(512);
    const int yr = (int)mx.y_rows;
#define LX2V_PT(GSV, ACTV, T)                                                                                      \
    hipLaunchKernelGGL((k_gemm_fp8_pt<GSV, ACTV, T>), grid, block, 0, s, a, sa, b, sb, bias, (T *)y,                 \
                       M, N, K, act, tiles_m, tiles_n, mx.y, yr, mx.wgs)
#define LX2V_PT_T(GSV, T)                          \
    do {                                           \
        if (act == LX2V_ACT_GELU_TANH)             \
            LX2V_PT(GSV, LX2V_ACT_GELU_TANH, T);   \
        else                                       \
            LX2V_PT(GSV, LX2V_ACT_NONE, T);        \
    } while (0)
#define LX2V_PT_Y(GSV)                                \
    do {                                              \
        if (y_dtype == LX2V_DTYPE_BF16)               \
            LX2V_PT_T(GSV, uint16_t);                 \
        else if (y_dtype == LX2V_DTYPE_F32)           \
            LX2V_PT_T(GSV, float);                    \
        else                                          \
            LX2V_PT_T(GSV, uint8_t);                  \
    } while (0)
    if (mx.wgs)
        LX2V_PT_Y(1);
    else
        LX2V_PT_Y(0);
#undef LX2V_PT_Y
#undef LX2V_PT_T
#undef LX2V_PT
}

// The persistent kernel with the overlapped epilogue: min(tiles, CUs)
// workgroups (a multiple of 8 whenever the tiles outnumber the CUs).
void launch_ov(hipStream_t s, int num_cu, const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
               const float *bias, int act, void *y, int y_dtype, int M, int N, int K, const Fp8Mx &mx) {
    const int tiles_m = (M + 255) / 256, tiles_n = N / 128, nt = tiles_m * tiles_n;
    int g = nt < num_cu ? nt : num_cu;
    if (g < nt && g >= 8) g = g / 8 * 8;
    const dim3 grid(g), block(512);
    const int yr = (int)mx.y_rows;
#define LX2V_OV_G(ACTV, T, GSV)                                                                                  \
    hipLaunchKernelGGL((k_gemm_fp8_ov<ACTV, T, GSV>), grid, block, 0, s, a, sa, b, sb, bias, (T *)y, M, N, K, tiles_m, \
                       tiles_n, mx.y, yr, mx.wgs)
#define LX2V_OV(ACTV, T)              \
    do {                              \
        if (mx.wgs)                   \
            LX2V_OV_G(ACTV, T, 1);    \
        else                          \
            LX2V_OV_G(ACTV, T, 0);    \
    } while (0)
    if (y_dtype == LX2V_DTYPE_BF16) {
        if (act == LX2V_ACT_GELU_TANH)
            LX2V_OV(LX2V_ACT_GELU_TANH, uint16_t);
        else
            LX2V_OV(LX2V_ACT_NONE, uint16_t);
    } else {
        if (act == LX2V_ACT_GELU_TANH)
            LX2V_OV(LX2V_ACT_GELU_TANH, uint8_t);
        else
            LX2V_OV(LX2V_ACT_NONE, uint8_t);
    }
#undef LX2V_OV
#undef LX2V_OV_G
}

// The persistent 256 x 256 kernel with one wave per SIMD: min(tiles, CUs)
// workgroups (a multiple of 8 whenever the tiles outnumber the CUs).
template <int BKB>
void launch_w4(hipStream_t s, int num_cu, const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
               const float *bias, int act, void *y, int y_dtype, int M, int N, int K, const Fp8Mx &mx) {
    const int tiles_m = (M + 255) / 256, tiles_n = N / 256, nt = tiles_m * tiles_n;
    int g = nt < num_cu ? nt : num_cu;
    if (g < nt && g >= 8) g = g / 8 * 8;
    const dim3 grid(g), block(256);
    const int yr = (int)mx.y_rows;
#define LX2V_W4(ACTV, T)                                                                                      \
    hipLaunchKernelGGL((k_gemm_fp8_w4<BKB, ACTV, T>), grid, block, 0, s, a, sa, b, sb, bias, (T *)y, M, N, K, tiles_m, \
                       tiles_n, mx.y, yr)
    if (y_dtype == LX2V_DTYPE_BF16) {
        if (act == LX2V_ACT_GELU_TANH)
            LX2V_W4(LX2V_ACT_GELU_TANH, uint16_t);
        else
            LX2V_W4(LX2V_ACT_NONE, uint16_t);
    } else {
        if (act == LX2V_ACT_GELU_TANH)
            LX2V_W4(LX2V_ACT_GELU_TANH, uint8_t);
        else
            LX2V_W4(LX2V_ACT_NONE, uint8_t);
    }
#undef LX2V_W4
}

// Direct-to-LDS configurations: tile (activation rows x channels), wave
// grid, K bytes per stage, stages.
struct DmaCfg {
    int bm, bn, wgm, wgn, bk, ns;
};
constexpr DmaCfg kDma[] = {
    // direct-to-LDS (k_gemm_fp8_dma)
    {256, 128, 4, 2, 128, 3},  // 0: one workgroup per CU
    {128, 256, 2, 4, 128, 3},  // 1: one per CU
    {256, 128, 4, 2, 64, 3},   // 2: two per CU
    {128, 128, 2, 2, 64, 3},   // 3: three per CU (4 waves)
    {128, 256, 2, 4, 64, 3},   // 4: two per CU
    // ping-pong (k_gemm_fp8_pp); wgm x wgn = one group's waves
    {256, 256, 1, 4, 64, 4},   // 5
    // persistent 256 x 128 (k_gemm_fp8_pt)
    {256, 128, 4, 2, 128, 3},  // 6
    // persistent 256 x 128, epilogue overlapped with the next tile (k_gemm_fp8_ov)
    {256, 128, 4, 2, 128, 3},  // 7
    // persistent 256 x 256, one wave per SIMD (k_gemm_fp8_w4)
    {256, 256, 2, 2, 64, 4},   // 8: 64-byte stages, 4 slots
    {256, 256, 2, 2, 128, 2},  // 9: 128-byte stages, 2 slots
    // direct-to-LDS 128 x 128, 128-byte stages, one per CU (few tiles; with
    // grouped scales on a 4 x 2 wave grid)
    {128, 128, 2, 2, 128, 3},  // 10
};

// Split K's second pass: y = act(sum_p part[p] * sa[m] * sb[n] + b[n]) in
// the direct epilogue's order of operations, stored as F32, BF16 or MX e4m3
// (a thread per 4 consecutive channels, so a 32-channel MX block is 8
// consecutive lanes).  N % 32 == 0.
template <int ACT, typename TY>
__global__ __launch_bounds__(256) void k_gemm_splitk_reduce(const float *__restrict__ part, int S, int M, int N,
                                                          const float *__restrict__ sa, const float *__restrict__ sb,
                                                          const float *__restrict__ bias, TY *__restrict__ Y,
                                                          uint8_t *__restrict__ ymx, int ymx_rows) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x, nq = (size_t)N / 4;
    const bool live = t < (size_t)M * nq;
    const size_t tt = live ? t : 0;
    const int m = (int)(tt / nq), c = (int)(tt % nq) * 4;
    const size_t off = (size_t)m * N + c;
    f32x4 acc = *(const f32x4 *)(part + off);
    for (int p = 1; p < S; p++) {
        const f32x4 a = *(const f32x4 *)(part + (size_t)p * M * N + off);
        acc = (f32x4){acc.x + a.x, acc.y + a.y, acc.z + a.z, acc.w + a.w};
    }
    const float am = sa ? sa[m] : 1.0f;
    const f32x4 s4 = sb ? *(const f32x4 *)(sb + c) : (f32x4){1.0f, 1.0f, 1.0f, 1.0f};
    const f32x4 b4 = bias ? *(const f32x4 *)(bias + c) : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    float v[4] = {acc.x * am * s4.x + b4.x, acc.y * am * s4.y + b4.y, acc.z * am * s4.z + b4.z,
                  acc.w * am * s4.w + b4.w};
    if constexpr (ACT == LX2V_ACT_GELU_TANH)
#pragma unroll
        for (int q = 0; q < 4; q++) v[q] = gelu_tanh_fast(v[q]);
    if constexpr (sizeof(TY) == 1) {
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
        const int k = mx_exponent(amax);
        const float inv = mx_inv(k);
        if (!live) return;
        *(uint32_t *)((uint8_t *)Y + off) = quant4(v, inv);
        if (c % 32 == 0) ymx[mx_sidx(m, c / 32, ymx_rows)] = (uint8_t)(k + 127);
    } else if constexpr (sizeof(TY) == 2) {
        if (!live) return;
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        *(u32x2_t *)((uint16_t *)Y + off) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    } else {
        if (!live) return;
        *(f32x4 *)((float *)Y + off) = (f32x4){v[0], v[1], v[2], v[3]};
    }
}

void launch_splitk_reduce(hipStream_t s, const float *part, int S, int M, int N, const float *sa, const float *sb,
                          const float *bias, int act, void *y, int y_dtype, uint8_t *ymx, int ymx_rows) {
    const size_t n = (size_t)M * (N / 4);
    const dim3 grid((unsigned)((n + 255) / 256));
#define LX2V_RED(ACTV, T)                                                                                          \
    hipLaunchKernelGGL((k_gemm_splitk_reduce<ACTV, T>), grid, dim3(256), 0, s, part, S, M, N, sa, sb, bias, (T *)y, \
                       ymx, ymx_rows)
#define LX2V_RED_T(ACTV)                                  \
    do {                                                  \
        if (y_dtype == LX2V_DTYPE_BF16)                   \
            LX2V_RED(ACTV, uint16_t);                     \
        else if (y_dtype == LX2V_DTYPE_MXE4M3)            \
            LX2V_RED(ACTV, uint8_t);                      \
        else                                              \
            LX2V_RED(ACTV, float);                        \
    } while (0)
    if (act == LX2V_ACT_GELU_TANH)
        LX2V_RED_T(LX2V_ACT_GELU_TANH);
    else
        LX2V_RED_T(LX2V_ACT_NONE);
#undef LX2V_RED_T
#undef LX2V_RED
}

void launch_dma_idx(int idx, hipStream_t s, const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
                    const float *bias, int act, void *y, int y_dtype, int M, int N, int K, const Fp8Mx &mx) {
    switch (idx) {
        case 0:
            launch_dma<256, 128, 4, 2, 128, 3, 1, true, true, true>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K,
                                                                    mx);
            break;
        case 1:
            launch_dma<128, 256, 2, 4, 128, 3, 1, true, true, true>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K,
                                                                    mx);
            break;
        case 2: launch_dma<256, 128, 4, 2, 64, 3, 2>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K, mx); break;
        case 3:
            launch_dma<128, 128, 2, 2, 64, 3, 3, true, true>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K, mx);
            break;
        case 4:
            launch_dma<128, 256, 2, 4, 64, 3, 2, true, false>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K, mx);
            break;
        case 5: launch_pp<256, 1, 4, 64, 4>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K); break;
        case 10:
            // grouped scales on eight waves (two per SIMD): with four, the
            // accumulators sit in AGPRs and each rescale multiply takes a
            // read and a write besides (kv2 12.4 -> 9.7 us, 880 x 14336 ->
            // 3072 76 -> 51 us); per-channel, four waves are as fast or faster
            if (mx.wgs)
                launch_dma<128, 128, 4, 2, 128, 3, 1, false, false, true>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N,
                                                                          K, mx);
            else
                launch_dma<128, 128, 2, 2, 128, 3, 1>(s, a, sa, b, sb, bias, act, y, y_dtype, M, N, K, mx);
            break;
        default: break;  // 6 .. 9: launch_pt / launch_ov / launch_w4 (need the CU count)
    }
}

// Tuning override: LIGHTX2V_HIP_FP8_CFG=<index into kDma> forces one
// direct-to-LDS configuration (-1 or unset: automatic).  Read on every
// plan, so a process (or a test) can change it between calls.
int forced_cfg() {
    const char *e = getenv("LIGHTX2V_HIP_FP8_CFG");
    return e ? atoi(e) : -1;
}

}  // namespace

bool gemm_fp8_residual_ok(const Fp8Plan &p) {
    return p.kernel >= 0 && p.kernel != 5 && p.kernel != 6 && p.kernel != 7 && p.kernel != 8 && p.kernel != 9;
}

bool gemm_fp8_grouped_supported(size_t M, size_t N, size_t K, size_t group) {
    return group == 128 && K % 128 == 0 && N % 4 == 0 && gemm_fp8_supported(M, N, K) &&
           (K / 64) * N * 4 < (1ull << 31);
}

bool gemm_fp8_supported(size_t M, size_t N, size_t K) {
    // 32-bit buffer offsets (the out-of-range offset 2^31 must stay past
    // the end); K a multiple of 16 (the 16-byte chunk loads).
    return M > 0 && N > 0 && K >= 16 && K % 16 == 0 && M * K < (1ull << 31) &&
           N * K < (1ull << 31) && M < (1u << 30) && N < (1u << 30);
}

// Time model of the K % 128 == 0 configurations, fitted (least squares)
// to measured launch times at 19 shapes: the Wan ones (M 512..4680, K
// 1536..14336, N 1536..14336) and 256..9360-row, 1024..4096-square ones:
//   t = per_stage * rounds * stages + per_round * rounds + fixed,
// rounds = ceil(tiles / CUs), stages = K / 128.  The configurations that
// fit two or three workgroups per CU pay a slower K loop (64-byte stages)
// but hide most of each workgroup's prologue and epilogue behind another's
// K loop; the 256 x 256 ping-pong tile has the cheapest K loop per unit of
// work and the most expensive rounds.
//
// The persistent kernels (6, 7) are offered only to shapes of two or more
// rounds: with one tile per workgroup there is nothing to overlap, and they
// measured no faster than the one-shot tiles there.  Their costs are per
// pass of a workgroup over its tiles (the same rounds count), measured on
// the Wan shapes: 7 (epilogue folded into the next tile) at 256 x 128 x
// 1536 tiles -- FFN up 6 passes 75 us, QKV 3 passes 38 us; with grouped
// scales 6 and 7 within 2% of each other at QKV (43-46 us) and the 30-layer
// K / V call (87-96 us), 7 ahead at FFN up (94 against 102 us).
//
// The one-per-CU tiles with 128-byte stages (0, 1, 10) have an occupancy
// term instead: their stages slow down with the share of CUs loading at
// once, so round r costs stages x (per_stage + occ_stage x busy_r) +
// per_round, busy_r the share of CUs with a tile in round r.  Fitted to
// launch times at 4680 x 1536 -> 1536, 4680 x 8960 -> 1536, 512 x 1536 ->
// 3072 and config 5's 2640- and 880-row shapes (256 x 128 and 128 x 256:
// 0.40 + 0.38 busy us per stage, 0.53 at a third of the CUs, 0.77 at all;
// 128 x 128: 0.26 + 0.18 busy): the 128 x 256 tile (1) fits 2640 rows
// into one round of 252 tiles where 256 x 128 needs two of 264 (2640 x
// 3072 -> 3072: 24.8 against 40.4 us; 2640 x 14336 -> 3072: 92.8 against
// 104.8 us on the 128 x 128 tile), and at 4680 rows it runs 222 tiles
// against 228 (cross-attention Q 13.6 against 14.3 us).
struct CfgCost {
    int idx;
    double per_stage_us, per_round_us, fixed_us;
    bool persistent;
    double occ_stage_us = 0.0;
};
constexpr CfgCost kAuto[] = {
    {0, 0.40, 5.30, 0.0, false, 0.38},  // 256 x 128, one workgroup per CU
    {1, 0.40, 5.00, 0.0, false, 0.38},  // 128 x 256, one per CU
    {2, 0.826, 4.21, 2.44, false},      // 256 x 128, two per CU
    {4, 0.926, 2.43, 4.47, false},      // 128 x 256, two per CU
    {3, 0.606, 0.44, 4.59, false},      // 128 x 128, three per CU
    {5, 1.40, 14.77, 0.0, false},       // 256 x 256 ping-pong (8192^3: 1.44 us per stage with every CU busy)
    {7, 0.80, 2.70, 0.80, true},        // 256 x 128 persistent, overlapped epilogue
    // 128 x 128, 128-byte stages, one per CU: 512 x 1536 -> 3072 7.8 us,
    // 880 x 14336 -> 3072 45 us (64 on the 256 x 128 or 128 x 256 tile)
    {10, 0.26, 4.00, 0.0, false, 0.18},
};
// Grouped weight scales (128-byte stages only): the one-per-CU tiles and
// the persistent 256 x 128 tiles, fitted to forced-configuration times at
// the Wan 2.1 and 2.2 shapes.  The one-per-CU tiles take the transposed
// layout (one ratio read per block) for bf16 / f32 output -- the 128 x 256
// tile then runs 4680 x 8960 -> 1536 at 62.8 us and 2640 x 14336 -> 3072 at
// 104 us, the eight-wave 128 x 128 one 880 x 14336 -> 3072 at 51 us -- and
// the plain layout for MX output (kGroupedMxOut).
constexpr CfgCost kGroupedAuto[] = {
    {0, 0.584, 5.85, 0.0, false, 0.275},  // 256 x 128
    {1, 0.346, 5.83, 0.0, false, 0.54},   // 128 x 256
    {6, 0.80, 3.50, 4.00, true},          // 256 x 128 persistent
    {7, 1.03, 2.70, 0.80, true},          // 256 x 128 persistent, overlapped epilogue (QKV 46 us, the K / V call 90)
    {10, 0.221, 5.13, 0.0, false, 0.29},  // 128 x 128, eight waves (shapes of few 256 x 128 tiles)
};
constexpr CfgCost kGroupedMxOut[] = {
    {0, 0.61, 5.30, 0.0, false, 0.42},  // 256 x 128
    {1, 0.61, 5.30, 0.0, false, 0.42},  // 128 x 256
    {6, 0.80, 3.50, 4.00, true},
    {7, 1.03, 2.70, 0.80, true},
};
// Modelled time of configuration c at M x N x K (rounds of tiles over num_cu CUs).
double cfg_cost(const CfgCost &c, size_t tiles, size_t num_cu, size_t K) {
    const size_t rounds = (tiles + num_cu - 1) / num_cu;
    const double st = (double)(K / 128);
    if (c.occ_stage_us <= 0.0) return (double)rounds * (st * c.per_stage_us + c.per_round_us) + c.fixed_us;
    double t = c.fixed_us;
    for (size_t r = 0; r < rounds; r++) {
        const size_t left = tiles - r * num_cu;
        const double busy = (double)(left < num_cu ? left : num_cu) / (double)num_cu;
        t += st * (c.per_stage_us + c.occ_stage_us * busy) + c.per_round_us;
    }
    return t;
}

// The configurations with MX-activation / MX-output kernels.  The 128 x 256
// two-per-CU tile takes no MX activations: their scale handling needs more
// than the 128 VGPRs two workgroups per CU leave a wave (its one-per-CU
// version, 1, has 256).
bool mx_capable(int idx, bool mx_in) { return idx <= 1 || idx == 3 || ((idx == 4 || idx == 6) && !mx_in); }
// The configurations built with grouped weight scales (128-byte stages, one
// workgroup per CU: the partial sums need the registers); MX output on the
// 256 x 128 and 128 x 256 tiles, MX activations on the one-shot ones.
bool grouped_capable(int idx, bool mx, bool mx_in) {
    return mx_in ? idx <= 1 : (idx <= 1 || idx == 6 || (idx == 10 && !mx));
}
// The overlapped-epilogue kernel (k_gemm_fp8_ov): per-token activations,
// per-channel or group-128 weight scales, bf16 or MX e4m3 output, whole 128-channel
// tiles, and enough stages to carry the previous tile's epilogue (4, or 8
// with GELU) plus the two the ring runs ahead.
bool ov_capable(size_t M, size_t N, size_t K, bool mx_in, bool grouped, int y_dtype, int act, bool residual) {
    const size_t eb = y_dtype == LX2V_DTYPE_BF16 ? 2 : (y_dtype == LX2V_DTYPE_MXE4M3 ? 1 : 0);
    const size_t ep = act == LX2V_ACT_GELU_TANH ? 8 : 4;
    (void)grouped;  // group-128 scales by the per-stage rescale (k_gemm_fp8_ov GS)
    return eb && !mx_in && !residual && N % 128 == 0 && K % 128 == 0 && K / 128 >= ep + 2 &&
           M * N * eb < (1ull << 31);
}

// The persistent 256 x 256 kernel (k_gemm_fp8_w4): per-token activations and
// per-channel weight scales, bf16 or MX e4m3 output, whole 256-channel
// tiles, K a multiple of 128 with at least four 64-byte stages.
bool w4_capable(size_t M, size_t N, size_t K, bool mx_in, bool grouped, int y_dtype, bool residual) {
    const size_t eb = y_dtype == LX2V_DTYPE_BF16 ? 2 : (y_dtype == LX2V_DTYPE_MXE4M3 ? 1 : 0);
    return eb && !mx_in && !grouped && !residual && N % 256 == 0 && K % 128 == 0 && K / 64 >= 4 &&
           M * N * eb < (1ull << 31);
}

Fp8Plan plan_gemm_fp8(int num_cu, size_t M, size_t N, size_t K, bool mx, bool mx_in, bool grouped, int y_dtype,
                      int act, bool residual, bool allow_split) {
    Fp8Plan p;
    if (K % 128 != 0) return p;  // the register-staged kernel
    // Split K where even the 256 x 128 tiles leave at least half the CUs
    // idle and K is long: S workgroups per tile (S <= CUs / tiles, >= 32
    // stages each, <= 8), their partial sums reduced by a second pass.  The
    // partial sums' store and the reduction cost about 10 us, which only a
    // long K loop repays (880 x 14336 -> 3072: 68.9 -> 51.0 us at S = 2;
    // 880 x 3072 -> 3072: 19.1 -> 23.3 us).  LIGHTX2V_HIP_FP8_SPLITK=0 turns
    // it off, =S forces S where it applies.
    if (allow_split && !mx_in && !grouped && !residual && N % 128 == 0 && forced_cfg() < 0) {
        const char *e = getenv("LIGHTX2V_HIP_FP8_SPLITK");
        const int mode = e ? atoi(e) : -1;
        const size_t tiles = ((M + 255) / 256) * (N / 128), kts = K / 128;
        size_t S = 1;
        if (mode >= 2)
            S = std::min<size_t>((size_t)mode, kts);
        else if (mode != 0 && tiles * 2 <= (size_t)num_cu)
            S = std::min<size_t>(std::min<size_t>((size_t)num_cu / tiles, kts / 32), 8);
        // ... unless the 128 x 128 one-per-CU tile (its 4x the tiles fill the
        // CUs without a reduction) is cheaper by the model below; a forced
        // split count always splits
        bool split = S >= 2 && (size_t)M * N * S * 4 < (1ull << 31);
        if (split && mode < 2 && y_dtype != LX2V_DTYPE_MXE4M3) {  // (no MX output on that tile)
            const size_t t10 = ((M + 127) / 128) * (N / 128);
            const double c10 = cfg_cost(kAuto[sizeof(kAuto) / sizeof(kAuto[0]) - 1], t10, (size_t)num_cu, K);
            // the split's tiles (one round) plus the partials' store and reduction
            const double busy = (double)std::min<size_t>(tiles * S, (size_t)num_cu) / num_cu;
            const double cs = (double)(kts / S) * (0.40 + 0.38 * busy) + 5.3 + 10.0;
            split = cs <= c10;
        }
        if (split) {
            p.kernel = 0;
            p.splits = (int)S;
            return p;
        }
    }
    const int nd = (int)(sizeof(kDma) / sizeof(kDma[0]));
    const int forced = forced_cfg();
    auto ok = [&](int idx) {
        if (residual && (idx == 5 || idx == 6)) return false;
        if (idx == 7) return ov_capable(M, N, K, mx_in, grouped, y_dtype, act, residual);
        if (idx == 8 || idx == 9) return w4_capable(M, N, K, mx_in, grouped, y_dtype, residual);
        return grouped ? grouped_capable(idx, mx, mx_in) : (!mx || mx_capable(idx, mx_in));
    };
    if (forced >= 0 && forced < nd && ok(forced) && (forced != 6 || K >= 256)) {
        p.kernel = forced;
        return p;
    }
    double best = 0.0;
    auto take = [&](int idx, double t) {
        if (p.kernel < 0 || t < best * 0.9999) {  // ties keep the earlier
            best = t;
            p.kernel = idx;
        }
    };
    const bool heavy_epi = y_dtype == LX2V_DTYPE_MXE4M3 || act == LX2V_ACT_GELU_TANH;
    auto consider = [&](const CfgCost &c) {
        if (!ok(c.idx)) return;
        const DmaCfg &d = kDma[c.idx];
        const size_t tiles = ((M + d.bm - 1) / d.bm) * ((N + d.bn - 1) / d.bn);
        const size_t rounds = (tiles + num_cu - 1) / num_cu;
        if (c.persistent && (rounds < 2 || K / 128 < 2)) return;
        // the overlapped epilogue's MX quantization (and GELU) cost per pass;
        // the grouped persistent tile's LDS-staged epilogue does its GELU / MX
        // work after the pass's last stage (measured ~3 us a pass at FFN up)
        const double epi = c.idx == 7 && y_dtype == LX2V_DTYPE_MXE4M3 ? 1.2 : (c.idx == 6 && heavy_epi ? 3.0 : 0.0);
        take(c.idx, cfg_cost(c, tiles, (size_t)num_cu, K) + (double)rounds * epi);
    };
    // The 256 x 256 tile with one wave per SIMD (9).  Its stages slow down
    // with the share of CUs loading at once (measured 1.33-1.36 us per
    // 128-byte stage with every CU busy, 1.07 us with half of them), so a
    // round costs stages x (0.63 + 0.72 occupancy) + its prologue and
    // register-direct epilogue (7 us; 9.5 with GELU or MX output).
    auto consider9 = [&]() {
        if (!ok(9)) return;
        const size_t tiles = ((M + 255) / 256) * (N / 256), full = tiles / num_cu, rem = tiles % num_cu;
        const double st = (double)(K / 128), b = heavy_epi ? 9.5 : 7.0;
        double t = (double)full * (st * (0.63 + 0.72) + b) + 0.5;
        if (rem) t += st * (0.63 + 0.72 * (double)rem / num_cu) + b;
        take(9, t);
    };
    if (grouped) {
        if (y_dtype == LX2V_DTYPE_MXE4M3)
            for (const CfgCost &c : kGroupedMxOut) consider(c);
        else
            for (const CfgCost &c : kGroupedAuto) consider(c);
        return p;
    }
    for (const CfgCost &c : kAuto) consider(c);
    consider9();
    return p;
}

void launch_gemm_fp8(hipStream_t s, int num_cu, const Fp8Plan &p, const uint8_t *a, const float *a_scale,
                     const uint8_t *b, const float *b_scale, const float *bias, int act, void *y,
                     int y_dtype, size_t M, size_t N, size_t K, const Fp8Mx &mx) {
    int m = (int)M, n = (int)N, k = (int)K;
    if (p.splits > 1) {
        // the partial sums without scales or bias, then the reduction
        launch_dma<256, 128, 4, 2, 128, 3, 1, true, true, true>(s, a, nullptr, b, nullptr, nullptr, LX2V_ACT_NONE,
                                                                mx.part, LX2V_DTYPE_F32, m, n, k, Fp8Mx{}, p.splits);
        launch_splitk_reduce(s, mx.part, p.splits, m, n, a_scale, b_scale, bias, act, y, y_dtype, mx.y,
                             (int)mx.y_rows);
        return;
    }
    if (p.kernel == 6) {
        launch_pt(s, num_cu, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k, mx);
        return;
    }
    if (p.kernel == 7) {
        launch_ov(s, num_cu, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k, mx);
        return;
    }
    if (p.kernel == 8 || p.kernel == 9) {
        (p.kernel == 8 ? launch_w4<64> : launch_w4<128>)(s, num_cu, a, a_scale, b, b_scale, bias, act, y, y_dtype, m,
                                                         n, k, mx);
        return;
    }
    if (p.kernel >= 0) {
        launch_dma_idx(p.kernel, s, a, a_scale, b, b_scale, bias, act, y, y_dtype, m, n, k, mx);
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

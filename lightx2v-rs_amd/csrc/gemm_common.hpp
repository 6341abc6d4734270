// gemm_common.hpp -- pieces shared by the gfx950 GEMM kernels: the
// direct-to-LDS 16-byte load, vmcnt waits, the LDS tile swizzle of the DMA
// kernels and the LDS-staged epilogue (token / channel scale, bias, GELU,
// f32 / bf16 / MX e4m3 output).
#pragma once

#include "device_common.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

// One 16-byte-per-lane buffer load straight into LDS at `lds` + 16 * lane
// (M0 carries the wave-uniform LDS address; nothing else in these kernels
// uses M0).  Issued from inline asm rather than the load-to-LDS builtin, so
// the compiler does not track these loads: with the builtin it cannot always
// tell which ring slot a pending load writes and then drains every load
// before a fragment read (once per pass over the ring).  Every user waits
// for its loads itself, with explicit vmcnt waits and barriers.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff) {
    typedef __attribute__((address_space(3))) uint8_t *lds_ptr;
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr)lds);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(base), "v"(voff), "s"(r)
                 : "memory");
}

// The same load given the LDS byte address (kernels that take it once from
// the __shared__ array itself, not through a generic pointer).
__device__ __forceinline__ void dma16_at(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t voff) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(base), "v"(voff), "s"(r)
                 : "memory");
}
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T *p) {
    typedef __attribute__((address_space(3))) uint8_t *lds_ptr;
    return (uint32_t)(uintptr_t)(lds_ptr)(uint8_t *)p;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    // gfx9 s_waitcnt: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8.
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The same wait that also retires every LDS read of this wave (lgkmcnt 0).
template <int N>
__device__ __forceinline__ void wait_vmcnt_lds0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// LDS-staged epilogue, used where the main loop leaves a large LDS ring
// free.  Stage 1 (acc_to_lds): each wave applies the token scale, channel
// scale, bias and GELU (in that order, in f32) and writes the results,
// already in the output type, into a staging tile of R rows x BN columns.
// Stage 2 (lds_to_global, after a barrier): the whole block stores the tile
// with consecutive lanes on consecutive 16-byte chunks of a row, so each
// store instruction writes whole 128-byte lines instead of 16-byte pieces
// of 32 rows.  The 16-byte chunks of staging row r sit at chunk c ^ (r % 16):
// the column-fragment writes of stage 1 (32 rows, one chunk each) and the
// row reads of stage 2 both spread over all 64 banks.  Needs a row of at
// least 16 chunks (BN * sizeof(TY) >= 256).

// Epilogue operands of a BM x BN tile: sc[r] is the token scale of tile row
// r (1 for MX activations or sa == null), sc[BM + c] the channel scale (1
// for sb == null) and sc[BM + BN + c] the bias of tile column c, zero
// outside M x N.  Loaded into registers when the workgroup starts (at most
// three per thread), so their latency hides under the K loop, and parked in
// a small LDS array after it.
template <int BM, int BN, int NT>
struct TileOps {
    static constexpr int NV = BM + 2 * BN, PER = (NV + NT - 1) / NT;
    static_assert(BM % 64 == 0 && BN % 64 == 0 && NT % 64 == 0, "entry kinds must be wave-uniform");
    // v[p]: entry tid + p NT, loaded branch-free (an out-of-range or absent
    // operand reads zero; park() supplies the defaults).  With a conditional
    // load per kind of entry the compiler waits for the first load before
    // the other paths write the same register -- a memory latency before
    // the main loop.  BM, BN and NT are multiples of 64, so one wave's
    // entries are all of one kind and the buffer descriptor is uniform.
    float v[PER];
    __device__ __forceinline__ static int kind(int i) { return i < BM ? 0 : (i < BM + BN ? 1 : 2); }
    __device__ __forceinline__ void load(int tid, int m0, int n0, int M, int N, const float *__restrict__ sa,
                                         const float *__restrict__ sb, const float *__restrict__ bias) {
        const auto ra = make_rsrc(sa ? sa + m0 : sa, sa ? (uint32_t)(M - m0) * 4u : 0u);
        const auto rb = make_rsrc(sb ? sb + n0 : sb, sb ? (uint32_t)(N - n0) * 4u : 0u);
        const auto rc = make_rsrc(bias ? bias + n0 : bias, bias ? (uint32_t)(N - n0) * 4u : 0u);
#pragma unroll
        for (int p = 0; p < PER; p++) {
            const int i = tid + p * NT;
            const int k = __builtin_amdgcn_readfirstlane(kind(i));
            const uint32_t off = (uint32_t)(i - (k == 0 ? 0 : (k == 1 ? BM : BM + BN))) * 4u;
            v[p] = __uint_as_float(buffer_load_x1(k == 0 ? ra : (k == 1 ? rb : rc), i < NV ? off : kOob));
        }
    }
    __device__ __forceinline__ void park(float *sc, int tid, int m0, int n0, int M, int N, const float *sa,
                                         const float *sb) const {
#pragma unroll
        for (int p = 0; p < PER; p++) {
            const int i = tid + p * NT;
            if (i >= NV) continue;
            float x = v[p];
            if (i < BM && !sa) x = m0 + i < M ? 1.0f : 0.0f;
            if (i >= BM && i < BM + BN && !sb) x = n0 + i - BM < N ? 1.0f : 0.0f;
            sc[i] = x;
        }
    }
};

// Staging rows hold BN outputs of TY; their 16-byte chunks are XOR-swizzled
// by row (chunk ^ row % SWZ) so the column-fragment writes of stage 1 (32
// rows, one chunk each) and the row reads of stage 2 spread over the banks.
template <int BN, typename TY>
constexpr int stage_swz() {
    return (BN * (int)sizeof(TY) / 16) < 16 ? BN * (int)sizeof(TY) / 16 : 16;
}

// Where MX output goes besides the codes: E8M0 scale bytes (mx_sidx
// layout, `rows` rows per 128-column group), starting at the output's row 0.
struct MxOut {
    uint8_t *scales = nullptr;
    int rows = 0;
    // Residual mode (bf16 / f32 output only): Y holds the residual stream h
    // and the tile is added in, Y[m][n] = Y[m][n] + y[m][n] * gate[n], with
    // y as the plain epilogue would have stored it.
    const float *gate = nullptr;
};

// Stage 1 of the staged epilogue for one wave: its accumulators, scaled by
// token and channel scale, biased and GELU'd, into the staging tile of a
// pass of R rows, where the wave's tile rows (from wr; columns from wc)
// start at staging row rloc: its 32-row blocks outside [0, R) wait for
// another pass.  TY = uint8_t is MX e4m3 output: each 32-column block of a
// row (one j of one lane pair l, l + 32) gets the scale 2^k of mx_exponent
// over its 32 values; the codes go to the staging tile and the scale byte
// straight to global memory (tile origin m0, n0).
//
// ACT (compile time, so the per-element code is branch-free): GELU or none.
// ALLROWS: the pass covers the whole tile (every block of the wave is in it).
//
// TR: the blocks are transposed (the MFMA took the activations as its first
// operand): lane l holds channel l % 32 of block (i, j) and its tile rows
// 8 g + 4 (l / 32) + q; bf16 / f32 output.  Each element gets the same
// operations in the same order as in the plain layout.
template <int BM, int BN, int TM, int TN, typename TY, int ACT, bool ALLROWS, bool TR = false>
__device__ __forceinline__ void acc_to_lds(const f32x16 (&acc)[TN][TM], const float *sc, uint8_t *stg, int rloc,
                                           int R, int wr, int wc, int lane, MxOut mx, int m0, int n0, int M,
                                           int N) {
    constexpr int EB = sizeof(TY), RB = BN * EB, SWZ = stage_swz<BN, TY>();
    static_assert(RB >= 128 && (RB & (RB - 1)) == 0, "staging row must be a power of two >= 128 bytes");
    const int l32 = lane & 31, hf = lane >> 5;
    if constexpr (TR) {
        static_assert(EB != 1, "transposed blocks: bf16 or f32 output");
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int c = wc + j * 32 + l32, cb = c * EB;
            const float cs = sc[BM + c], bs = sc[BM + BN + c];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                if (!ALLROWS && (rloc + i * 32 < 0 || rloc + i * 32 >= R)) continue;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const f32x4 ts = *(const f32x4 *)(sc + wr + i * 32 + 8 * g + 4 * hf);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        float t = acc[j][i][4 * g + q] * ts[q] * cs + bs;
                        if constexpr (ACT == LX2V_ACT_GELU_TANH) t = gelu_tanh_fast(t);
                        const int r = rloc + i * 32 + 8 * g + 4 * hf + q;
                        uint8_t *p = stg + r * RB + ((((cb >> 4) ^ (r & (SWZ - 1)))) << 4) + (cb & 15);
                        if constexpr (EB == 4)
                            *(float *)p = t;
                        else
                            *(uint16_t *)p = (uint16_t)pack_bf16x2(t, t);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        return;
    }
    float sam[TM];
#pragma unroll
    for (int i = 0; i < TM; i++) sam[i] = sc[wr + i * 32 + l32];
    // A 32-column block's channel scales and biases, read from LDS in one
    // round trip (one per channel group would be serialized by the
    // scheduling barriers that keep the accumulators in place).
    auto col_ops = [&](int j, f32x4 (&s4)[4], f32x4 (&b4)[4]) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int c = wc + j * 32 + 8 * g + 4 * hf;
            s4[g] = *(const f32x4 *)(sc + BM + c);
            b4[g] = *(const f32x4 *)(sc + BM + BN + c);
        }
    };
    if constexpr (EB == 1) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            f32x4 s4[4], b4[4];
            col_ops(j, s4, b4);
#pragma unroll
            for (int i = 0; i < TM; i++) {
                if (!ALLROWS && (rloc + i * 32 < 0 || rloc + i * 32 >= R)) continue;
                float v[16];
                float amax = 0.0f;
#pragma unroll
                for (int g = 0; g < 4; g++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        float t = acc[j][i][4 * g + q] * sam[i] * s4[g][q] + b4[g][q];
                        if constexpr (ACT == LX2V_ACT_GELU_TANH) t = gelu_tanh_fast(t);
                        v[4 * g + q] = t;
                        amax = fmaxf(amax, fabsf(t));
                    }
                amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
                const int k = mx_exponent(amax);
                const float inv = mx_inv(k);
                const int r = rloc + i * 32 + l32;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int cb = wc + j * 32 + 8 * g + 4 * hf;
                    *(uint32_t *)(stg + r * RB + ((((cb >> 4) ^ (r & (SWZ - 1)))) << 4) + (cb & 15)) =
                        quant4(v + 4 * g, inv);
                }
                const int m = m0 + wr + i * 32 + l32, n = n0 + wc + j * 32;
                if (hf == 0 && m < M && n < N) mx.scales[mx_sidx(m, n / 32, mx.rows)] = (uint8_t)(k + 127);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        return;
    }
    // f32 output keeps one group's operands live at a time: the block's
    // would push the two-per-CU tiles past the 128 VGPRs they may use.
    constexpr bool BLOCK_OPS = EB != 4;
#pragma unroll
    for (int j = 0; j < TN; j++) {
        f32x4 s4j[4], b4j[4];
        if constexpr (BLOCK_OPS) col_ops(j, s4j, b4j);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int c = wc + j * 32 + 8 * g + 4 * hf;
            f32x4 s4, b4;
            if constexpr (BLOCK_OPS) {
                s4 = s4j[g];
                b4 = b4j[g];
            } else {
                s4 = *(const f32x4 *)(sc + BM + c);
                b4 = *(const f32x4 *)(sc + BM + BN + c);
            }
            const int cb = c * EB;  // byte column in the row
#pragma unroll
            for (int i = 0; i < TM; i++) {
                if (!ALLROWS && (rloc + i * 32 < 0 || rloc + i * 32 >= R)) continue;
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    v[q] = acc[j][i][4 * g + q] * sam[i] * s4[q] + b4[q];
                    if constexpr (ACT == LX2V_ACT_GELU_TANH) v[q] = gelu_tanh_fast(v[q]);
                }
                const int r = rloc + i * 32 + l32;
                uint8_t *p = stg + r * RB + ((((cb >> 4) ^ (r & (SWZ - 1)))) << 4) + (cb & 15);
                if constexpr (EB == 4) {
                    *(f32x4 *)p = (f32x4){v[0], v[1], v[2], v[3]};
                } else {
                    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
                    *(u32x2_t *)p = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                }
            }
            if constexpr (!BLOCK_OPS) __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// h + y * g for one staged element, the product and the sum rounded apart
// (no contraction): the result of storing y, then h += y * g in f32.
template <typename TY>
__device__ __forceinline__ TY residual1(TY h, TY y, float g) {
#pragma clang fp contract(off)
    if constexpr (sizeof(TY) == 2) {
        const float r = bf16_bits_to_f32(h) + bf16_bits_to_f32(y) * g;
        return f32_to_bf16_bits(r);
    } else {
        return h + y * g;
    }
}

template <int R, int BN, int NT, typename TY, bool RES = true>
__device__ __forceinline__ void lds_to_global(const uint8_t *stg, int tid, int m0, int n0, int M, int N,
                                              TY *__restrict__ Y, const float *__restrict__ gate_arg = nullptr) {
    const float *gate = RES ? gate_arg : nullptr;
    constexpr int EB = sizeof(TY), RB = BN * EB, CPR = RB / 16, EPC = 16 / EB, SWZ = stage_swz<BN, TY>();
    constexpr int IT = R * CPR / NT;
    static_assert((R * CPR) % NT == 0, "staging tile must split evenly over the block");
    const bool vec = N % EPC == 0;
    // Residual mode (uniform): every read of h and of the gate row for this
    // pass is issued before the first use, so their latencies overlap.
    // A thread's chunk column is the same in every iteration (NT is a
    // multiple of the chunks per row), so its gate values are read once.
    static_assert(NT % CPR == 0, "a thread keeps one chunk column");
    u32x4 hv[RES ? IT : 1];
    float gv[EPC];
    if constexpr (RES) {
        if (gate) {
            const int n = n0 + (tid % CPR) * EPC;
#pragma unroll
            for (int q = 0; q < EPC; q++) gv[q] = 0.0f;
            if (n + EPC <= N && (((uintptr_t)(gate + n)) & 15) == 0) {
#pragma unroll
                for (int q = 0; q < EPC; q += 4) {
                    const f32x4 g4 = *(const f32x4 *)(gate + n + q);
                    gv[q] = g4.x, gv[q + 1] = g4.y, gv[q + 2] = g4.z, gv[q + 3] = g4.w;
                }
            } else {
#pragma unroll
                for (int q = 0; q < EPC; q++)
                    if (n + q < N) gv[q] = gate[n + q];
            }
#pragma unroll
            for (int it = 0; it < IT; it++) {
                const int idx = it * NT + tid, r = idx / CPR, m = m0 + r;
                hv[it] = (u32x4){};
                if (m >= M || n >= N) continue;
                const TY *yp = Y + (size_t)m * N + n;
                if (vec) {
                    hv[it] = *(const u32x4 *)yp;
                } else {
                    TY *he = (TY *)&hv[it];
#pragma unroll
                    for (int q = 0; q < EPC; q++)
                        if (n + q < N) he[q] = yp[q];
                }
            }
        }
    }
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const int idx = it * NT + tid, r = idx / CPR, c = idx % CPR;
        const int m = m0 + r, n = n0 + c * EPC;
        if (m >= M || n >= N) continue;
        u32x4 v = *(const u32x4 *)(stg + r * RB + ((c ^ (r & (SWZ - 1))) << 4));
        TY *yp = Y + (size_t)m * N + n;
        if (RES && gate) {
            TY *e = (TY *)&v;
            const TY *he = (const TY *)&hv[RES ? it : 0];
#pragma unroll
            for (int q = 0; q < EPC; q++) e[q] = residual1<TY>(he[q], e[q], gv[q]);
        }
        if (vec) {
            *(u32x4 *)yp = v;
        } else {
            const TY *e = (const TY *)&v;
#pragma unroll
            for (int q = 0; q < EPC; q++)
                if (n + q < N) yp[q] = e[q];
        }
    }
}

// Whole-tile store of a staged pass (R rows x BN) for tiles whose columns
// all lie inside N, N a multiple of the 16-byte chunk's elements and M * N *
// sizeof(TY) < 2^31: every LDS read is issued first, then every store, through
// a descriptor of Y that drops rows past M -- no branches and no waits between
// the stores.  RES (residual mode): h's chunks and the gate are loaded first
// and h + y * gate stored.  CP: the stores' cache-policy bits (buffer_store_x4).
template <int R, int BN, int NT, typename TY, bool RES, int CP = 0>
__device__ __forceinline__ void lds_to_global_fast(const uint8_t *stg, int tid, int m0, int n0, int M, int N,
                                                   TY *__restrict__ Y, const float *__restrict__ gate) {
    constexpr int EB = sizeof(TY), RB = BN * EB, CPR = RB / 16, EPC = 16 / EB, SWZ = stage_swz<BN, TY>();
    constexpr int IT = R * CPR / NT;
    // chunks read from LDS ahead of their stores, four at a time (the
    // two-workgroup-per-CU tiles have no registers for more)
    constexpr int BATCH = IT < 4 ? IT : 4;
    static_assert((R * CPR) % NT == 0 && NT % CPR == 0 && IT % BATCH == 0, "staging tile must split evenly");
    const auto ry = make_rsrc(Y, (uint32_t)M * (uint32_t)N * EB);
    const int c = tid % CPR, n = n0 + c * EPC;
    auto off = [&](int it) {
        const int m = m0 + (it * NT + tid) / CPR;
        return m < M ? ((uint32_t)m * (uint32_t)N + (uint32_t)n) * EB : kOob;
    };
    u32x4 hv[RES ? IT : 1];
    float gv[RES ? EPC : 1];
    if constexpr (RES) {
#pragma unroll
        for (int it = 0; it < IT; it++) hv[it] = buffer_load_x4(ry, off(it));
#pragma unroll
        for (int q = 0; q < EPC; q += 4) {
            const f32x4 g4 = *(const f32x4 *)(gate + n + q);
            gv[q] = g4.x, gv[q + 1] = g4.y, gv[q + 2] = g4.z, gv[q + 3] = g4.w;
        }
    }
#pragma unroll
    for (int b = 0; b < IT; b += BATCH) {
        u32x4 v[BATCH];
#pragma unroll
        for (int k = 0; k < BATCH; k++) {
            const int r = ((b + k) * NT + tid) / CPR;
            v[k] = *(const u32x4 *)(stg + r * RB + ((c ^ (r & (SWZ - 1))) << 4));
        }
#pragma unroll
        for (int k = 0; k < BATCH; k++) {
            if constexpr (RES) {
                TY *e = (TY *)&v[k];
                const TY *he = (const TY *)&hv[b + k];
#pragma unroll
                for (int q = 0; q < EPC; q++) e[q] = residual1<TY>(he[q], e[q], gv[q]);
            }
            buffer_store_x4<CP>(v[k], ry, off(b + k));
        }
    }
}

constexpr int pow2_floor(int v) { return v < 2 ? 1 : 2 * pow2_floor(v / 2); }

// The staged epilogue of a BM x BN block tile through SMEM bytes of LDS,
// in passes of R rows (whole 32-row blocks) when the whole tile does not fit.  Waits for every
// outstanding DMA of the main loop (stages past K still write zeros) and
// for every wave's last fragment reads before reusing the ring; the
// operands in sc (TileOps) must be parked before the call.  The wave owns
// tile rows [wr, wr + 32 TM) and columns [wc, wc + 32 TN).
//
// ACT: the activation, fixed at compile time (LX2V_ACT_*), or -1 to take
// `act` at run time (two copies of the staging code in the kernel: more
// registers).
//
// WAIT0 = false: the caller's loads into `smem` are known complete (only a
// barrier is taken first), so loads still in flight elsewhere -- the next
// tile's stages of a persistent kernel -- keep flying through the epilogue.
//
// CP: the cache-policy bits of the tile's stores (buffer_store_x4).
//
// TR: the accumulator blocks are transposed (acc_to_lds).
template <int BM, int BN, int NT, int SMEM, int TM, int TN, typename TY, bool RES = true, int ACT = -1,
          bool WAIT0 = true, int CP = 0, bool TR = false>
__device__ __forceinline__ void staged_epilogue(const f32x16 (&acc)[TN][TM], uint8_t *smem, const float *sc, int wr,
                                                int wc, int tid, int lane, int m0, int n0, int M, int N, int act,
                                                TY *__restrict__ Y, MxOut mx = MxOut()) {
    constexpr int RB = BN * (int)sizeof(TY);
    constexpr int R = pow2_floor(SMEM / RB < BM ? SMEM / RB : BM);
    static_assert(BM % R == 0 && R % 32 == 0, "passes of whole 32-row blocks");
    if constexpr (WAIT0) wait_vmcnt<0>();
    __syncthreads();
    constexpr int EPC = 16 / (int)sizeof(TY);
    // Uniform per workgroup: the branch-free store path applies (bf16 and
    // MX output; with f32 output its registers would spill the 128 x 128
    // three-per-CU tile).
    const bool fast = sizeof(TY) != 4 && n0 + BN <= N && N % EPC == 0 && (uint64_t)M * (uint64_t)N * sizeof(TY) < (1ull << 31) &&
                      (((uintptr_t)mx.gate) & 15) == 0;
#pragma unroll
    for (int p = 0; p < BM / R; p++) {
        if (p) __syncthreads();
        if (wr < (p + 1) * R && wr + 32 * TM > p * R) {
            if constexpr (ACT >= 0)
                acc_to_lds<BM, BN, TM, TN, TY, ACT, R == BM, TR>(acc, sc, smem, wr - p * R, R, wr, wc, lane, mx, m0,
                                                                 n0, M, N);
            else if (act == LX2V_ACT_GELU_TANH)
                acc_to_lds<BM, BN, TM, TN, TY, LX2V_ACT_GELU_TANH, R == BM, TR>(acc, sc, smem, wr - p * R, R, wr, wc,
                                                                                lane, mx, m0, n0, M, N);
            else
                acc_to_lds<BM, BN, TM, TN, TY, LX2V_ACT_NONE, R == BM, TR>(acc, sc, smem, wr - p * R, R, wr, wc, lane,
                                                                           mx, m0, n0, M, N);
        }
        __syncthreads();
        if constexpr (sizeof(TY) == 1 || !RES) {
            if (fast)
                lds_to_global_fast<R, BN, NT, TY, false, CP>(smem, tid, m0 + p * R, n0, M, N, Y, nullptr);
            else
                lds_to_global<R, BN, NT, TY, false>(smem, tid, m0 + p * R, n0, M, N, Y);
        } else if (mx.gate) {
            if (fast)
                lds_to_global_fast<R, BN, NT, TY, true, CP>(smem, tid, m0 + p * R, n0, M, N, Y, mx.gate);
            else
                lds_to_global<R, BN, NT, TY, true>(smem, tid, m0 + p * R, n0, M, N, Y, mx.gate);
        } else {
            if (fast)
                lds_to_global_fast<R, BN, NT, TY, false, CP>(smem, tid, m0 + p * R, n0, M, N, Y, nullptr);
            else
                lds_to_global<R, BN, NT, TY, false>(smem, tid, m0 + p * R, n0, M, N, Y);
        }
    }
}

// Chunk slot of 16-byte chunk `c` in row `row` of a BK-byte-row tile:
// consecutive rows of one 256-byte LDS bank window keep their chunks in
// distinct banks, and a 16-lane read of one chunk column is conflict free.
template <int BKB>
__device__ __forceinline__ uint32_t dma_slot(uint32_t row, uint32_t c) {
    constexpr uint32_t CPR = BKB / 16, RW = 256 / BKB;
    return c ^ ((row / RW) % CPR);
}

}  // namespace

}  // namespace lx2v

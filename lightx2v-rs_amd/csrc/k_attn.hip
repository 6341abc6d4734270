// k_attn.hip -- softmax attention (Backend::attention / causal_attention,
// crates/lightx2v-core/src/backend.rs:276-305; CPU reference
// crates/lightx2v-cpu/src/lib.rs:155-203) on the gfx950 bf16 MFMA.
//
//   out[q, h*d + j] = sum_k softmax_k(q.k / sqrt(d), masked) v[k, j]
//   q [heads, sq, d], k / v [heads, sk, d], mask [sq, sk] (1 = allowed)
//
// k_attn_mfma (d = 64 or 128): one workgroup per (head, 128 queries), four
// waves of 32 queries, keys in tiles of 64 through LDS, online softmax
// (running max and sum per query, exp2 with log2(e)/sqrt(d) folded in).
// Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (K is the A
// operand, Q the B operand held in registers), so a lane owns one query and
// 32 of its keys: the row max and sum take one cross-lane step.  P^T stays
// in the registers it was computed in and is the B operand of O^T = V^T P^T;
// the keys of each 16-key MFMA step are taken in the order the S^T layout
// left them in the lane (4 keys of group g, then 4 of group g + 1), and V^T
// is read from LDS in that same order, so no transpose of P is needed.
// A per-(query tile, key tile) mask summary skips fully masked tiles and
// reads mask bytes only in mixed ones.
//
// k_attn_rows: any d <= 256, one wave per (head, query), keys one at a
// time -- the correctness path for other head sizes.
#include "device_common.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

constexpr int AQ = 256;  // queries per workgroup (eight waves of 32: K / V tiles shared by 256 queries)
constexpr int AK = 64;   // keys per tile
constexpr int AT = 512;  // threads per workgroup
constexpr int TROW = 2048;  // key tiles whose mask summary is staged in LDS (sk <= 131072)

__device__ __forceinline__ float ld_f(const void *p, size_t i, int dt) {
    return dt == LX2V_DTYPE_BF16 ? bf16_bits_to_f32(((const uint16_t *)p)[i]) : ((const float *)p)[i];
}

// Eight elements i .. i + 7 of an F32 or BF16 array as packed bf16 (RNE).
template <int DT>
__device__ __forceinline__ u32x4 ld8_bf16(const void *p, size_t i) {
    if constexpr (DT == LX2V_DTYPE_BF16) {
        return *(const u32x4 *)((const uint16_t *)p + i);
    } else {
        const f32x4 a = *(const f32x4 *)((const float *)p + i), b = *(const f32x4 *)((const float *)p + i + 4);
        return (u32x4){pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w), pack_bf16x2(b.x, b.y), pack_bf16x2(b.z, b.w)};
    }
}

template <int D, int DT, int ODT>
__global__ __launch_bounds__(AT) void k_attn_mfma(const void *__restrict__ Q, const void *__restrict__ K,
                                                  const void *__restrict__ V, int heads, int sq, int sk, int kvs,
                                                  const uint8_t *__restrict__ tiles, const uint32_t *__restrict__ mbits,
                                                  float c, void *__restrict__ out, uint8_t *__restrict__ omx,
                                                  int omx_rows, float *__restrict__ part, int nsplit) {
    constexpr int KSTR = D * 2 + 16;   // bytes per K row in LDS (padded: conflict-free fragment reads)
    // bytes per V^T row (one d, 64 keys): 9 16-byte chunks, so the 16-byte
    // fragment reads of 16 consecutive rows fall in distinct bank groups
    constexpr int VSTR = AK * 2 + 16;
    constexpr int QS = D / 16;         // 16-wide d steps of S^T
    constexpr int DB = D / 32;         // 32-row d blocks of O^T
    constexpr int KN = AK * D / 8, VN = AK * D / 16, KI = (KN + AT - 1) / AT, VI = (VN + AT - 1) / AT;
    constexpr int KSZ = AK * KSTR, VSZ = D * VSTR;
    // K of tiles t + 1 and t + 2, V of tiles t and t + 1: [K0 K1 V0 V1].
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * (KSZ + VSZ)];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, l32 = lane & 31, hf = lane >> 5;
    // XCD-aware order: workgroups b, b + 8, ... run on one XCD, so give each
    // XCD a contiguous range of (head, query tile) items -- the workgroups of
    // a head then share its K / V in one L2.
    //
    // Split mode (nsplit = S > 1, part != null): every item is S pieces, each
    // over about 1/S of its allowed key tiles, writing its unnormalized O^T,
    // running max and sum to `part` for k_attn_merge -- S times the
    // workgroups where the items alone would leave CUs idle.  An XCD's pieces
    // are dispatched from the last query tile down (under a causal mask the
    // tiles that see the most keys start first), an item's S pieces side by
    // side.
    const int nqt = (sq + AQ - 1) / AQ, items = nqt * heads, per_xcd = (items + 7) / 8;
    const bool split = nsplit > 1;
    const int b = blockIdx.x;
    int item = -1, piece = 0;
    if (!split) {
        item = (b % 8) * per_xcd + b / 8;
    } else {
        // XCD x owns positions [lo, hi) of the heads' query tiles, position
        // h nqt + i holding query tile (i st) mod nqt of head h: a stride
        // near nqt / golden ratio, so that the part of a head one XCD gets
        // mixes early and late query tiles (light and heavy under a causal
        // mask) rather than taking a run of them.
        const int lo = (b % 8) * per_xcd, hi = min(items, lo + per_xcd);
        int st = (int)(0.618034f * (float)nqt + 0.5f);
        st = st < 1 ? 1 : st;
        auto gcd = [](int a, int c) {
            while (c) {
                const int t = a % c;
                a = c;
                c = t;
            }
            return a;
        };
        while (gcd(st, nqt) != 1) st++;
        int r0 = nqt, r1 = st % nqt, t0 = 0, t1 = 1;  // extended Euclid: st * sinv = 1 mod nqt
        while (r1) {
            const int qq = r0 / r1, r2 = r0 - qq * r1, t2 = t0 - qq * t1;
            r0 = r1;
            r1 = r2;
            t0 = t1;
            t1 = t2;
        }
        const int sinv = ((t0 % nqt) + nqt) % nqt;
        int r = (b / 8) / nsplit;
        piece = (b / 8) % nsplit;
        for (int t = nqt - 1; t >= 0 && item < 0; t--) {
            // the heads h whose query tile t sits at a position in [lo, hi)
            const int i = (int)(((long long)t * sinv) % nqt);
            const int h0 = lo <= i ? 0 : (lo - i + nqt - 1) / nqt;
            const int h1 = hi - 1 < i ? -1 : (hi - 1 - i) / nqt;
            const int cnt = h1 >= h0 ? h1 - h0 + 1 : 0;
            if (r < cnt)
                item = (h0 + r) * nqt + t;
            else
                r -= cnt;
        }
    }
    if (item < 0 || item >= items) return;
    const int head = item / nqt, qt = item % nqt, nkt = (sk + AK - 1) / AK;
    const int q = qt * AQ + wv * 32 + l32;  // this lane's query
    const bool qin = q < sq;
    const size_t qbase = ((size_t)head * sq + (qin ? q : 0)) * D;
    const size_t kvbase = (size_t)head * kvs * D;  // kvs: rows between heads of K / V (>= sk)

    // Q^T fragments (B operand): d 16 s + 8 hf .. + 8 of this lane's query.
    bf16x8 qf[QS];
#pragma unroll
    for (int s = 0; s < QS; s++)
        qf[s] = __builtin_bit_cast(bf16x8, qin ? ld8_bf16<DT>(Q, qbase + 16 * s + 8 * hf) : (u32x4){});

    // Q in registers before the loop: otherwise the first use of qf in every
    // iteration waits for all loads in flight, the next tile's included.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

    f32x16 o[DB];
#pragma unroll
    for (int b = 0; b < DB; b++) o[b] = (f32x16){};
    float m = -INFINITY, lsum = 0.0f;  // running max (log2 domain, scaled) and sum

    // This query tile's row of the mask summary, staged in LDS (a global
    // load per tile would cost a memory latency per tile); rows longer than
    // the stage skip the summary: every tile is then read as mixed.
    __shared__ uint8_t trow[TROW];
    const bool tlds = tiles && nkt <= TROW;
    if (tlds)
        for (int i = tid; i < nkt; i += AT) trow[i] = tiles[(size_t)qt * nkt + i];
    __syncthreads();
    auto tstate = [&](int kt) -> int { return !tiles ? 1 : (tlds ? (int)trow[kt] : 2); };
    // This workgroup's key tiles [klo, khi): all of them, or in split mode,
    // of the n tiles with an allowed pair, those after the floor(p n / S)-th
    // up to and including the floor((p + 1) n / S)-th (piece p; the last
    // piece runs to the end).  Wave 0 counts with ballots.
    int klo = 0, khi = nkt;
    if (split) {
        __shared__ int scut[2];
        if (wv == 0) {
            int total = 0;
            for (int base = 0; base < nkt; base += 64) {
                const int t = base + lane;
                total += __popcll(__ballot(t < nkt && tstate(t) != 0));
            }
            // cut(c): the tile after the c-th allowed one (cut(0) = 0)
            const int c0 = (int)((long long)piece * total / nsplit), c1 = (int)((long long)(piece + 1) * total / nsplit);
            int cut0 = 0, cut1 = 0, acc = 0;
            for (int base = 0; base < nkt; base += 64) {
                const int t = base + lane;
                const bool al = t < nkt && tstate(t) != 0;
                const uint64_t bal = __ballot(al);
                const int cnt = __popcll(bal);
                const uint64_t upto = lane == 63 ? ~0ull : ((2ull << lane) - 1ull);
                const int upto_cnt = acc + __popcll(bal & upto);
                if (c0 > acc && c0 <= acc + cnt)
                    cut0 = base + __ffsll((long long)__ballot(al && upto_cnt == c0));
                if (c1 > acc && c1 <= acc + cnt)
                    cut1 = base + __ffsll((long long)__ballot(al && upto_cnt == c1));
                acc += cnt;
            }
            if (lane == 0) {
                scut[0] = cut0;
                scut[1] = piece == nsplit - 1 ? nkt : cut1;
            }
        }
        __syncthreads();
        klo = scut[0];
        khi = scut[1];
    }
    // The next key tile at or after kt with an allowed pair (uniform).
    auto next_tile = [&](int kt) {
        while (kt < khi && tstate(kt) == 0) kt++;
        return kt;
    };

    // Tiles from global memory into registers: K as 16-byte chunks (key,
    // chunk), V as chunk pairs of two consecutive keys (for V^T).  Buffer
    // loads: keys past sk (and unused lanes, offset kOob) read zero, and
    // every load is issued, so waits can count the loads in flight.
    constexpr uint32_t ES = DT == LX2V_DTYPE_BF16 ? 2 : 4;
    const auto ksrc = make_rsrc((const uint8_t *)K + kvbase * ES, (uint32_t)sk * D * ES);
    const auto vsrc = make_rsrc((const uint8_t *)V + kvbase * ES, (uint32_t)sk * D * ES);
    auto ld8 = [&](__amdgpu_buffer_rsrc_t r, uint32_t off, bool in) -> u32x4 {
        if constexpr (DT == LX2V_DTYPE_BF16) {
            return buffer_load_x4(r, in ? off * 2 : kOob);
        } else {
            const f32x4 a = __builtin_bit_cast(f32x4, buffer_load_x4(r, in ? off * 4 : kOob));
            const f32x4 b = __builtin_bit_cast(f32x4, buffer_load_x4(r, in ? off * 4 + 16 : kOob));
            return (u32x4){pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w), pack_bf16x2(b.x, b.y), pack_bf16x2(b.z, b.w)};
        }
    };
    u32x4 kr[KI], va[VI], vb[VI];
    uint32_t mwn[2];  // mask bits of the V tile loaded last (mixed tiles; kOob reads 0 otherwise)
    const uint32_t nw = ((uint32_t)sk + 31) / 32;
    const auto msrc = make_rsrc(mbits, mbits ? (uint32_t)sq * nw * 4 : 0u);
    auto gload_k = [&](int kt) {
        const uint32_t k0 = (uint32_t)kt * AK;
#pragma unroll
        for (int it = 0; it < KI; it++) {
            const int idx = it * AT + tid, key = idx / (D / 8), ch = idx % (D / 8);
            kr[it] = ld8(ksrc, (k0 + key) * D + 8 * ch, idx < KN && kt < khi);
        }
    };
    auto gload_v = [&](int kt) {
        const uint32_t k0 = (uint32_t)kt * AK;
        const bool mixed = kt < khi && tstate(kt) == 2 && qin;
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
            mwn[kb] = buffer_load_x1(msrc, mixed ? ((uint32_t)q * nw + k0 / 32 + (uint32_t)kb) * 4 : kOob);
        // V item idx: key pair idx % 32 (keys 2 p, 2 p + 1), chunk idx / 32 --
        // consecutive lanes take consecutive key pairs, so the transposed
        // stores below hit consecutive LDS words
#pragma unroll
        for (int it = 0; it < VI; it++) {
            const int idx = it * AT + tid, key = 2 * (idx % (AK / 2)), ch = idx / (AK / 2);
            va[it] = ld8(vsrc, (k0 + key) * D + 8 * ch, idx < VN && kt < khi);
            vb[it] = ld8(vsrc, (k0 + key + 1) * D + 8 * ch, idx < VN && kt < khi);
        }
    };
    // Registers into LDS: K rows; V transposed (one d per row).
    auto lstore_k = [&](int buf) {
        uint8_t *ks = lds + buf * KSZ;
#pragma unroll
        for (int it = 0; it < KI; it++) {
            const int idx = it * AT + tid, key = idx / (D / 8), ch = idx % (D / 8);
            if (idx < KN) *(u32x4 *)(ks + key * KSTR + ch * 16) = kr[it];
        }
    };
    // V^T key order: bits 2 and 3 of the key swapped, so that the 8 keys a
    // lane feeds one 16-key MFMA step (4 of group g and 4 of group g + 2,
    // the order the S^T layout leaves them in) are 16 consecutive bytes.
    auto vpos = [](int key) { return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1); };
    auto lstore_v = [&](int buf) {
        uint8_t *vt = lds + 2 * KSZ + buf * VSZ;
#pragma unroll
        for (int it = 0; it < VI; it++) {
            const int idx = it * AT + tid, key = 2 * (idx % (AK / 2)), ch = idx / (AK / 2);
            if (idx >= VN) continue;
            const uint32_t av[4] = {va[it].x, va[it].y, va[it].z, va[it].w};
            const uint32_t bv[4] = {vb[it].x, vb[it].y, vb[it].z, vb[it].w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t lo = (e & 1) ? av[e / 2] >> 16 : av[e / 2] & 0xFFFFu;
                const uint32_t hi = (e & 1) ? bv[e / 2] >> 16 : bv[e / 2] & 0xFFFFu;
                *(uint32_t *)(vt + (8 * ch + e) * VSTR + vpos(key) * 2) = lo | (hi << 16);
            }
        }
    };
    // S^T = K Q^T for the 64 keys in K buffer kb: keys 32 j + (8 g + 4 hf + r),
    // r = 0..3, in registers 4 g + r of st[j].
    // (the two 32-key blocks' MFMA chains alternate, so that no MFMA waits
    // for the one just before it)
    auto scores = [&](int kbuf, f32x16 *st) {
        const uint8_t *ks = lds + kbuf * KSZ;
        st[0] = (f32x16){};
        st[1] = (f32x16){};
#pragma unroll
        for (int s = 0; s < QS; s++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const bf16x8 kf = __builtin_bit_cast(bf16x8, *(const u32x4 *)(ks + (32 * j + l32) * KSTR + (2 * s + hf) * 16));
                st[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], st[j], 0, 0, 0);
            }
    };

    // Mask tile kt's scores in place: a full tile with every pair allowed is
    // left alone; otherwise keys past sk and, in mixed tiles, pairs whose
    // mask bit is clear become -inf.  mwk: the tile's two mask words.
    auto apply_mask = [&](f32x16 *st, int kt, const uint32_t *mwk) {
        const int state = tstate(kt), k0 = kt * AK;
        if (state == 1 && k0 + AK <= sk) return;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            // allowed keys of this 32-key block as bits (mask word, keys
            // before sk), shifted so that register i tests a constant bit
            const int left = sk - (k0 + 32 * j);
            uint32_t allow = state == 2 ? mwk[j] : ~0u;
            allow &= left >= 32 ? ~0u : (left <= 0 ? 0u : (1u << left) - 1u);
            allow >>= 4 * hf;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const bool ok = (allow >> (8 * (i / 4) + (i % 4))) & 1u;
                st[j][i] = ok ? st[j][i] : -INFINITY;
            }
        }
    };

    // Software pipeline: while tile t's softmax and O^T += V^T P^T run, the
    // scores of tile t + 1 are computed (its K is already in LDS) and the K of
    // tile t + 2 and V of t + 1 are loaded.  The MFMAs of S(t + 1) and the
    // softmax of t are independent, so the matrix cores and the vector ALUs
    // of a SIMD work at once.  Explicit vmcnt(0) after each store: the mask
    // words were loaded before V and are complete once V is, but the
    // compiler cannot see that across the loop's back edge.
    int kt = next_tile(klo);
    int kn = kt < khi ? next_tile(kt + 1) : khi;
    f32x16 sc[2];  // scores of tile kt (raw q.k)
    uint32_t mw[2] = {0u, 0u};
    if (kt < khi) {
        gload_k(kt);
        gload_v(kt);
        lstore_k(0);
        lstore_v(0);
        mw[0] = mwn[0];
        mw[1] = mwn[1];
        gload_k(kn);
        lstore_k(1);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (kt < khi) {
        scores(0, sc);
        apply_mask(sc, kt, mw);
    }
    __syncthreads();  // K buffer 0 is rewritten at the end of the first iteration
    int kbi = 1, vbi = 0;  // K buffer holding K(kn); V buffer holding V(kt)
    const float tau = 8.0f;  // rescale O only when a query's max grows by more than 2^8
    while (kt < khi) {
        const int knn = kn < khi ? next_tile(kn + 1) : khi;
        // loads for the stores at the end of this iteration (kOob when past the last tile)
        __builtin_amdgcn_sched_barrier(0);
        gload_k(knn);
        gload_v(kn);

        // S(kn), unconditionally (past the last tile it reads a stale buffer
        // and is not used): a branch here would keep these MFMAs from being
        // interleaved with the softmax below.
        f32x16 sn[2];
        scores(kbi, sn);
        // The loads go between the first MFMAs of S(kn): issued back to back
        // by all eight waves they held each wave's issue for hundreds of
        // cycles at the top of every tile.
        constexpr int NVM = (KI + 2 * VI) * (DT == LX2V_DTYPE_BF16 ? 1 : 2) + 2;
#pragma unroll
        for (int i = 0; i < NVM; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // an MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // a global load
        }

        // tile kt's scores were masked when they were computed
        float tmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 16; i++) tmax = fmaxf(tmax, sc[j][i]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64)) * c;
        // The reference point moves only when the tile's max passes it by more
        // than tau: p = 2^(s c - m) <= 2^tau in between, exact in f32, and O
        // is rescaled far less often.  With no key allowed yet (m = -inf) any
        // finite reference works: use 0.  The raw v_exp_f32 flushes results
        // below 2^-126 to 0 (no contribution a softmax sum in f32 could
        // register).
        const float mn = tmax > m + tau ? tmax : m;
        const float mref = mn == -INFINITY ? 0.0f : mn;
        const float alpha = __builtin_amdgcn_exp2f(m - mref);
        float psum = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j][i], c, -mref));
                sc[j][i] = p;
                psum += p;
            }
        psum += __shfl_xor(psum, 32, 64);
        lsum = lsum * alpha + psum;
        m = mn;
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int b = 0; b < DB; b++)
#pragma unroll
                for (int i = 0; i < 16; i++) o[b][i] *= alpha;
        }

        // O^T += V^T P^T, four 16-key steps: step u = 2 j + t takes registers
        // 8 t .. 8 t + 7 of sc[j], i.e. keys 32 j + 16 t + 4 hf + 0..3 and
        // 32 j + 16 t + 8 + 4 hf + 0..3, which V^T holds as the 16 bytes at
        // key position 16 u + 8 hf (vpos).  Step u + 1's V fragments are read
        // while step u's MFMAs run.
        const uint8_t *vt = lds + 2 * KSZ + vbi * VSZ;
        auto vread = [&](int u, bf16x8 *vf) {
#pragma unroll
            for (int b = 0; b < DB; b++)
                vf[b] = __builtin_bit_cast(bf16x8, *(const u32x4 *)(vt + (32 * b + l32) * VSTR + (16 * u + 8 * hf) * 2));
        };
        bf16x8 vcur[DB], vnxt[DB];
        vread(0, vcur);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (u < 3) vread(u + 1, vnxt);
            __builtin_amdgcn_sched_barrier(0);
            const f32x16 &sp = sc[u >> 1];
            const int t = u & 1;
            const u32x4 pw = (u32x4){pack_bf16x2(sp[8 * t + 0], sp[8 * t + 1]), pack_bf16x2(sp[8 * t + 2], sp[8 * t + 3]),
                                     pack_bf16x2(sp[8 * t + 4], sp[8 * t + 5]), pack_bf16x2(sp[8 * t + 6], sp[8 * t + 7])};
            const bf16x8 pf = __builtin_bit_cast(bf16x8, pw);
#pragma unroll
            for (int b = 0; b < DB; b++) o[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vcur[b], pf, o[b], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (u < 3)
#pragma unroll
                for (int b = 0; b < DB; b++) vcur[b] = vnxt[b];
        }
        // K(kt) and V of the previous tile were last read before the previous
        // barrier (stores past the last tile write zeros, unused)
        lstore_k(kbi ^ 1);
        lstore_v(vbi ^ 1);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        mw[0] = mwn[0];
        mw[1] = mwn[1];
        if (kn < khi) apply_mask(sn, kn, mw);
        __syncthreads();
        sc[0] = sn[0];
        sc[1] = sn[1];
        kbi ^= 1;
        vbi ^= 1;
        kt = kn;
        kn = knn;
    }

    if (!qin) return;
    if (split) {
        // this piece's O^T (unnormalized), running max (log2 domain) and sum
        const size_t slot = (size_t)item * nsplit + piece, row = slot * AQ + (size_t)(q - qt * AQ);
        float *po = part + row * D;
#pragma unroll
        for (int b = 0; b < DB; b++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *(f32x4 *)(po + 32 * b + 8 * g + 4 * hf) =
                    (f32x4){o[b][4 * g], o[b][4 * g + 1], o[b][4 * g + 2], o[b][4 * g + 3]};
        typedef float f32x2_t __attribute__((ext_vector_type(2)));
        if (hf == 0) *(f32x2_t *)(part + (size_t)items * nsplit * AQ * D + row * 2) = (f32x2_t){m, lsum};
        return;
    }
    // No allowed key: 0 / 0 = NaN, as the reference's softmax of all -inf;
    // no key at all (sk = 0): 0, the reference's empty sum.
    const float inv = sk == 0 ? 0.0f : 1.0f / lsum;
    if constexpr (ODT == LX2V_DTYPE_MXE4M3) {
        // MX e4m3 rows of heads * D columns (the input of the O linear): block
        // b of this head is d 32 b .. 32 b + 31, split between lanes l and l
        // + 32 (d 32 b + 8 g + 4 hf + 0..3); the pair's amax gives the block's
        // scale 2^k, codes = RNE e4m3 of v 2^-k (NaN stays NaN: no clamp is
        // needed once |v| 2^-k <= 448), the scale byte goes to the scale
        // array (mx_sidx, omx_rows rows per 128-column group).
        const size_t row0 = (size_t)q * heads * D + (size_t)head * D;
#pragma unroll
        for (int b = 0; b < DB; b++) {
            float v[16];
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                v[i] = o[b][i] * inv;
                amax = fmaxf(amax, fabsf(v[i]));
            }
            amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
            const int k = mx_exponent(amax);
            const float msc = mx_scale(k);
#pragma unroll
            for (int g = 0; g < 4; g++)
                *(uint32_t *)((uint8_t *)out + row0 + 32 * b + 8 * g + 4 * hf) = quant4_sc(v + 4 * g, msc);
            if (hf == 0) omx[mx_sidx(q, (head * D + 32 * b) / 32, omx_rows)] = (uint8_t)(k + 127);
        }
        return;
    }
#pragma unroll
    for (int b = 0; b < DB; b++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = 32 * b + 8 * g + 4 * hf;
            const size_t oi = ((size_t)q * heads + head) * D + d0;
            const float v0 = o[b][4 * g] * inv, v1 = o[b][4 * g + 1] * inv, v2 = o[b][4 * g + 2] * inv,
                        v3 = o[b][4 * g + 3] * inv;
            if constexpr (ODT == LX2V_DTYPE_BF16) {
                typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
                *(u32x2_t *)((uint16_t *)out + oi) = (u32x2_t){pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
            } else {
                *(f32x4 *)((float *)out + oi) = (f32x4){v0, v1, v2, v3};
            }
        }
}

// Split mode's second pass: the S pieces of each (query, head) row
// combined, O = sum_p O_p 2^(m_p - m) / sum_p l_p 2^(m_p - m) with m = max_p
// m_p, stored as the one-pass kernel stores (F32 / BF16 rows, or MX e4m3 and
// its scale bytes).  A thread per 4 consecutive d of a row, so a 32-d MX
// block is 8 consecutive lanes.
template <int D, int ODT>
__global__ __launch_bounds__(256) void k_attn_merge(const float *__restrict__ part, int nsplit, int heads, int sq,
                                                   int sk, void *__restrict__ out, uint8_t *__restrict__ omx,
                                                   int omx_rows) {
    constexpr int CH = D / 4;
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x, rows = (size_t)sq * heads;
    const bool live = t < rows * CH;
    const size_t r = live ? t / CH : 0;  // q * heads + head, the output row
    const int ch = (int)(t % CH), q = (int)(r / heads), head = (int)(r % heads);
    const int nqt = (sq + AQ - 1) / AQ, qt = q / AQ, items = nqt * heads;
    const size_t row0 = (size_t)(head * nqt + qt) * nsplit * AQ + (size_t)(q - qt * AQ);
    const float *ml = part + (size_t)items * nsplit * AQ * D;
    float mm = -INFINITY;
    for (int p = 0; p < nsplit; p++) mm = fmaxf(mm, ml[2 * (row0 + (size_t)p * AQ)]);
    // an empty piece (m = -inf) weighs 0; no allowed key in any: 0 / 0 = NaN
    float l = 0.0f, v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int p = 0; p < nsplit; p++) {
        const size_t rp = row0 + (size_t)p * AQ;
        const float mp = ml[2 * rp];
        const float w = mp == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mp - mm);
        l = __builtin_fmaf(ml[2 * rp + 1], w, l);
        const f32x4 a = *(const f32x4 *)(part + rp * D + 4 * ch);
        v[0] = __builtin_fmaf(a.x, w, v[0]);
        v[1] = __builtin_fmaf(a.y, w, v[1]);
        v[2] = __builtin_fmaf(a.z, w, v[2]);
        v[3] = __builtin_fmaf(a.w, w, v[3]);
    }
    const float inv = sk == 0 ? 0.0f : 1.0f / l;
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] *= inv;
    const size_t oi = r * D + 4 * ch;
    if constexpr (ODT == LX2V_DTYPE_MXE4M3) {
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
        const int k = mx_exponent(amax);
        const float msc = mx_scale(k);
        if (!live) return;
        *(uint32_t *)((uint8_t *)out + oi) = quant4_sc(v, msc);
        if (ch % 8 == 0) omx[mx_sidx(q, (head * D + 4 * ch) / 32, omx_rows)] = (uint8_t)(k + 127);
    } else if constexpr (ODT == LX2V_DTYPE_BF16) {
        if (!live) return;
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        *(u32x2_t *)((uint16_t *)out + oi) = (u32x2_t){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    } else {
        if (!live) return;
        *(f32x4 *)((float *)out + oi) = (f32x4){v[0], v[1], v[2], v[3]};
    }
}

// Any head size d <= 256: one wave per (head, query), lane j owning
// elements j, j + 64, ...; keys one at a time with an online softmax in f32.
__global__ __launch_bounds__(AT) void k_attn_rows(const void *__restrict__ Q, const void *__restrict__ K,
                                                  const void *__restrict__ V, int dt, int heads, int sq, int sk,
                                                  int kvs, int d, const uint8_t *__restrict__ mask, float c,
                                                  void *__restrict__ out, int odt) {
    const int lane = threadIdx.x & 63;
    const size_t row = blockIdx.x * (size_t)(AT / 64) + (threadIdx.x >> 6);  // head * sq + query
    if (row >= (size_t)heads * sq) return;
    const int head = (int)(row / sq), q = (int)(row % sq);
    float qv[4], acc[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int j = lane + 64 * e;
        qv[e] = j < d ? ld_f(Q, row * d + j, dt) : 0.0f;
        acc[e] = 0.0f;
    }
    float m = -INFINITY, lsum = 0.0f;
    for (int key = 0; key < sk; key++) {
        if (mask && !mask[(size_t)q * sk + key]) continue;
        const size_t kb = ((size_t)head * kvs + key) * d;
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int j = lane + 64 * e;
            if (j < d) s += qv[e] * ld_f(K, kb + j, dt);
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
        const float x = s * c, mn = fmaxf(m, x), alpha = exp2f(m - mn), p = exp2f(x - mn);
        lsum = lsum * alpha + p;
        m = mn;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int j = lane + 64 * e;
            acc[e] = acc[e] * alpha + (j < d ? p * ld_f(V, kb + j, dt) : 0.0f);
        }
    }
    const float inv = sk == 0 ? 0.0f : 1.0f / lsum;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int j = lane + 64 * e;
        if (j >= d) continue;
        const size_t oi = ((size_t)q * heads + head) * d + j;
        if (odt == LX2V_DTYPE_BF16)
            ((uint16_t *)out)[oi] = f32_to_bf16_bits(acc[e] * inv);
        else
            ((float *)out)[oi] = acc[e] * inv;
    }
}

// Mask summary per (256-query, 64-key) tile: 0 no pair allowed, 1 every
// pair allowed, 2 mixed; pairs past sq / sk ignored.  From the packed bits
// (launch_mask_pack's words): a wave per tile reads its 256 queries' two
// words (2 KB, where the bytes would be 16 KB).
__global__ __launch_bounds__(AT) void k_mask_tiles_bits(const uint32_t *__restrict__ bits, int sq, int sk, int nqt,
                                                        int nkt, uint8_t *__restrict__ tiles) {
    const int lane = threadIdx.x & 63, nw = (sk + 31) / 32;
    const size_t t = blockIdx.x * (size_t)(AT / 64) + (threadIdx.x >> 6);
    if (t >= (size_t)nqt * nkt) return;
    const int qt = (int)(t / nkt), kt = (int)(t % nkt);
    bool any = false, all = true;
    for (int i = lane; i < 2 * AQ; i += 64) {
        const int q = qt * AQ + i / 2, j = i % 2, left = sk - (kt * AK + 32 * j);
        if (q >= sq || left <= 0) continue;
        const uint32_t vm = left >= 32 ? ~0u : (1u << left) - 1u;
        const uint32_t w = bits[(size_t)q * nw + 2 * kt + j] & vm;
        any |= w != 0;
        all &= w == vm;
    }
    const bool wany = __ballot(any) != 0, wall = __ballot(!all) == 0;
    if (lane == 0) tiles[t] = !wany ? 0 : (wall ? 1 : 2);
}

// Mask bits: word w of query q holds keys 32 w .. 32 w + 31 (bit = key % 32),
// keys past sk clear.  One wave per (query, 64 keys).
__global__ __launch_bounds__(AT) void k_mask_pack(const uint8_t *__restrict__ mask, int sq, int sk,
                                                  uint32_t *__restrict__ bits) {
    const int lane = threadIdx.x & 63;
    const int nw = (sk + 31) / 32, nw2 = (nw + 1) / 2;
    const size_t t = blockIdx.x * (size_t)(AT / 64) + (threadIdx.x >> 6);
    if (t >= (size_t)sq * nw2) return;
    const int q = (int)(t / nw2), key = (int)(t % nw2) * 64 + lane;
    const bool a = key < sk && mask[(size_t)q * sk + key] != 0;
    const uint64_t b = __ballot(a);
    const int w = key / 32;
    if ((lane & 31) == 0 && w < nw) bits[(size_t)q * nw + w] = (uint32_t)(lane ? b >> 32 : b);
}

// The MemRoPE block mask from temporal indices (dit.rs:643-653): pair
// (q, k) is allowed iff tk[k] <= tq[q].  Bytes: a thread per 4 keys of a
// query row (rows from blockIdx.y); bits: a wave per 64-key block and 64
// queries, one ballot per query; tile summary: a wave per tile from the
// min / max of the tile's query and key indices (all allowed iff
// max tk <= min tq, none iff min tk > max tq).
__global__ __launch_bounds__(AT) void k_mask_temporal_bytes(const uint64_t *__restrict__ tq, const uint64_t *__restrict__ tk,
                                                            int sq, int sk, uint8_t *__restrict__ mask) {
    const int chunks = (sk + 3) / 4;
    for (int q = blockIdx.y; q < sq; q += gridDim.y) {
        const uint64_t tqv = tq[q];
        uint8_t *row = mask + (size_t)q * sk;
        for (int c = blockIdx.x * AT + threadIdx.x; c < chunks; c += gridDim.x * AT) {
            const int k0 = 4 * c;
            uint32_t v = 0;
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (k0 + e < sk && tk[k0 + e] <= tqv) v |= 1u << (8 * e);
            if (k0 + 4 <= sk && (((uintptr_t)(row + k0)) & 3) == 0) {
                *(uint32_t *)(row + k0) = v;
            } else {
                for (int e = 0; e < 4 && k0 + e < sk; e++) row[k0 + e] = (uint8_t)(v >> (8 * e));
            }
        }
    }
}

__global__ __launch_bounds__(AT) void k_mask_temporal_bits(const uint64_t *__restrict__ tq, const uint64_t *__restrict__ tk,
                                                           int sq, int sk, uint32_t *__restrict__ bits) {
    const int lane = threadIdx.x & 63, nw = (sk + 31) / 32, nkb = (sk + 63) / 64;
    const size_t wave = blockIdx.x * (size_t)(AT / 64) + (threadIdx.x >> 6);
    const int kb = (int)(wave % nkb), qg = (int)(wave / nkb);
    if (qg * 64 >= sq) return;
    const int k = 64 * kb + lane;
    const uint64_t tkv = k < sk ? tk[k] : ~0ull;  // keys past sk: never allowed
    const int q1 = min(qg * 64 + 64, sq);
    for (int q = qg * 64; q < q1; q++) {
        const uint64_t b = __ballot(k < sk && tkv <= tq[q]);
        const int w = 2 * kb + (lane >> 5);
        if ((lane & 31) == 0 && w < nw) bits[(size_t)q * nw + w] = (uint32_t)(lane ? b >> 32 : b);
    }
}

__global__ __launch_bounds__(AT) void k_mask_temporal_tiles(const uint64_t *__restrict__ tq, const uint64_t *__restrict__ tk,
                                                            int sq, int sk, int nqt, int nkt, uint8_t *__restrict__ tiles) {
    const int lane = threadIdx.x & 63;
    const size_t t = blockIdx.x * (size_t)(AT / 64) + (threadIdx.x >> 6);
    if (t >= (size_t)nqt * nkt) return;
    const int qt = (int)(t / nkt), kt = (int)(t % nkt);
    uint64_t qmin = ~0ull, qmax = 0, kmin = ~0ull, kmax = 0;
    for (int i = lane; i < AQ; i += 64) {
        const int q = qt * AQ + i;
        if (q < sq) qmin = min(qmin, tq[q]), qmax = max(qmax, tq[q]);
    }
    {
        const int k = kt * AK + lane;
        if (k < sk) kmin = tk[k], kmax = tk[k];
    }
    for (int o = 32; o >= 1; o >>= 1) {
        qmin = min(qmin, (uint64_t)__shfl_xor((unsigned long long)qmin, o, 64));
        qmax = max(qmax, (uint64_t)__shfl_xor((unsigned long long)qmax, o, 64));
        kmin = min(kmin, (uint64_t)__shfl_xor((unsigned long long)kmin, o, 64));
        kmax = max(kmax, (uint64_t)__shfl_xor((unsigned long long)kmax, o, 64));
    }
    if (lane == 0) tiles[t] = kmin > qmax ? 0 : (kmax <= qmin ? 1 : 2);
}

template <int D, int DT>
void attn_mfma_od(hipStream_t s, dim3 grid, const void *q, const void *k, const void *v, int heads, int sq, int sk,
                  int kvs, const uint8_t *tiles, const uint32_t *mask, float c, void *out, int odt, uint8_t *omx,
                  int omx_rows, float *part, int nsplit) {
    if (nsplit > 1) {  // pieces into `part` (the output type only matters to the merge)
        hipLaunchKernelGGL((k_attn_mfma<D, DT, LX2V_DTYPE_F32>), grid, dim3(AT), 0, s, q, k, v, heads, sq, sk, kvs,
                           tiles, mask, c, nullptr, nullptr, 0, part, nsplit);
        const size_t n = (size_t)sq * heads * (D / 4);
        const dim3 mg((unsigned)((n + 255) / 256));
        if (odt == LX2V_DTYPE_BF16)
            hipLaunchKernelGGL((k_attn_merge<D, LX2V_DTYPE_BF16>), mg, dim3(256), 0, s, part, nsplit, heads, sq, sk, out,
                               omx, omx_rows);
        else if (odt == LX2V_DTYPE_MXE4M3)
            hipLaunchKernelGGL((k_attn_merge<D, LX2V_DTYPE_MXE4M3>), mg, dim3(256), 0, s, part, nsplit, heads, sq, sk,
                               out, omx, omx_rows);
        else
            hipLaunchKernelGGL((k_attn_merge<D, LX2V_DTYPE_F32>), mg, dim3(256), 0, s, part, nsplit, heads, sq, sk, out,
                               omx, omx_rows);
        return;
    }
    if (odt == LX2V_DTYPE_BF16)
        hipLaunchKernelGGL((k_attn_mfma<D, DT, LX2V_DTYPE_BF16>), grid, dim3(AT), 0, s, q, k, v, heads, sq, sk, kvs,
                           tiles, mask, c, out, omx, omx_rows, nullptr, 0);
    else if (odt == LX2V_DTYPE_MXE4M3)
        hipLaunchKernelGGL((k_attn_mfma<D, DT, LX2V_DTYPE_MXE4M3>), grid, dim3(AT), 0, s, q, k, v, heads, sq, sk, kvs,
                           tiles, mask, c, out, omx, omx_rows, nullptr, 0);
    else
        hipLaunchKernelGGL((k_attn_mfma<D, DT, LX2V_DTYPE_F32>), grid, dim3(AT), 0, s, q, k, v, heads, sq, sk, kvs,
                           tiles, mask, c, out, omx, omx_rows, nullptr, 0);
}

}  // namespace

bool attention_mfma_supported(size_t d) { return d == 64 || d == 128; }

// Split mode: S = 2, 4 or 8 pieces per (head, query tile), merged in a
// second pass, where the items alone would leave at least half the CUs idle
// (the largest S with items * S <= CUs and 8 S key tiles).  At the Wan
// chunk's 228 items a two-way split balances the causal mask's heavy and
// light query tiles but measured no faster: the merge pass and the piece
// boundaries cost what the balance gains.  LIGHTX2V_HIP_ATTN_SPLIT=0 turns
// it off, =S (2..16) forces S pieces on every MFMA call.
int attention_split(size_t heads, size_t sq, size_t sk, size_t d, int num_cu, size_t *bytes) {
    *bytes = 0;
    if (!attention_mfma_supported(d) || heads == 0 || sq == 0) return 1;
    const char *e = getenv("LIGHTX2V_HIP_ATTN_SPLIT");
    const int mode = e ? atoi(e) : -1;
    const size_t items = ((sq + AQ - 1) / AQ) * heads, nkt = (sk + AK - 1) / AK;
    int S = 1;
    if (mode >= 2)
        S = mode > 16 ? 16 : mode;
    else if (mode != 0)
        while (S < 8 && items * (size_t)S * 2 <= (size_t)num_cu && nkt >= (size_t)S * 16) S *= 2;
    if (S > 1) *bytes = items * (size_t)S * AQ * (d + 2) * 4;
    return S;
}

void launch_mask_tiles_bits(hipStream_t s, const uint32_t *bits, size_t sq, size_t sk, uint8_t *tiles) {
    const int nqt = (int)((sq + AQ - 1) / AQ), nkt = (int)((sk + AK - 1) / AK);
    const size_t n = (size_t)nqt * nkt;
    if (n == 0) return;
    hipLaunchKernelGGL(k_mask_tiles_bits, dim3((unsigned)((n + AT / 64 - 1) / (AT / 64))), dim3(AT), 0, s, bits,
                       (int)sq, (int)sk, nqt, nkt, tiles);
}

void launch_mask_temporal(hipStream_t s, const uint64_t *tq, size_t sq, const uint64_t *tk, size_t sk, uint8_t *mask,
                          uint32_t *bits, uint8_t *tiles) {
    if (sq == 0 || sk == 0) return;
    const size_t chunks = (sk + 3) / 4;
    hipLaunchKernelGGL(k_mask_temporal_bytes,
                       dim3((unsigned)((chunks + AT - 1) / AT), (unsigned)std::min<size_t>(sq, 65535)), dim3(AT), 0, s,
                       tq, tk, (int)sq, (int)sk, mask);
    const size_t waves = ((sk + 63) / 64) * ((sq + 63) / 64);
    hipLaunchKernelGGL(k_mask_temporal_bits, dim3((unsigned)((waves + AT / 64 - 1) / (AT / 64))), dim3(AT), 0, s, tq, tk,
                       (int)sq, (int)sk, bits);
    const int nqt = (int)((sq + AQ - 1) / AQ), nkt = (int)((sk + AK - 1) / AK);
    const size_t n = (size_t)nqt * nkt;
    hipLaunchKernelGGL(k_mask_temporal_tiles, dim3((unsigned)((n + AT / 64 - 1) / (AT / 64))), dim3(AT), 0, s, tq, tk,
                       (int)sq, (int)sk, nqt, nkt, tiles);
}

size_t mask_tile_count(size_t sq, size_t sk) { return ((sq + AQ - 1) / AQ) * ((sk + AK - 1) / AK); }

size_t mask_word_count(size_t sq, size_t sk) { return sq * ((sk + 31) / 32); }

void launch_mask_pack(hipStream_t s, const uint8_t *mask, size_t sq, size_t sk, uint32_t *bits) {
    const size_t n = sq * (((sk + 31) / 32 + 1) / 2);
    if (n == 0) return;
    hipLaunchKernelGGL(k_mask_pack, dim3((unsigned)((n + AT / 64 - 1) / (AT / 64))), dim3(AT), 0, s, mask, (int)sq,
                       (int)sk, bits);
}

void launch_attention(hipStream_t s, const void *q, const void *k, const void *v, int dt, size_t heads, size_t sq,
                      size_t sk, size_t kvs, size_t d, const uint8_t *mask, const uint32_t *mbits,
                      const uint8_t *tiles, void *out, int odt, uint8_t *omx, size_t omx_rows, float *part,
                      int nsplit) {
    if (heads == 0 || sq == 0) return;
    const float c = 1.4426950408889634f / sqrtf((float)d);  // log2(e) / sqrt(d): softmax in base 2
    if (attention_mfma_supported(d)) {
        const size_t items = ((sq + AQ - 1) / AQ) * heads;
        nsplit = part && nsplit > 1 ? nsplit : 1;
        const dim3 grid((unsigned)(8 * nsplit * ((items + 7) / 8)));
        const int hq = (int)heads, iq = (int)sq, ik = (int)sk, is = (int)kvs;
        if (d == 128) {
            if (dt == LX2V_DTYPE_BF16)
                attn_mfma_od<128, LX2V_DTYPE_BF16>(s, grid, q, k, v, hq, iq, ik, is, tiles, mbits, c, out, odt, omx,
                                                   (int)omx_rows, part, nsplit);
            else
                attn_mfma_od<128, LX2V_DTYPE_F32>(s, grid, q, k, v, hq, iq, ik, is, tiles, mbits, c, out, odt, omx,
                                                  (int)omx_rows, part, nsplit);
        } else {
            if (dt == LX2V_DTYPE_BF16)
                attn_mfma_od<64, LX2V_DTYPE_BF16>(s, grid, q, k, v, hq, iq, ik, is, tiles, mbits, c, out, odt, omx,
                                                  (int)omx_rows, part, nsplit);
            else
                attn_mfma_od<64, LX2V_DTYPE_F32>(s, grid, q, k, v, hq, iq, ik, is, tiles, mbits, c, out, odt, omx,
                                                 (int)omx_rows, part, nsplit);
        }
        return;
    }
    const size_t rows = heads * sq;
    hipLaunchKernelGGL(k_attn_rows, dim3((unsigned)((rows + AT / 64 - 1) / (AT / 64))), dim3(AT), 0, s, q, k, v, dt,
                       (int)heads, (int)sq, (int)sk, (int)kvs, (int)d, mask, c, out, odt);
}

}  // namespace lx2v

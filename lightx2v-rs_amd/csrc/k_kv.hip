// k_kv.hip -- the per-layer KV cache on the device (Backend::kv_cache_*,
// crates/lightx2v-core/src/backend.rs:333-392).
//
// The cache keeps K and V as [heads, cap, d] (cap rows reserved per head) in
// one allocation, K first, so attention reads it in place with a head
// stride of cap rows.  The reference keeps [rows, heads*d] and transposes to
// [heads, rows, d] on every kv_cache_kv (crates/lightx2v-cpu/src/lib.rs:
// 689-705); here rows of one head are contiguous, so append / put / kv move
// whole per-head row ranges and the MemRoPE update is one gather.
//
// k_kv_copy:  [heads, rows, d] blocks between two such layouts (different
//             head strides and first rows), converting F32 <-> BF16.
// k_kv_remap: the MemRoPE update's new layout, row by row: a copy of an old
//             row, zeros (a freshly seeded EMA frame), or an EMA slot row
//             folded with the evicted frames in order,
//             e = (1 - alpha) * e + alpha * f  (memrope.rs:57-63; built with
//             -ffp-contract=off so the two products and the sum round apart,
//             as in the reference).
#include "device_common.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

constexpr int KT = 256;

template <int DT>
__device__ __forceinline__ float kv_ld(const void *p, size_t i) {
    if constexpr (DT == LX2V_DTYPE_BF16)
        return bf16_bits_to_f32(((const uint16_t *)p)[i]);
    else
        return ((const float *)p)[i];
}

template <int DT>
__device__ __forceinline__ void kv_st(void *p, size_t i, float x) {
    if constexpr (DT == LX2V_DTYPE_BF16)
        ((uint16_t *)p)[i] = f32_to_bf16_bits(x);
    else
        ((float *)p)[i] = x;
}

// One thread per (row, group of V elements) of head blockIdx.y; V = 4 when
// d % 4 == 0.  rows * d < 2^31 (checked by the host).
template <int SDT, int DDT, int V>
__global__ __launch_bounds__(KT) void k_kv_copy(const void *__restrict__ src, size_t sstride, size_t srow0,
                                                void *__restrict__ dst, size_t dstride, size_t drow0, uint32_t rows,
                                                uint32_t d) {
    const uint32_t per_row = d / V, n = rows * per_row;
    const size_t h = blockIdx.y;
    for (uint32_t t = blockIdx.x * KT + threadIdx.x; t < n; t += gridDim.x * KT) {
        const uint32_t c = t % per_row, r = t / per_row;
        const size_t si = ((h * sstride + srow0 + r) * d) + c * V, di = ((h * dstride + drow0 + r) * d) + c * V;
        if constexpr (SDT == DDT && SDT == LX2V_DTYPE_F32 && V == 4) {
            *(f32x4 *)((float *)dst + di) = *(const f32x4 *)((const float *)src + si);
        } else if constexpr (SDT == DDT && SDT == LX2V_DTYPE_BF16 && V == 4) {
            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
            *(u32x2_t *)((uint16_t *)dst + di) = *(const u32x2_t *)((const uint16_t *)src + si);
        } else {
#pragma unroll
            for (int e = 0; e < V; e++) kv_st<DDT>(dst, di + e, kv_ld<SDT>(src, si + e));
        }
    }
}

// plan: map[new_rows], then per EMA slot s (0 long, 1 short): init[ft] and
// n_ev[s] rows of ev[ft] (old row indices, -1 = a zero row).
// map[r] >= 0: old row; -1: zeros; <= -2: slot s = c / ft, offset o = c % ft
// with c = -map[r] - 2.
struct RemapArgs {
    int ft;
    int n_ev[2];
    int init_at[2], ev_at[2];  // plan offsets of each slot's init row list / first evicted row list
    float alpha[2];
};

// V consecutive elements at element index i (16 B for F32, 8 B for BF16
// when V = 4; i is a multiple of V).
template <int DT, int V>
__device__ __forceinline__ void kv_ldv(const void *p, size_t i, float (&x)[V]) {
    if constexpr (V == 4 && DT == LX2V_DTYPE_F32) {
        const f32x4 a = *(const f32x4 *)((const float *)p + i);
        x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w;
    } else if constexpr (V == 4) {
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x2_t a = *(const u32x2_t *)((const uint16_t *)p + i);
        x[0] = __uint_as_float(a.x << 16), x[1] = __uint_as_float(a.x & 0xFFFF0000u);
        x[2] = __uint_as_float(a.y << 16), x[3] = __uint_as_float(a.y & 0xFFFF0000u);
    } else {
#pragma unroll
        for (int e = 0; e < V; e++) x[e] = kv_ld<DT>(p, i + e);
    }
}

template <int DT, int V>
__device__ __forceinline__ void kv_stv(void *p, size_t i, const float (&x)[V]) {
    if constexpr (V == 4 && DT == LX2V_DTYPE_F32) {
        *(f32x4 *)((float *)p + i) = (f32x4){x[0], x[1], x[2], x[3]};
    } else if constexpr (V == 4) {
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        *(u32x2_t *)((uint16_t *)p + i) =
            (u32x2_t){f32_to_bf16_bits(x[0]) | ((uint32_t)f32_to_bf16_bits(x[1]) << 16),
                      f32_to_bf16_bits(x[2]) | ((uint32_t)f32_to_bf16_bits(x[3]) << 16)};
    } else {
#pragma unroll
        for (int e = 0; e < V; e++) kv_st<DT>(p, i + e, x[e]);
    }
}

// One thread per (row, group of V elements) of head blockIdx.y.
template <int DT, int V>
__global__ __launch_bounds__(KT) void k_kv_remap(const void *__restrict__ src, size_t sstride,
                                                 void *__restrict__ dst, size_t dstride, uint32_t rows, uint32_t d,
                                                 const int *__restrict__ plan, RemapArgs a) {
    const uint32_t per_row = d / V, n = rows * per_row;
    const size_t h = blockIdx.y;
    for (uint32_t t = blockIdx.x * KT + threadIdx.x; t < n; t += gridDim.x * KT) {
        const uint32_t j = (t % per_row) * V, r = t / per_row;
        const size_t sh = h * sstride * d + j;  // (head, element) base in the old layout
        const int m = plan[r];
        float x[V];
        if (m >= 0) {
            kv_ldv<DT, V>(src, sh + (size_t)m * d, x);
        } else if (m == -1) {
#pragma unroll
            for (int e = 0; e < V; e++) x[e] = 0.0f;
        } else {
            const int c = -m - 2, s = c / a.ft, o = c % a.ft;
            const int i0 = plan[a.init_at[s] + o];
            if (i0 >= 0) {
                kv_ldv<DT, V>(src, sh + (size_t)i0 * d, x);
            } else {
#pragma unroll
                for (int e = 0; e < V; e++) x[e] = 0.0f;
            }
            const float al = a.alpha[s], keep = 1.0f - al;
            for (int i = 0; i < a.n_ev[s]; i++) {
                const int ri = plan[a.ev_at[s] + i * a.ft + o];
                float f[V];
                if (ri >= 0) {
                    kv_ldv<DT, V>(src, sh + (size_t)ri * d, f);
                } else {
#pragma unroll
                    for (int e = 0; e < V; e++) f[e] = 0.0f;
                }
#pragma unroll
                for (int e = 0; e < V; e++) x[e] = keep * x[e] + al * f[e];
            }
        }
        kv_stv<DT, V>(dst, (h * dstride + r) * d + j, x);
    }
}

// x: enough workgroups for n items of one head, at most 4096 / heads (>= 1)
// so the whole launch stays near 4096 workgroups; y: the heads.
dim3 grid_for(size_t n, size_t heads) {
    const size_t cap = std::max<size_t>(4096 / heads, 1);
    return dim3((unsigned)std::min<size_t>((n + KT - 1) / KT, cap), (unsigned)heads);
}

template <int SDT, int DDT>
void copy_dt(hipStream_t s, const void *src, size_t sstride, size_t srow0, void *dst, size_t dstride, size_t drow0,
             size_t heads, size_t rows, size_t d) {
    if (d % 4 == 0)
        hipLaunchKernelGGL((k_kv_copy<SDT, DDT, 4>), grid_for(rows * d / 4, heads), dim3(KT), 0, s, src, sstride, srow0,
                           dst, dstride, drow0, (uint32_t)rows, (uint32_t)d);
    else
        hipLaunchKernelGGL((k_kv_copy<SDT, DDT, 1>), grid_for(rows * d, heads), dim3(KT), 0, s, src, sstride, srow0, dst,
                           dstride, drow0, (uint32_t)rows, (uint32_t)d);
}

}  // namespace

void launch_kv_copy(hipStream_t s, const void *src, int sdt, size_t sstride, size_t srow0, void *dst, int ddt,
                    size_t dstride, size_t drow0, size_t heads, size_t rows, size_t d) {
    if (heads * rows * d == 0) return;
    const bool sb = sdt == LX2V_DTYPE_BF16, db = ddt == LX2V_DTYPE_BF16;
    if (sb && db)
        copy_dt<LX2V_DTYPE_BF16, LX2V_DTYPE_BF16>(s, src, sstride, srow0, dst, dstride, drow0, heads, rows, d);
    else if (sb)
        copy_dt<LX2V_DTYPE_BF16, LX2V_DTYPE_F32>(s, src, sstride, srow0, dst, dstride, drow0, heads, rows, d);
    else if (db)
        copy_dt<LX2V_DTYPE_F32, LX2V_DTYPE_BF16>(s, src, sstride, srow0, dst, dstride, drow0, heads, rows, d);
    else
        copy_dt<LX2V_DTYPE_F32, LX2V_DTYPE_F32>(s, src, sstride, srow0, dst, dstride, drow0, heads, rows, d);
}

void launch_kv_remap(hipStream_t s, const void *src, size_t sstride, void *dst, size_t dstride, int dt, size_t heads,
                     size_t rows, size_t d, const int *plan, int ft, const int n_ev[2], const int init_at[2],
                     const int ev_at[2], const float alpha[2]) {
    if (heads * rows * d == 0) return;
    RemapArgs a;
    a.ft = ft;
    for (int i = 0; i < 2; i++) {
        a.n_ev[i] = n_ev[i];
        a.init_at[i] = init_at[i];
        a.ev_at[i] = ev_at[i];
        a.alpha[i] = alpha[i];
    }
    const bool v4 = d % 4 == 0;
    const dim3 g = grid_for(v4 ? rows * d / 4 : rows * d, heads);
    if (dt == LX2V_DTYPE_BF16) {
        if (v4)
            hipLaunchKernelGGL((k_kv_remap<LX2V_DTYPE_BF16, 4>), g, dim3(KT), 0, s, src, sstride, dst, dstride,
                               (uint32_t)rows, (uint32_t)d, plan, a);
        else
            hipLaunchKernelGGL((k_kv_remap<LX2V_DTYPE_BF16, 1>), g, dim3(KT), 0, s, src, sstride, dst, dstride,
                               (uint32_t)rows, (uint32_t)d, plan, a);
    } else {
        if (v4)
            hipLaunchKernelGGL((k_kv_remap<LX2V_DTYPE_F32, 4>), g, dim3(KT), 0, s, src, sstride, dst, dstride,
                               (uint32_t)rows, (uint32_t)d, plan, a);
        else
            hipLaunchKernelGGL((k_kv_remap<LX2V_DTYPE_F32, 1>), g, dim3(KT), 0, s, src, sstride, dst, dstride,
                               (uint32_t)rows, (uint32_t)d, plan, a);
    }
}

}  // namespace lx2v

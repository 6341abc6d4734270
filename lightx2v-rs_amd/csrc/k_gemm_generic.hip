// k_gemm_generic.hip -- the any-shape linear: one thread per output,
// operands decoded exactly as the reference's dequantize() does
// (quant.rs:180-186, 294-303, 449-455).  It serves shapes the MFMA kernels do
// not tile (K not a multiple of 16, groups that do not divide 32, tiny
// matrices such as crates/lightx2v-model/src/check.rs:74-103's 4x3 case).
#include "device_common.hpp"
#include "runtime.hpp"

namespace lx2v {

namespace {

__device__ __forceinline__ float load_a(const void *a, int amode, size_t i) {
    if (amode == A_BF16) return bf16_bits_to_f32(((const uint16_t *)a)[i]);
    if (amode == A_E4M3) return e4m3_ocp_decode(((const uint8_t *)a)[i]);
    return ((const float *)a)[i];
}

__device__ __forceinline__ float load_w(int fmt, const void *codes, const float *scales,
                                        const float *zeros, size_t group, size_t i) {
    if (fmt == LX2V_WFMT_F32) return ((const float *)codes)[i];
    if (fmt == LX2V_WFMT_Q8) return (float)((const int8_t *)codes)[i] * scales[i / group];
    if (fmt == LX2V_WFMT_Q4) {
        uint32_t c = (((const uint8_t *)codes)[i >> 1] >> (4 * (i & 1))) & 15u;
        size_t g = i / group;
        return ((float)c - zeros[g]) * scales[g];
    }
    return e4m3_ref_decode(((const uint8_t *)codes)[i]) * scales[i / group];
}

__global__ __launch_bounds__(256) void k_gemm_generic(const void *a, int amode, const float *a_scale,
                                                      int fmt, const void *codes,
                                                      const float *scales, const float *zeros,
                                                      size_t group, const float *bias, int act,
                                                      void *y, int y_dtype, size_t M, size_t N,
                                                      size_t K) {
    size_t n = blockIdx.x * (size_t)16 + (threadIdx.x & 15);
    size_t m = blockIdx.y * (size_t)16 + (threadIdx.x >> 4);
    if (m >= M || n >= N) return;
    float acc = 0.0f;
    for (size_t k = 0; k < K; k++)
        acc += load_a(a, amode, m * K + k) * load_w(fmt, codes, scales, zeros, group, n * K + k);
    if (amode == A_E4M3) acc *= a_scale[m];
    if (bias) acc += bias[n];
    if (act == LX2V_ACT_GELU_TANH) acc = gelu_tanh(acc);
    if (y_dtype == LX2V_DTYPE_BF16)
        ((uint16_t *)y)[m * N + n] = f32_to_bf16_bits(acc);
    else
        ((float *)y)[m * N + n] = acc;
}

}  // namespace

void launch_gemm_generic(hipStream_t s, const void *a, int amode, const float *a_scale,
                         const lx2v_hip_weight *w, const float *bias, int act, void *y,
                         int y_dtype, size_t M) {
    size_t N = w->rows, K = w->cols;
    if (M == 0 || N == 0) return;
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
    hipLaunchKernelGGL(k_gemm_generic, grid, dim3(256), 0, s, a, amode, a_scale, w->fmt, w->codes,
                       w->scales, w->zeros, w->group ? w->group : 1, bias, act, y, y_dtype, M, N, K);
}

}  // namespace lx2v

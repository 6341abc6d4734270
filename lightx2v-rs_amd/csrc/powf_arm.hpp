// powf_arm.hpp -- f32 pow with the algorithm of Arm's optimized-routines
// powf (Szabolcs Nagy, 2018; math/powf.c, shipped as glibc's powf since
// 2.28), which is what the reference's `f32::powf` calls on Linux
// (crates/lightx2v-core/src/quant.rs:261, the HQQ shrink).  glibc's powf is
// not correctly rounded (up to ~0.82 ulp), so a double pow rounded once
// differs from it in the last bit for ~0.06% of arguments; this restatement
// reproduces it bit for bit.
//
// Method: x = 2^k z with z in [0x3f330000, 2 * 0x3f330000) as f32 bits; a
// 16-entry table of (1/c, log2 c) for c near the centre of z's subinterval;
// log2 x = k + log2 c + P5(z/c - 1) in double; then 2^(y log2 x) as
// 2^(j/32) * Q3(r) with |r| <= 1/64 and a 32-entry table of 2^(j/32) bit
// patterns; one rounding to f32 at the end.  The tables and polynomial
// coefficients are the published ones.  exp2 table entry j is
// bits(RN(2^(j/32))) - (j << 47), which the host test regenerates from its
// definition.
//
// Checked on the host (tests/test_powf_arm.py builds this header with g++
// and compares against the libm powf): identical results on every finite
// positive f32 (subnormals included) at y = 0.7f - 1.0f and five other
// exponents.  Each multiply-add below is one fused operation, as in the FMA
// build glibc selects on x86-64; the unfused evaluation also matched the
// libm at these exponents.
//
// Domain: x > 0 finite and |y log2 x| < 126 (no overflow / underflow
// handling).  The HQQ shrink only calls it with x = |e| > 0 and y = -0.3.
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define LX2V_HD __host__ __device__
#else
#define LX2V_HD
#endif

namespace lx2v {
namespace powf_arm {

struct LogEntry {
    double invc, logc;
};

// (1/c, log2 c) per subinterval i of z (i = top 4 mantissa bits of z - OFF).
#define LX2V_POWF_LOG2_TAB                                                                         \
    {{0x1.661ec79f8f3bep+0, -0x1.efec65b963019p-2}, {0x1.571ed4aaf883dp+0, -0x1.b0b6832d4fca4p-2}, \
     {0x1.49539f0f010bp+0, -0x1.7418b0a1fb77bp-2},  {0x1.3c995b0b80385p+0, -0x1.39de91a6dcf7bp-2}, \
     {0x1.30d190c8864a5p+0, -0x1.01d9bf3f2b631p-2}, {0x1.25e227b0b8eap+0, -0x1.97c1d1b3b7afp-3},   \
     {0x1.1bb4a4a1a343fp+0, -0x1.2f9e393af3c9fp-3}, {0x1.12358f08ae5bap+0, -0x1.960cbbf788d5cp-4}, \
     {0x1.0953f419900a7p+0, -0x1.a6f9db6475fcep-5}, {0x1p+0, 0x0p+0},                              \
     {0x1.e608cfd9a47acp-1, 0x1.338ca9f24f53dp-4},  {0x1.ca4b31f026aap-1, 0x1.476a9543891bap-3},   \
     {0x1.b2036576afce6p-1, 0x1.e840b4ac4e4d2p-3},  {0x1.9c2d163a1aa2dp-1, 0x1.40645f0c6651cp-2},  \
     {0x1.886e6037841edp-1, 0x1.88e9c2c1b9ff8p-2},  {0x1.767dcf5534862p-1, 0x1.ce0a44eb17bccp-2}}

// bits(RN(2^(j/32))) - (j << 47), j = 0..31.
#define LX2V_POWF_EXP2_TAB                                                                  \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

LX2V_HD inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
LX2V_HD inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
LX2V_HD inline uint64_t d2u(double f) {
    uint64_t u;
    memcpy(&u, &f, 8);
    return u;
}
LX2V_HD inline double u2d(uint64_t u) {
    double f;
    memcpy(&f, &u, 8);
    return f;
}

constexpr LogEntry kLog2Tab[16] = LX2V_POWF_LOG2_TAB;
constexpr uint64_t kExp2Tab[32] = LX2V_POWF_EXP2_TAB;

// One rounding: a * b + c.
LX2V_HD inline double fma_d(double a, double b, double c) { return __builtin_fma(a, b, c); }

// log2 of the normal f32 with bits ix, in double.
LX2V_HD inline double log2_inline(uint32_t ix) {
    const LogEntry *T = kLog2Tab;
    constexpr double A0 = 0x1.27616c9496e0bp-2, A1 = -0x1.71969a075c67ap-2, A2 = 0x1.ec70a6ca7baddp-2,
                     A3 = -0x1.7154748bef6c8p-1, A4 = 0x1.71547652ab82bp0;
    const uint32_t tmp = ix - 0x3f330000u;
    const int i = (int)((tmp >> 19) % 16u);
    const uint32_t top = tmp & 0xff800000u;
    const uint32_t iz = ix - top;
    const int k = (int32_t)top >> 23;  // arithmetic shift
    const double z = (double)u2f(iz);
    const double r = fma_d(z, T[i].invc, -1.0);
    const double y0 = T[i].logc + (double)k;
    const double r2 = r * r;
    double y = fma_d(A0, r, A1);
    const double p = fma_d(A2, r, A3);
    const double r4 = r2 * r2;
    double q = fma_d(A4, r, y0);
    q = fma_d(p, r2, q);
    y = fma_d(y, r4, q);
    return y;
}

// 2^xd rounded to f32, |xd| < 126.
LX2V_HD inline float exp2_inline(double xd) {
    const uint64_t *T = kExp2Tab;
    constexpr double C0 = 0x1.c6af84b912394p-5, C1 = 0x1.ebfce50fac4f3p-3, C2 = 0x1.62e42ff0c52d6p-1;
    constexpr double SHIFT = 0x1.8p+52 / 32;
    double kd = xd + SHIFT;  // round xd to a multiple of 1/32
    const uint64_t ki = d2u(kd);
    kd -= SHIFT;
    const double r = xd - kd;
    uint64_t t = T[ki % 32];
    t += ki << 47;
    const double s = u2d(t);
    const double z = fma_d(C0, r, C1);
    const double r2 = r * r;
    double y = fma_d(C2, r, 1.0);
    y = fma_d(z, r2, y);
    y = y * s;
    return (float)y;
}

// x^y for x > 0 finite, |y log2 x| < 126.
LX2V_HD inline float powf_pos(float x, float y) {
    uint32_t ix = f2u(x);
    if (ix < 0x00800000u) {  // subnormal: normalize, take 23 off the exponent
        ix = f2u(x * 0x1p23f);
        ix -= 23u << 23;
    }
    const double ylogx = (double)y * log2_inline(ix);
    return exp2_inline(ylogx);
}

#undef LX2V_POWF_LOG2_TAB
#undef LX2V_POWF_EXP2_TAB

}  // namespace powf_arm
}  // namespace lx2v

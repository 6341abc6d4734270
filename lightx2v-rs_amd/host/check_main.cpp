// check_main.cpp -- `lightx2v check --backend hip` for the linear path
// (crates/lightx2v-cli/src/main.rs:265-289 -> crates/lightx2v-model/src/
// check.rs:57-103): each check runs one op through the C ABI and compares
// with a host-computed reference, printing
//   PASS <name> max_abs_err=<e> tol=<t>
// and exits 1 on the first failure; prints `skip: <reason>` and exits 0
// when no gfx950 device answers (main.rs:232-236).
//
// Beyond the reference's 4x3 f32 `linear` check, it adds the quantized
// linears the reference's check lacks (Q8, Q4, FP8) on inputs chosen so
// every product and partial sum is exact in f32: the device result must then
// equal the host's sequential f32 loop exactly, whatever the summation order
// or the MFMA operand rounding.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "hip_backend.hpp"

using namespace lx2v_host;

namespace {

struct Result {
    std::string name;
    float err, tol;
};

float max_err(const std::vector<float> &a, const std::vector<float> &b) {
    float m = 0.0f;
    for (size_t i = 0; i < a.size() && i < b.size(); i++) m = std::fmax(m, std::fabs(a[i] - b[i]));
    if (a.size() != b.size()) m = INFINITY;
    return m;
}

uint32_t bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// y = x . w^T + b with the reference's sequential f32 loop
// (crates/lightx2v-cpu/src/lib.rs:296-326).
std::vector<float> host_linear(const std::vector<float> &x, size_t rows, const std::vector<float> &w,
                               size_t n, size_t k, const std::vector<float> &b) {
    std::vector<float> y(rows * n);
    for (size_t r = 0; r < rows; r++)
        for (size_t o = 0; o < n; o++) {
            float acc = 0.0f;
            for (size_t i = 0; i < k; i++) acc += x[r * k + i] * w[o * k + i];
            acc += b[o];
            y[r * n + o] = acc;
        }
    return y;
}

// quant.rs:409-420 closed form.
float e4m3_ref(uint8_t c) {
    float s = (c & 0x80) ? -1.0f : 1.0f;
    int e = (c >> 3) & 15, m = c & 7;
    if (e == 0) return s * ((float)m / 8.0f) * ldexpf(1.0f, -9);
    if (e == 15 && m == 7) return NAN;
    return s * (1.0f + (float)m / 8.0f) * ldexpf(1.0f, e - 7);
}

// Smallest e4m3 code whose reference value equals v (v on the grid).
uint8_t e4m3_code_of(float v) {
    for (int c = 0; c < 256; c++)
        if (e4m3_ref((uint8_t)c) == v && !((c & 0x78) == 0 && (c & 7))) return (uint8_t)c;
    return 0;
}

Result check_linear(HipBackend &be) {  // check.rs:74-103
    std::vector<float> x = {1, 2, 3, 4, 5, 6};
    std::vector<float> w = {1, 0, -1, 0.5, 1, 0.5, 2, -1, 0, 0, 1, 2};
    std::vector<float> b = {0.5, -0.5, 1, 0};
    auto xb = be.upload(x);
    auto yb = be.alloc(2 * 4);
    auto wb = be.weight(w, 4, 3);
    auto bb = be.upload(b);
    be.linear(xb, 0, 2, wb, &bb, Act::None, yb, 0);
    return {"linear", max_err(be.download(yb), host_linear(x, 2, w, 4, 3, b)), 1e-6f};
}

constexpr size_t R = 40, N = 64, K = 128;

std::vector<float> pow2_scales(size_t n, int lo) {
    std::vector<float> s(n);
    for (size_t i = 0; i < n; i++) s[i] = ldexpf(1.0f, -(lo + (int)(i * 7 % 4)));
    return s;
}

std::vector<float> exact_bias(size_t n) {
    std::vector<float> b(n);
    for (size_t i = 0; i < n; i++) b[i] = ldexpf((float)((int)(i * 37 % 29) - 14), -8);
    return b;
}

Result check_linear_q8(HipBackend &be) {
    Q8 q{std::vector<int8_t>(N * K), pow2_scales(N * K / 32, 5), N, K, 32};
    for (size_t i = 0; i < N * K; i++) q.q[i] = (int8_t)((int)(i * 7919 % 255) - 127);
    std::vector<float> x(R * K), wd(N * K);
    for (size_t i = 0; i < R * K; i++) x[i] = (float)((int)(i * 31 % 17) - 8) / 8.0f;  // bf16-exact
    for (size_t i = 0; i < N * K; i++) wd[i] = (float)q.q[i] * q.scales[i / 32];  // quant.rs:180-186
    auto b = exact_bias(N);
    auto xb = be.upload(x);
    auto bb = be.upload(b);
    auto yb = be.alloc(R * N);
    auto wb = be.weight_q8(q);
    be.linear(xb, 0, R, wb, &bb, Act::None, yb, 0);
    return {"linear q8 g32 (bf16 mfma)", max_err(be.download(yb), host_linear(x, R, wd, N, K, b)), 1e-6f};
}

Result check_linear_q4(HipBackend &be) {
    Q4 q{std::vector<uint8_t>(N * K), pow2_scales(N * K / 32, 6), std::vector<float>(N * K / 32, 8.0f), N, K, 32};
    for (size_t i = 0; i < N * K; i++) q.q[i] = (uint8_t)(i * 7919 % 16);
    std::vector<float> x(R * K), wd(N * K);
    for (size_t i = 0; i < R * K; i++) x[i] = (float)((int)(i * 13 % 15) - 7) / 4.0f;
    for (size_t i = 0; i < N * K; i++) wd[i] = ((float)q.q[i] - q.zeros[i / 32]) * q.scales[i / 32];
    auto b = exact_bias(N);
    auto xb = be.upload(x);
    auto bb = be.upload(b);
    auto yb = be.alloc(R * N);
    auto wb = be.weight_q4(q);
    be.linear(xb, 0, R, wb, &bb, Act::None, yb, 0);
    return {"linear q4 g32 (bf16 mfma)", max_err(be.download(yb), host_linear(x, R, wd, N, K, b)), 1e-6f};
}

Result check_linear_fp8(HipBackend &be) {
    // W: multiples of 1/4 in [-4, 4] (all on the e4m3 grid), per-channel
    // power-of-two scales.  X: multiples of 1/2 in [-4, 4] plus one 448 per
    // row, so the per-token scale is exactly 1 and the e4m3 activations are
    // exact.  Products are multiples of 2^-3 below 2^11: every sum is exact.
    Fp8E4M3 q{std::vector<uint8_t>(N * K), pow2_scales(N, 4), N, K, K};
    std::vector<float> x(R * K), wd(N * K);
    for (size_t i = 0; i < N * K; i++) {
        float v = (float)((int)(i * 7919 % 33) - 16) / 4.0f;
        q.q[i] = e4m3_code_of(v);
        wd[i] = e4m3_ref(q.q[i]) * q.scales[i / K];
    }
    for (size_t i = 0; i < R * K; i++) x[i] = (float)((int)(i * 29 % 17) - 8) / 2.0f;
    for (size_t r = 0; r < R; r++) x[r * K + (r * 5 % K)] = (r & 1) ? -448.0f : 448.0f;
    auto b = exact_bias(N);
    auto xb = be.upload(x);
    auto bb = be.upload(b);
    auto yb = be.alloc(R * N);
    auto wb = be.weight_fp8(q);
    be.linear(xb, 0, R, wb, &bb, Act::None, yb, 0);
    return {"linear fp8 per-channel (e4m3 mfma)", max_err(be.download(yb), host_linear(x, R, wd, N, K, b)),
            1e-6f};
}

Result check_dequant(HipBackend &be) {
    // All 256 e4m3 codes, all int8 codes, all nibbles: device decode equals
    // quant.rs's dequantize() bit for bit (NaN as NaN).
    size_t bad = 0;
    {
        Fp8E4M3 q{std::vector<uint8_t>(4 * 256), {0.5f, 0.0123f, 3.0f, 1e-3f}, 4, 256, 256};
        for (size_t i = 0; i < q.q.size(); i++) q.q[i] = (uint8_t)i;
        auto w = be.weight_fp8(q);
        auto d = be.dequantize(w);
        for (size_t i = 0; i < d.size(); i++) {
            float want = e4m3_ref(q.q[i]) * q.scales[i / 256];
            if (!(bits(d[i]) == bits(want) || (std::isnan(d[i]) && std::isnan(want)))) bad++;
        }
    }
    {
        Q8 q{std::vector<int8_t>(2 * 256), {0.25f, 0.007f, 1.5f, 3e-5f}, 2, 256, 128};
        for (size_t i = 0; i < q.q.size(); i++) q.q[i] = (int8_t)(i & 0xFF);
        auto d = be.dequantize(be.weight_q8(q));
        for (size_t i = 0; i < d.size(); i++)
            if (bits(d[i]) != bits((float)q.q[i] * q.scales[i / 128])) bad++;
    }
    {
        Q4 q{std::vector<uint8_t>(2 * 64), {0.1f, 0.03f, 2.0f, 0.5f}, {7.5f, 8.0f, 0.0f, 15.0f}, 2, 64, 32};
        for (size_t i = 0; i < q.q.size(); i++) q.q[i] = (uint8_t)(i % 16);
        auto d = be.dequantize(be.weight_q4(q));
        for (size_t i = 0; i < d.size(); i++)
            if (bits(d[i]) != bits(((float)q.q[i] - q.zeros[i / 32]) * q.scales[i / 32])) bad++;
    }
    return {"dequant q8/q4/fp8 bit-exact", (float)bad, 0.0f};
}

}  // namespace

int main() {
    std::string why;
    auto be = HipBackend::try_new(0, &why);
    if (!be) {
        printf("skip: hip backend unavailable (%s)\n", why.c_str());
        return 0;
    }
    printf("backend: %s\n", be->name().c_str());
    std::vector<std::function<Result(HipBackend &)>> checks = {check_linear, check_linear_q8, check_linear_q4,
                                                               check_linear_fp8, check_dequant};
    int passed = 0, failed = 0;
    for (auto &c : checks) {
        Result r;
        try {
            r = c(*be);
        } catch (const std::exception &e) {
            printf("FAIL error: %s\n", e.what());
            failed++;
            continue;
        }
        bool ok = r.err <= r.tol;
        printf("%s %-40s max_abs_err=%.3e tol=%.0e\n", ok ? "PASS" : "FAIL", r.name.c_str(), r.err, r.tol);
        (ok ? passed : failed)++;
    }
    printf("%d checks, %d passed, %d failed\n", passed + failed, passed, failed);
    return failed ? 1 : 0;
}

// hip_backend.hpp -- C++ host mirror of the lightx2v-rs `Backend` trait's
// linear path (crates/lightx2v-core/src/backend.rs:145-212) over the C ABI of
// include/lightx2v_hip.h: the same surface a `lightx2v-hip` Rust crate binds,
// with the same names, argument meaning and error behaviour (misuse throws,
// as the trait panics; try_new returns nullopt on a host without a gfx950
// device, as WgpuBackend::try_new returns None).
#pragma once

#include <cstdint>
#include <cstring>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "lightx2v_hip.h"

namespace lx2v_host {

// The reference's host-side weight types (crates/lightx2v-core/src/quant.rs),
// as plain data the backend borrows and copies into HBM.
struct Q8 {  // quant.rs:142-151
    std::vector<int8_t> q;
    std::vector<float> scales;  // [rows, cols / group]
    size_t rows = 0, cols = 0, group = 0;
};
struct Q4 {  // quant.rs:211-220 (one code 0..15 per byte)
    std::vector<uint8_t> q;
    std::vector<float> scales, zeros;
    size_t rows = 0, cols = 0, group = 0;
};
struct Fp8E4M3 {  // quant.rs:364-373
    std::vector<uint8_t> q;
    std::vector<float> scales;
    size_t rows = 0, cols = 0, group = 0;
};

enum class Act { None = LX2V_ACT_NONE, GeluTanh = LX2V_ACT_GELU_TANH };  // backend.rs:38-43

struct Error : std::runtime_error {
    int status;
    Error(int s, const std::string &m) : std::runtime_error(m), status(s) {}
};

inline void check(int rc) {
    if (rc != LX2V_OK) throw Error(rc, std::string("lightx2v-hip: ") + lx2v_hip_last_error());
}

class HipBackend;

class Buf {
  public:
    Buf(lx2v_hip_ctx *ctx, lx2v_hip_buf *h) : ctx_(ctx), h_(h) {}
    Buf(Buf &&o) noexcept : ctx_(o.ctx_), h_(std::exchange(o.h_, nullptr)) {}
    Buf &operator=(Buf &&o) noexcept {
        std::swap(ctx_, o.ctx_);
        std::swap(h_, o.h_);
        return *this;
    }
    Buf(const Buf &) = delete;
    ~Buf() {
        if (h_) lx2v_hip_buf_free(ctx_, h_);
    }
    lx2v_hip_buf *raw() const { return h_; }

  private:
    lx2v_hip_ctx *ctx_;
    lx2v_hip_buf *h_;
};

class Weight {
  public:
    Weight(lx2v_hip_ctx *ctx, lx2v_hip_weight *h) : ctx_(ctx), h_(h) {}
    Weight(Weight &&o) noexcept : ctx_(o.ctx_), h_(std::exchange(o.h_, nullptr)) {}
    Weight(const Weight &) = delete;
    ~Weight() {
        if (h_) lx2v_hip_weight_free(ctx_, h_);
    }
    lx2v_hip_weight *raw() const { return h_; }
    lx2v_hip_weight_info_t info() const {
        lx2v_hip_weight_info_t i;
        check(lx2v_hip_weight_info(h_, &i));
        return i;
    }

  private:
    lx2v_hip_ctx *ctx_;
    lx2v_hip_weight *h_;
};

class HipBackend {
  public:
    explicit HipBackend(int device = 0) { check(lx2v_hip_create(device, &ctx_)); }
    HipBackend(const HipBackend &) = delete;
    HipBackend(HipBackend &&o) noexcept : ctx_(std::exchange(o.ctx_, nullptr)) {}
    ~HipBackend() {
        if (ctx_) lx2v_hip_destroy(ctx_);
    }

    // WgpuBackend::try_new (crates/lightx2v-wgpu/src/lib.rs:282-287).
    static std::optional<HipBackend> try_new(int device = 0, std::string *why = nullptr) {
        lx2v_hip_ctx *c = nullptr;
        int rc = lx2v_hip_create(device, &c);
        if (rc == LX2V_ERR_NO_DEVICE) {
            if (why) *why = lx2v_hip_last_error();
            return std::nullopt;
        }
        check(rc);
        return HipBackend(c);
    }

    std::string name() const {  // backend.rs:158
        char b[256];
        check(lx2v_hip_name(ctx_, b, sizeof b));
        return b;
    }
    void set_act_dtype(int dtype) { check(lx2v_hip_set_act_dtype(ctx_, dtype)); }
    void set_fp8_act(int mode) { check(lx2v_hip_set_fp8_act(ctx_, mode)); }

    // ---- memory (backend.rs:160-177)
    Buf alloc(size_t len) {
        lx2v_hip_buf *h = nullptr;
        check(lx2v_hip_alloc(ctx_, len, &h));
        return Buf(ctx_, h);
    }
    Buf upload(const std::vector<float> &data) {
        lx2v_hip_buf *h = nullptr;
        check(lx2v_hip_upload(ctx_, data.data(), data.size(), &h));
        return Buf(ctx_, h);
    }
    void write(const Buf &b, const std::vector<float> &data) {
        check(lx2v_hip_write(ctx_, b.raw(), data.data(), data.size()));
    }
    std::vector<float> download(const Buf &b) {
        std::vector<float> out(buf_len(b));
        check(lx2v_hip_download(ctx_, b.raw(), out.data(), out.size()));
        return out;
    }
    size_t buf_len(const Buf &b) const {
        size_t n = 0;
        check(lx2v_hip_buf_len(b.raw(), &n));
        return n;
    }
    void copy(const Buf &src, size_t src_off, const Buf &dst, size_t dst_off, size_t len) {
        check(lx2v_hip_copy(ctx_, src.raw(), src_off, dst.raw(), dst_off, len));
    }

    // ---- weights (backend.rs:178-188)
    Weight weight(const std::vector<float> &data, size_t rows, size_t cols) {
        if (data.size() != rows * cols) throw Error(LX2V_ERR_BAD_SHAPE, "weight: data.len() != rows * cols");
        lx2v_hip_weight *h = nullptr;
        check(lx2v_hip_weight_f32(ctx_, data.data(), rows, cols, &h));
        return Weight(ctx_, h);
    }
    Weight weight_q8(const Q8 &q) {
        lx2v_hip_weight *h = nullptr;
        check(lx2v_hip_weight_q8(ctx_, q.q.data(), q.scales.data(), q.rows, q.cols, q.group, &h));
        return Weight(ctx_, h);
    }
    Weight weight_q4(const Q4 &q) {
        lx2v_hip_weight *h = nullptr;
        check(lx2v_hip_weight_q4(ctx_, q.q.data(), 0, q.scales.data(), q.zeros.data(), q.rows, q.cols,
                                 q.group, &h));
        return Weight(ctx_, h);
    }
    Weight weight_fp8(const Fp8E4M3 &q) {
        lx2v_hip_weight *h = nullptr;
        check(lx2v_hip_weight_fp8(ctx_, q.q.data(), q.scales.data(), q.rows, q.cols, q.group, &h));
        return Weight(ctx_, h);
    }
    std::vector<float> dequantize(const Weight &w) {
        auto i = w.info();
        std::vector<float> out(i.rows * i.cols);
        check(lx2v_hip_weight_dequantize(ctx_, w.raw(), out.data(), out.size()));
        return out;
    }

    void sync() { check(lx2v_hip_sync(ctx_)); }  // backend.rs:189-190
    std::optional<std::string> profile_report() {  // backend.rs:192-195
        std::string s(1 << 16, '\0');
        check(lx2v_hip_profile_report(ctx_, s.data(), s.size()));
        s.resize(strlen(s.c_str()));
        if (s.empty()) return std::nullopt;
        return s;
    }
    void profile_reset() { check(lx2v_hip_profile_reset(ctx_)); }  // backend.rs:196
    void profile_enable(bool on) { check(lx2v_hip_profile_enable(ctx_, on ? 1 : 0)); }

    // ---- transformer (backend.rs:198-212)
    void linear(const Buf &x, size_t x_row, size_t rows, const Weight &w, const Buf *bias, Act act,
                const Buf &y, size_t y_row) {
        check(lx2v_hip_linear(ctx_, x.raw(), x_row, rows, w.raw(), bias ? bias->raw() : nullptr, (int)act,
                              y.raw(), y_row));
    }

  private:
    explicit HipBackend(lx2v_hip_ctx *c) : ctx_(c) {}
    lx2v_hip_ctx *ctx_ = nullptr;
};

}  // namespace lx2v_host

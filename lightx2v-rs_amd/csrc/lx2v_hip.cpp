// lx2v_hip.cpp -- the C ABI of include/lightx2v_hip.h: context, buffers,
// weights, the linear dispatch and the per-kernel profiler.  Each entry point
// cites the Backend trait method it implements (crates/lightx2v-core/src/
// backend.rs).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "runtime.hpp"

using namespace lx2v;

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(e == hipErrorOutOfMemory ? LX2V_ERR_OOM : LX2V_ERR_HIP, "%s: %s", what,
                hipGetErrorString(e));
}

#define HIP_TRY(call, what)                     \
    do {                                        \
        hipError_t e_ = (call);                 \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

#define NEED(p, name) \
    if (!(p)) return fail(LX2V_ERR_BAD_ARG, "%s is null", name)

int ok() {
    g_err.clear();
    return LX2V_OK;
}

bool valid_dtype(int d) { return d == LX2V_DTYPE_F32 || d == LX2V_DTYPE_BF16; }

int ensure(lx2v_hip_ctx *ctx, void **ptr, size_t *have, size_t need, const char *what) {
    if (*have >= need) return LX2V_OK;
    if (ctx->capturing)
        return fail(LX2V_ERR_UNSUPPORTED, "%s: would grow a workspace during graph capture (run the sequence "
                    "once before capturing)", what);
    if (*ptr) {
        HIP_TRY(hipStreamSynchronize(ctx->stream), what);
        HIP_TRY(hipFree(*ptr), what);
        *ptr = nullptr;
        *have = 0;
    }
    size_t sz = std::max<size_t>(need, 1 << 20);
    HIP_TRY(hipMalloc(ptr, sz), what);
    *have = sz;
    return LX2V_OK;
}


// Byte ranges [a, a+na) and [b, b+nb) overlap.
bool overlap(const void *a, size_t na, const void *b, size_t nb) {
    uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return na && nb && x < y + nb && y < x + na;
}

int set_dev(const lx2v_hip_ctx *ctx) {
    HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
    return LX2V_OK;
}

// Calls that allocate, free, move host data or synchronise cannot be
// recorded into a graph.
int not_capturing(const lx2v_hip_ctx *ctx, const char *what) {
    if (ctx->capturing) return fail(LX2V_ERR_UNSUPPORTED, "%s is not allowed during graph capture", what);
    return LX2V_OK;
}

}  // namespace

namespace lx2v {

void prof_begin(lx2v_hip_ctx *ctx, const char *name, hipEvent_t *a, hipEvent_t *b) {
    auto &p = ctx->prof;
    for (hipEvent_t *e : {a, b}) {
        if (!p.pool.empty()) {
            *e = p.pool.back();
            p.pool.pop_back();
        } else if (hipEventCreate(e) != hipSuccess) {
            *e = nullptr;
        }
    }
    if (*a) (void)hipEventRecord(*a, ctx->stream);
    p.pending.push_back({name, *a, *b});
}

void prof_end(lx2v_hip_ctx *ctx, hipEvent_t b) {
    if (b) (void)hipEventRecord(b, ctx->stream);
}

}  // namespace lx2v

namespace {

void prof_harvest(lx2v_hip_ctx *ctx) {
    auto &p = ctx->prof;
    if (p.pending.empty()) return;
    (void)hipStreamSynchronize(ctx->stream);
    for (auto &e : p.pending) {
        float ms = 0.0f;
        if (e.a && e.b && hipEventElapsedTime(&ms, e.a, e.b) == hipSuccess) {
            auto &s = p.stats[e.name];
            s.first += 1;
            s.second += ms;
        }
        if (e.a) p.pool.push_back(e.a);
        if (e.b) p.pool.push_back(e.b);
    }
    p.pending.clear();
}

template <class F>
int run(lx2v_hip_ctx *ctx, const char *name, F &&fn) {
    if (ctx->capturing) {  // no per-kernel events inside a graph
        fn();
        hipError_t e = hipGetLastError();
        return e == hipSuccess ? LX2V_OK : hip_fail(e, name);
    }
    hipError_t e = timed(ctx, name, fn);
    if (ctx->prof.on && ctx->prof.pending.size() > 8192) prof_harvest(ctx);
    if (e != hipSuccess) return hip_fail(e, name);
    return LX2V_OK;
}

int stage_for(lx2v_hip_ctx *ctx, size_t bytes, void **out) {
    auto &st = ctx->stage;
    int rc = ensure(ctx, &st.ptr, &st.bytes, bytes, "staging alloc");
    if (rc) return rc;
    *out = st.ptr;
    return LX2V_OK;
}

int alloc_buf(lx2v_hip_ctx *ctx, size_t len, int dtype, lx2v_hip_buf **out) {
    auto *b = new lx2v_hip_buf;
    b->len = len;
    b->dtype = dtype;
    hipError_t e = hipMalloc(&b->ptr, std::max<size_t>(b->bytes(), 4));
    if (e != hipSuccess) {
        delete b;
        return hip_fail(e, "hipMalloc(buffer)");
    }
    e = hipMemsetAsync(b->ptr, 0, std::max<size_t>(b->bytes(), 4), ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(b->ptr);
        delete b;
        return hip_fail(e, "hipMemsetAsync(buffer)");
    }
    *out = b;
    return LX2V_OK;
}

// host f32 -> device buffer elements [off, off+len)
int write_range(lx2v_hip_ctx *ctx, lx2v_hip_buf *b, size_t off, const float *data, size_t len) {
    if (!len) return LX2V_OK;
    if (b->dtype == LX2V_DTYPE_F32) {
        HIP_TRY(hipMemcpyAsync((float *)b->ptr + off, data, len * 4, hipMemcpyHostToDevice, ctx->stream),
                "hipMemcpyAsync(write)");
        return LX2V_OK;
    }
    void *st;
    int rc = stage_for(ctx, len * 4, &st);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(st, data, len * 4, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync(write)");
    return run(ctx, "convert", [&] {
        launch_convert(ctx->stream, st, LX2V_DTYPE_F32, (uint16_t *)b->ptr + off, LX2V_DTYPE_BF16, len);
    });
}

template <class T>
int upload_raw(T **dst, const void *src, size_t bytes, hipStream_t s, const char *what) {
    hipError_t e = hipMalloc((void **)dst, std::max<size_t>(bytes, 4));
    if (e != hipSuccess) return hip_fail(e, what);
    if (bytes) {
        e = hipMemcpyAsync(*dst, src, bytes, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return hip_fail(e, what);
    }
    return LX2V_OK;
}

void free_weight(lx2v_hip_weight *w) {
    if (!w) return;
    if (w->codes) (void)hipFree(w->codes);
    if (w->scales) (void)hipFree(w->scales);
    if (w->zeros) (void)hipFree(w->zeros);
    if (w->raw_e4m3) (void)hipFree(w->raw_e4m3);
    if (w->sscale) (void)hipFree(w->sscale);
    if (w->szero) (void)hipFree(w->szero);
    if (w->gratio) (void)hipFree(w->gratio);
    if (w->glast) (void)hipFree(w->glast);
    if (w->wbf16) (void)hipFree(w->wbf16);
    delete w;
}

int group_ratios(lx2v_hip_ctx *ctx, lx2v_hip_weight *w);

// The stage-major scale copy (lx2v_hip_weight::sscale) of a weight the
// direct-to-LDS bf16 GEMM takes, built on the stream after the scales.
int stage_scales(lx2v_hip_ctx *ctx, lx2v_hip_weight *w) {
    if (w->fmt == LX2V_WFMT_F32 || w->cols % 64 || w->group % 16) return LX2V_OK;
    const size_t g = w->group;
    w->spr = g % 64 == 0 ? 1 : (g == 32 ? 2 : 4);
    const size_t n = w->cols / 64 * w->rows * (size_t)w->spr;
    HIP_TRY(hipMalloc((void **)&w->sscale, n * 4), "stage_scales alloc");
    if (w->fmt == LX2V_WFMT_Q4) HIP_TRY(hipMalloc((void **)&w->szero, n * 4), "stage_scales alloc");
    w->device_bytes += n * 4 * (w->szero ? 2 : 1);
    if (int rc = run(ctx, "stage_scales", [&] { launch_stage_scales(ctx->stream, w); })) return rc;
    return group_ratios(ctx, w);
}

// FP8 group 128: the per-group scale ratios and last-group scales the fp8
// MFMA kernels take (lx2v_hip_weight::gratio), from the weight's scales
// (load time: one copy to the host and back).
int group_ratios(lx2v_hip_ctx *ctx, lx2v_hip_weight *w) {
    if (w->fmt != LX2V_WFMT_FP8 || w->group != 128 || w->cols % 128) return LX2V_OK;
    const size_t rows = w->rows, G = w->cols / 128;
    std::vector<float> s(rows * G), r(rows * G), last(rows);
    HIP_TRY(hipMemcpyAsync(s.data(), w->scales, s.size() * 4, hipMemcpyDeviceToHost, ctx->stream), "group scales");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "group scales");
    bool ok = true;
    for (size_t n = 0; n < rows && ok; n++) {
        const float *sn = s.data() + n * G;
        float lo = sn[0], hi = sn[0];
        for (size_t g = 0; g < G; g++) {
            if (!(sn[g] > 0.0f && sn[g] <= 3.4e38f)) ok = false;  // finite and positive (NaN fails)
            lo = std::min(lo, sn[g]);
            hi = std::max(hi, sn[g]);
        }
        if (ok && hi > lo * 0x1p60f) ok = false;
        for (size_t g = 0; g < G; g++) r[g * rows + n] = g == 0 ? 1.0f : sn[g - 1] / sn[g];
        last[n] = sn[G - 1];
    }
    w->gratio_ok = ok;
    if (!ok) return LX2V_OK;
    HIP_TRY(hipMalloc((void **)&w->gratio, r.size() * 4), "group ratios alloc");
    HIP_TRY(hipMalloc((void **)&w->glast, rows * 4), "group ratios alloc");
    w->device_bytes += (r.size() + rows) * 4;
    HIP_TRY(hipMemcpyAsync(w->gratio, r.data(), r.size() * 4, hipMemcpyHostToDevice, ctx->stream), "group ratios");
    HIP_TRY(hipMemcpyAsync(w->glast, last.data(), rows * 4, hipMemcpyHostToDevice, ctx->stream), "group ratios");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "group ratios");
    return LX2V_OK;
}

int check_quant_shape(size_t rows, size_t cols, size_t group) {
    if (!rows || !cols) return fail(LX2V_ERR_BAD_SHAPE, "empty weight %zux%zu", rows, cols);
    if (!group || cols % group)
        return fail(LX2V_ERR_BAD_SHAPE, "group %zu does not divide cols %zu", group, cols);
    return LX2V_OK;
}

}  // namespace

// ============================================================================
extern "C" {

const char *lx2v_hip_last_error(void) { return g_err.c_str(); }

int lx2v_hip_device_count(int *count) {
    NEED(count, "count");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return ok();
}

int lx2v_hip_create(int device, lx2v_hip_ctx **out) {
    NEED(out, "out");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(LX2V_ERR_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= n)
        return fail(LX2V_ERR_NO_DEVICE, "device %d out of range (%d visible)", device, n);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(LX2V_ERR_NO_DEVICE, "device %d is %s, this build targets gfx950", device,
                    prop.gcnArchName);
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    // The no-alloc entry point's scratch on this device (resolved once per
    // device; a failure is retried and reported by that entry point).
    (void)scratch_setup(device);
    auto *ctx = new lx2v_hip_ctx;
    ctx->device = device;
    ctx->num_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    ctx->name = std::string("hip:") + prop.name + " (" + prop.gcnArchName + ")";
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return hip_fail(e, "hipStreamCreate");
    }
    e = hipEventCreateWithFlags(&ctx->scratch_done, hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return hip_fail(e, "hipEventCreate");
    }
    const char *pv = getenv("LIGHTX2V_PROFILE");
    ctx->prof.on = pv && strcmp(pv, "0") != 0;
    *out = ctx;
    return ok();
}

int lx2v_hip_destroy(lx2v_hip_ctx *ctx) {
    if (!ctx) return ok();
    set_dev(ctx);
    if (ctx->capturing) {  // abandon an unfinished capture
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(ctx->stream, &g);
        if (g) (void)hipGraphDestroy(g);
        ctx->capturing = false;
    }
    (void)hipStreamSynchronize(ctx->stream);
    scratch_release(ctx->device, ctx);
    if (ctx->scratch_done) (void)hipEventDestroy(ctx->scratch_done);
    prof_harvest(ctx);
    for (auto e : ctx->prof.pool) (void)hipEventDestroy(e);
    for (auto &r : ctx->prof.open_regions) (void)hipEventDestroy(r.second);
    if (ctx->ws) (void)hipFree(ctx->ws);
    for (lx2v::Stage *x : {&ctx->stage, &ctx->mask, &ctx->kv_spare, &ctx->resid, &ctx->attn, &ctx->splitk})
        if (x->ptr) (void)hipFree(x->ptr);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return ok();
}

int lx2v_hip_name(const lx2v_hip_ctx *ctx, char *out, size_t cap) {
    NEED(ctx, "ctx");
    NEED(out, "out");
    if (!cap) return fail(LX2V_ERR_BAD_ARG, "cap is 0");
    snprintf(out, cap, "%s", ctx->name.c_str());
    return ok();
}

int lx2v_hip_set_act_dtype(lx2v_hip_ctx *ctx, int dtype) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "set_act_dtype")) return rc;
    if (!valid_dtype(dtype)) return fail(LX2V_ERR_BAD_ARG, "unknown dtype %d", dtype);
    ctx->act_dtype = dtype;
    return ok();
}

int lx2v_hip_set_native_mode(lx2v_hip_ctx *ctx, int mode) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "set_native_mode")) return rc;
    if (mode != LX2V_NATIVE_BF16 && mode != LX2V_NATIVE_F32)
        return fail(LX2V_ERR_BAD_ARG, "unknown native weight mode %d", mode);
    ctx->native_mode = mode;
    return ok();
}

int lx2v_hip_set_fp8_act(lx2v_hip_ctx *ctx, int mode) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "set_fp8_act")) return rc;
    if (mode != LX2V_FP8_ACT_E4M3 && mode != LX2V_FP8_ACT_BF16)
        return fail(LX2V_ERR_BAD_ARG, "unknown fp8 activation mode %d", mode);
    ctx->fp8_act = mode;
    return ok();
}

// ---- buffers -------------------------------------------------------------------

int lx2v_hip_alloc_dtype(lx2v_hip_ctx *ctx, size_t len, int dtype, lx2v_hip_buf **out) {
    NEED(ctx, "ctx");
    NEED(out, "out");
    if (!valid_dtype(dtype))
        return fail(LX2V_ERR_BAD_ARG, "unknown dtype %d (E4M3 / MXE4M3 buffers come from lx2v_hip_alloc_e4m3 / _mx)",
                    dtype);
    if (int rc = not_capturing(ctx, "alloc")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    if (int rc = alloc_buf(ctx, len, dtype, out)) return rc;
    return ok();
}

int lx2v_hip_alloc(lx2v_hip_ctx *ctx, size_t len, lx2v_hip_buf **out) {
    NEED(ctx, "ctx");
    return lx2v_hip_alloc_dtype(ctx, len, ctx->act_dtype, out);
}

int lx2v_hip_upload(lx2v_hip_ctx *ctx, const float *data, size_t len, lx2v_hip_buf **out) {
    NEED(ctx, "ctx");
    NEED(out, "out");
    if (len) NEED(data, "data");
    if (int rc = not_capturing(ctx, "upload")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    lx2v_hip_buf *b = nullptr;
    if (int rc = alloc_buf(ctx, len, ctx->act_dtype, &b)) return rc;
    if (int rc = write_range(ctx, b, 0, data, len)) {
        (void)hipFree(b->ptr);
        delete b;
        return rc;
    }
    *out = b;
    return ok();
}

int lx2v_hip_write(lx2v_hip_ctx *ctx, lx2v_hip_buf *buf, const float *data, size_t len) {
    NEED(ctx, "ctx");
    NEED(buf, "buf");
    if (len) NEED(data, "data");
    if (buf->quantized())
        return fail(LX2V_ERR_BAD_ARG, "write into an E4M3 / MXE4M3 buffer (use lx2v_hip_quantize_act / _mx)");
    if (len > buf->len) return fail(LX2V_ERR_BAD_SHAPE, "write of %zu elements into a buffer of %zu", len, buf->len);
    if (int rc = not_capturing(ctx, "write")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    if (int rc = write_range(ctx, buf, 0, data, len)) return rc;
    return ok();
}

int lx2v_hip_download(lx2v_hip_ctx *ctx, const lx2v_hip_buf *buf, float *out, size_t len) {
    NEED(ctx, "ctx");
    NEED(buf, "buf");
    if (len != buf->len) return fail(LX2V_ERR_BAD_SHAPE, "download of %zu elements from a buffer of %zu", len, buf->len);
    if (len) NEED(out, "out");
    if (int rc = not_capturing(ctx, "download")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    if (len) {
        const void *src = buf->ptr;
        if (buf->dtype == LX2V_DTYPE_E4M3) {  // the values the codes stand for: code * row scale
            void *st;
            if (int rc = stage_for(ctx, len * 4, &st)) return rc;
            if (int rc = run(ctx, "convert", [&] {
                    launch_decode_e4m3_rows(ctx->stream, (const uint8_t *)buf->ptr, buf->scales, buf->rows, buf->cols,
                                            (float *)st);
                }))
                return rc;
            src = st;
        } else if (buf->dtype == LX2V_DTYPE_MXE4M3) {  // code * 2^(scale byte - 127)
            void *st;
            if (int rc = stage_for(ctx, len * 4, &st)) return rc;
            if (int rc = run(ctx, "convert", [&] {
                    launch_decode_mx(ctx->stream, (const uint8_t *)buf->ptr, buf->mxs, buf->rows, buf->cols,
                                     buf->srows, (float *)st);
                }))
                return rc;
            src = st;
        } else if (buf->dtype == LX2V_DTYPE_BF16) {
            void *st;
            if (int rc = stage_for(ctx, len * 4, &st)) return rc;
            if (int rc = run(ctx, "convert", [&] {
                    launch_convert(ctx->stream, buf->ptr, LX2V_DTYPE_BF16, st, LX2V_DTYPE_F32, len);
                }))
                return rc;
            src = st;
        }
        HIP_TRY(hipMemcpyAsync(out, src, len * 4, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync(download)");
    }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(download)");
    return ok();
}

int lx2v_hip_buf_len(const lx2v_hip_buf *buf, size_t *len) {
    NEED(buf, "buf");
    NEED(len, "len");
    *len = buf->len;
    return ok();
}

int lx2v_hip_buf_dtype(const lx2v_hip_buf *buf, int *dtype) {
    NEED(buf, "buf");
    NEED(dtype, "dtype");
    *dtype = buf->dtype;
    return ok();
}

int lx2v_hip_copy(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t src_off, lx2v_hip_buf *dst,
                  size_t dst_off, size_t len) {
    NEED(ctx, "ctx");
    NEED(src, "src");
    NEED(dst, "dst");
    if (src_off > src->len || len > src->len - src_off || dst_off > dst->len || len > dst->len - dst_off)
        return fail(LX2V_ERR_BAD_SHAPE, "copy [%zu,+%zu) -> [%zu,+%zu) out of range (%zu, %zu)", src_off, len,
                    dst_off, len, src->len, dst->len);
    if (src->quantized() || dst->quantized()) return fail(LX2V_ERR_BAD_ARG, "copy to or from an E4M3 / MXE4M3 buffer");
    if (!len) return ok();
    if (int rc = set_dev(ctx)) return rc;
    const char *s = (const char *)src->ptr + src_off * src->elem_bytes();
    char *d = (char *)dst->ptr + dst_off * dst->elem_bytes();
    if (src->dtype == dst->dtype) {
        HIP_TRY(hipMemcpyAsync(d, s, len * src->elem_bytes(), hipMemcpyDeviceToDevice, ctx->stream),
                "hipMemcpyAsync(copy)");
        return ok();
    }
    if (int rc = run(ctx, "convert", [&] { launch_convert(ctx->stream, s, src->dtype, d, dst->dtype, len); }))
        return rc;
    return ok();
}

int lx2v_hip_buf_free(lx2v_hip_ctx *ctx, lx2v_hip_buf *buf) {
    NEED(ctx, "ctx");
    if (!buf) return ok();
    if (int rc = not_capturing(ctx, "buf_free")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(free)");
    (void)hipFree(buf->ptr);
    delete buf;
    return ok();
}

// ---- weights ---------------------------------------------------------------------

int lx2v_hip_weight_f32(lx2v_hip_ctx *ctx, const float *data, size_t rows, size_t cols,
                        lx2v_hip_weight **out) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "weight_f32")) return rc;
    NEED(out, "out");
    NEED(data, "data");
    if (!rows || !cols) return fail(LX2V_ERR_BAD_SHAPE, "empty weight %zux%zu", rows, cols);
    if (int rc = set_dev(ctx)) return rc;
    auto *w = new lx2v_hip_weight;
    w->fmt = LX2V_WFMT_F32;
    w->rows = rows;
    w->cols = cols;
    w->group = cols;
    int rc = upload_raw((float **)&w->codes, data, rows * cols * 4, ctx->stream, "weight_f32");
    if (rc) {
        free_weight(w);
        return rc;
    }
    w->device_bytes = rows * cols * 4;
    // The bf16 copy the bf16 MFMA reads (RNE), for shapes it tiles.
    if (cols % 64 == 0 && rows * cols * 2 < (1ull << 31)) {
        if (hipMalloc((void **)&w->wbf16, rows * cols * 2) != hipSuccess) {
            w->wbf16 = nullptr;
            free_weight(w);
            return fail(LX2V_ERR_OOM, "weight_f32: %zu bytes for the bf16 copy", rows * cols * 2);
        }
        launch_convert(ctx->stream, w->codes, LX2V_DTYPE_F32, w->wbf16, LX2V_DTYPE_BF16, rows * cols);
        w->device_bytes += rows * cols * 2;
    }
    {
        const hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            free_weight(w);
            return hip_fail(e, "weight upload");
        }
    }
    *out = w;
    return ok();
}

int lx2v_hip_weight_q8(lx2v_hip_ctx *ctx, const int8_t *q, const float *scales, size_t rows,
                       size_t cols, size_t group, lx2v_hip_weight **out) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "weight_q8")) return rc;
    NEED(out, "out");
    NEED(q, "q");
    NEED(scales, "scales");
    if (int rc = check_quant_shape(rows, cols, group)) return rc;
    if (int rc = set_dev(ctx)) return rc;
    auto *w = new lx2v_hip_weight;
    w->fmt = LX2V_WFMT_Q8;
    w->rows = rows;
    w->cols = cols;
    w->group = group;
    size_t n = rows * cols, ns = n / group;
    int rc = upload_raw((int8_t **)&w->codes, q, n, ctx->stream, "weight_q8");
    if (!rc) rc = upload_raw(&w->scales, scales, ns * 4, ctx->stream, "weight_q8 scales");
    if (rc) {
        free_weight(w);
        return rc;
    }
    w->device_bytes = n + ns * 4;
    if (int rc2 = stage_scales(ctx, w)) {
        free_weight(w);
        return rc2;
    }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "weight upload");
    *out = w;
    return ok();
}

int lx2v_hip_weight_q4(lx2v_hip_ctx *ctx, const uint8_t *codes, int packed, const float *scales,
                       const float *zeros, size_t rows, size_t cols, size_t group,
                       lx2v_hip_weight **out) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "weight_q4")) return rc;
    NEED(out, "out");
    NEED(codes, "codes");
    NEED(scales, "scales");
    NEED(zeros, "zeros");
    if (int rc = check_quant_shape(rows, cols, group)) return rc;
    if (int rc = set_dev(ctx)) return rc;
    size_t n = rows * cols, np = (n + 1) / 2, ns = n / group;
    std::vector<uint8_t> pk;
    const uint8_t *src = codes;
    if (!packed) {  // Q4::packed (quant.rs:305-311)
        pk.resize(np);
        for (size_t i = 0; i < n; i += 2) {
            uint8_t lo = codes[i], hi = i + 1 < n ? codes[i + 1] : 0;
            if (lo > 15 || hi > 15)
                return fail(LX2V_ERR_BAD_ARG, "q4 code %u at %zu is not in 0..15", lo > 15 ? lo : hi,
                            lo > 15 ? i : i + 1);
            pk[i / 2] = (uint8_t)(lo | (hi << 4));
        }
        src = pk.data();
    }
    auto *w = new lx2v_hip_weight;
    w->fmt = LX2V_WFMT_Q4;
    w->rows = rows;
    w->cols = cols;
    w->group = group;
    int rc = upload_raw((uint8_t **)&w->codes, src, np, ctx->stream, "weight_q4");
    if (!rc) rc = upload_raw(&w->scales, scales, ns * 4, ctx->stream, "weight_q4 scales");
    if (!rc) rc = upload_raw(&w->zeros, zeros, ns * 4, ctx->stream, "weight_q4 zeros");
    if (rc) {
        free_weight(w);
        return rc;
    }
    w->device_bytes = np + 2 * ns * 4;
    w->zero8 = std::all_of(zeros, zeros + ns, [](float z) { return z == 8.0f; });
    if (int rc2 = stage_scales(ctx, w)) {
        free_weight(w);
        return rc2;
    }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "weight upload");  // pk must outlive the copy
    *out = w;
    return ok();
}

int lx2v_hip_weight_fp8(lx2v_hip_ctx *ctx, const uint8_t *q, const float *scales, size_t rows,
                        size_t cols, size_t group, lx2v_hip_weight **out) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "weight_fp8")) return rc;
    NEED(out, "out");
    NEED(q, "q");
    NEED(scales, "scales");
    if (int rc = check_quant_shape(rows, cols, group)) return rc;
    if (int rc = set_dev(ctx)) return rc;
    size_t n = rows * cols, ns = n / group;
    // Exponent-0, non-zero-mantissa codes: the reference decodes m * 2^-12
    // (quant.rs:413-414), the MFMA would decode m * 2^-9; store signed zero.
    std::vector<uint8_t> canon;
    size_t changed = 0;
    for (size_t i = 0; i < n; i++)
        if ((q[i] & 0x78) == 0 && (q[i] & 7) != 0) {
            if (canon.empty()) canon.assign(q, q + n);
            canon[i] = q[i] & 0x80;
            changed++;
        }
    auto *w = new lx2v_hip_weight;
    w->fmt = LX2V_WFMT_FP8;
    w->rows = rows;
    w->cols = cols;
    w->group = group;
    w->canonicalized = changed;
    int rc = upload_raw((uint8_t **)&w->codes, changed ? canon.data() : q, n, ctx->stream, "weight_fp8");
    if (!rc && changed) rc = upload_raw(&w->raw_e4m3, q, n, ctx->stream, "weight_fp8 raw");
    if (!rc) rc = upload_raw(&w->scales, scales, ns * 4, ctx->stream, "weight_fp8 scales");
    if (rc) {
        free_weight(w);
        return rc;
    }
    w->device_bytes = n + ns * 4;
    if (int rc2 = stage_scales(ctx, w)) {
        free_weight(w);
        return rc2;
    }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "weight upload");
    *out = w;
    return ok();
}

int lx2v_hip_weight_free(lx2v_hip_ctx *ctx, lx2v_hip_weight *w) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "weight_free")) return rc;
    if (!w) return ok();
    if (int rc = set_dev(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(weight_free)");
    free_weight(w);
    return ok();
}

int lx2v_hip_weight_info(const lx2v_hip_weight *w, lx2v_hip_weight_info_t *info) {
    NEED(w, "weight");
    NEED(info, "info");
    info->fmt = w->fmt;
    info->rows = w->rows;
    info->cols = w->cols;
    info->group = w->group;
    info->device_bytes = w->device_bytes;
    info->canonicalized = w->canonicalized;
    return ok();
}

int lx2v_hip_weight_dequantize(lx2v_hip_ctx *ctx, const lx2v_hip_weight *w, float *out, size_t len) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "weight_dequantize")) return rc;
    NEED(w, "weight");
    NEED(out, "out");
    size_t n = w->rows * w->cols;
    if (len != n) return fail(LX2V_ERR_BAD_SHAPE, "dequantize into %zu elements, weight has %zu", len, n);
    if (int rc = set_dev(ctx)) return rc;
    void *st;
    if (int rc = stage_for(ctx, n * 4, &st)) return rc;
    const uint8_t *fp8 = w->raw_e4m3 ? w->raw_e4m3 : (const uint8_t *)w->codes;
    if (int rc = run(ctx, "dequant", [&] { launch_dequant(ctx->stream, w, fp8, (float *)st); })) return rc;
    HIP_TRY(hipMemcpyAsync(out, st, n * 4, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync(dequant)");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(dequant)");
    return ok();
}

// ---- device quantizers -------------------------------------------------------------

static int quant_src_check(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows, size_t cols,
                           size_t group) {
    NEED(ctx, "ctx");
    NEED(src, "src");
    if (int rc = not_capturing(ctx, "quantize")) return rc;
    if (src->dtype != LX2V_DTYPE_F32) return fail(LX2V_ERR_BAD_ARG, "quantizer source must be an f32 buffer");
    if (int rc = check_quant_shape(rows, cols, group)) return rc;
    if (rows * cols > src->len)
        return fail(LX2V_ERR_BAD_SHAPE, "source has %zu elements, %zux%zu needs %zu", src->len, rows, cols,
                    rows * cols);
    return set_dev(ctx);
}

int lx2v_hip_quantize_q8(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows, size_t cols,
                         size_t group, lx2v_hip_weight **out) {
    NEED(out, "out");
    if (int rc = quant_src_check(ctx, src, rows, cols, group)) return rc;
    auto *w = new lx2v_hip_weight;
    w->fmt = LX2V_WFMT_Q8;
    w->rows = rows;
    w->cols = cols;
    w->group = group;
    size_t n = rows * cols, ns = n / group;
    hipError_t e = hipMalloc(&w->codes, n);
    if (e == hipSuccess) e = hipMalloc((void **)&w->scales, ns * 4);
    if (e != hipSuccess) {
        free_weight(w);
        return hip_fail(e, "quantize_q8 alloc");
    }
    w->device_bytes = n + ns * 4;
    int rc = run(ctx, "quantize_q8", [&] {
        launch_quantize_q8(ctx->stream, (const float *)src->ptr, rows, cols, group, (int8_t *)w->codes, w->scales);
    });
    if (rc) {
        free_weight(w);
        return rc;
    }
    if (int rc2 = stage_scales(ctx, w)) {
        free_weight(w);
        return rc2;
    }
    *out = w;
    return ok();
}

int lx2v_hip_quantize_q4_sym(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows, size_t cols,
                             size_t group, lx2v_hip_weight **out) {
    NEED(out, "out");
    if (int rc = quant_src_check(ctx, src, rows, cols, group)) return rc;
    if (group % 2) return fail(LX2V_ERR_BAD_SHAPE, "q4 group %zu must be even", group);
    auto *w = new lx2v_hip_weight;
    w->fmt = LX2V_WFMT_Q4;
    w->rows = rows;
    w->cols = cols;
    w->group = group;
    size_t n = rows * cols, ns = n / group;
    hipError_t e = hipMalloc(&w->codes, n / 2);
    if (e == hipSuccess) e = hipMalloc((void **)&w->scales, ns * 4);
    if (e == hipSuccess) e = hipMalloc((void **)&w->zeros, ns * 4);
    if (e != hipSuccess) {
        free_weight(w);
        return hip_fail(e, "quantize_q4 alloc");
    }
    w->device_bytes = n / 2 + 2 * ns * 4;
    int rc = run(ctx, "quantize_q4", [&] {
        launch_quantize_q4_sym(ctx->stream, (const float *)src->ptr, rows, cols, group, (uint8_t *)w->codes,
                               w->scales, w->zeros);
    });
    if (rc) {
        free_weight(w);
        return rc;
    }
    w->zero8 = true;  // k_quantize_q4_sym's zeros
    if (int rc2 = stage_scales(ctx, w)) {
        free_weight(w);
        return rc2;
    }
    *out = w;
    return ok();
}

int lx2v_hip_quantize_fp8(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows, size_t cols,
                          size_t group, lx2v_hip_weight **out) {
    NEED(out, "out");
    if (int rc = quant_src_check(ctx, src, rows, cols, group)) return rc;
    auto *w = new lx2v_hip_weight;
    w->fmt = LX2V_WFMT_FP8;
    w->rows = rows;
    w->cols = cols;
    w->group = group;
    size_t n = rows * cols, ns = n / group;
    hipError_t e = hipMalloc(&w->codes, n);
    if (e == hipSuccess) e = hipMalloc((void **)&w->scales, ns * 4);
    if (e != hipSuccess) {
        free_weight(w);
        return hip_fail(e, "quantize_fp8 alloc");
    }
    w->device_bytes = n + ns * 4;
    int rc = run(ctx, "quantize_fp8", [&] {
        launch_quantize_fp8(ctx->stream, (const float *)src->ptr, rows, cols, group, (uint8_t *)w->codes,
                            w->scales);
    });
    if (rc) {
        free_weight(w);
        return rc;
    }
    if (int rc2 = stage_scales(ctx, w)) {
        free_weight(w);
        return rc2;
    }
    *out = w;
    return ok();
}

int lx2v_hip_quantize_q4(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows, size_t cols, size_t group,
                         int hqq, lx2v_hip_weight **out) {
    NEED(out, "out");
    if (int rc = quant_src_check(ctx, src, rows, cols, group)) return rc;
    if (group % 2) return fail(LX2V_ERR_BAD_SHAPE, "q4 group %zu must be even (two codes per byte)", group);
    auto *w = new lx2v_hip_weight;
    w->fmt = LX2V_WFMT_Q4;
    w->rows = rows;
    w->cols = cols;
    w->group = group;
    size_t n = rows * cols, ns = n / group;
    hipError_t e = hipMalloc(&w->codes, n / 2);
    if (e == hipSuccess) e = hipMalloc((void **)&w->scales, ns * 4);
    if (e == hipSuccess) e = hipMalloc((void **)&w->zeros, ns * 4);
    if (e != hipSuccess) {
        free_weight(w);
        return hip_fail(e, "quantize_q4 alloc");
    }
    w->device_bytes = n / 2 + 2 * ns * 4;
    int rc = run(ctx, "quantize_q4_ref", [&] {
        launch_quantize_q4_ref(ctx->stream, (const float *)src->ptr, rows, cols, group, hqq ? 1 : 0,
                               (uint8_t *)w->codes, w->scales, w->zeros);
    });
    if (!rc) rc = stage_scales(ctx, w);
    if (rc) {
        free_weight(w);
        return rc;
    }
    *out = w;
    return ok();
}

int lx2v_hip_quantize_fp8_ref(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows, size_t cols, size_t group,
                              lx2v_hip_weight **out) {
    NEED(out, "out");
    if (int rc = quant_src_check(ctx, src, rows, cols, group)) return rc;
    auto *w = new lx2v_hip_weight;
    w->fmt = LX2V_WFMT_FP8;
    w->rows = rows;
    w->cols = cols;
    w->group = group;
    size_t n = rows * cols, ns = n / group;
    unsigned long long *count = nullptr;
    hipError_t e = hipMalloc(&w->codes, n);
    if (e == hipSuccess) e = hipMalloc((void **)&w->raw_e4m3, n);
    if (e == hipSuccess) e = hipMalloc((void **)&w->scales, ns * 4);
    if (e == hipSuccess) e = hipMalloc((void **)&count, sizeof(*count));
    if (e != hipSuccess) {
        if (count) (void)hipFree(count);
        free_weight(w);
        return hip_fail(e, "quantize_fp8_ref alloc");
    }
    w->device_bytes = n + ns * 4;
    // The reference's codes go to raw_e4m3 (what dequantize and export read);
    // the GEMMs read the canonical copy.
    unsigned long long changed = 0;
    int rc = run(ctx, "quantize_fp8_ref", [&] {
        (void)hipMemsetAsync(count, 0, sizeof(*count), ctx->stream);
        launch_quantize_fp8_ref(ctx->stream, (const float *)src->ptr, rows, cols, group, w->raw_e4m3, w->scales);
        launch_fp8_canon(ctx->stream, w->raw_e4m3, (uint8_t *)w->codes, n, count);
    });
    if (!rc) {
        hipError_t e2 = hipMemcpyAsync(&changed, count, sizeof(changed), hipMemcpyDeviceToHost, ctx->stream);
        if (e2 == hipSuccess) e2 = hipStreamSynchronize(ctx->stream);
        if (e2 != hipSuccess) rc = hip_fail(e2, "quantize_fp8_ref count");
    }
    (void)hipFree(count);
    if (!rc && !changed) {  // every code is already canonical: drop the copy
        (void)hipFree(w->raw_e4m3);
        w->raw_e4m3 = nullptr;
    }
    w->canonicalized = changed;
    if (!rc) rc = stage_scales(ctx, w);
    if (rc) {
        free_weight(w);
        return rc;
    }
    *out = w;
    return ok();
}

int lx2v_hip_weight_export(lx2v_hip_ctx *ctx, const lx2v_hip_weight *w, void *codes, size_t codes_bytes,
                           float *scales, float *zeros) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "weight_export")) return rc;
    NEED(w, "weight");
    NEED(codes, "codes");
    const size_t n = w->rows * w->cols;
    size_t cb = n;  // Q8, FP8: one byte per element
    if (w->fmt == LX2V_WFMT_F32) cb = n * 4;
    if (w->fmt == LX2V_WFMT_Q4) cb = (n + 1) / 2;
    if (codes_bytes != cb)
        return fail(LX2V_ERR_BAD_SHAPE, "export codes into %zu bytes, the weight has %zu", codes_bytes, cb);
    if (w->fmt != LX2V_WFMT_F32 && !scales) return fail(LX2V_ERR_BAD_ARG, "scales is null");
    if (w->fmt == LX2V_WFMT_Q4 && !zeros) return fail(LX2V_ERR_BAD_ARG, "zeros is null");
    if (int rc = set_dev(ctx)) return rc;
    const void *src = w->fmt == LX2V_WFMT_FP8 && w->raw_e4m3 ? (const void *)w->raw_e4m3 : w->codes;
    HIP_TRY(hipMemcpyAsync(codes, src, cb, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync(export codes)");
    if (w->fmt != LX2V_WFMT_F32) {
        const size_t ns = n / w->group;
        HIP_TRY(hipMemcpyAsync(scales, w->scales, ns * 4, hipMemcpyDeviceToHost, ctx->stream),
                "hipMemcpyAsync(export scales)");
        if (w->fmt == LX2V_WFMT_Q4)
            HIP_TRY(hipMemcpyAsync(zeros, w->zeros, ns * 4, hipMemcpyDeviceToHost, ctx->stream),
                    "hipMemcpyAsync(export zeros)");
    }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(export)");
    return ok();
}

// ---- norms and residuals around the linears --------------------------------------

// `dim` f32 values of parameter buffer b from element off: an F32 buffer in
// place, a BF16 one converted into staging slot `slot` (3 slots of dim).
static int param_f32(lx2v_hip_ctx *ctx, const lx2v_hip_buf *b, size_t off, size_t dim, int slot, const float **out,
                     const char *what) {
    if (!b) return fail(LX2V_ERR_BAD_ARG, "%s: buffer is null", what);
    if (b->quantized()) return fail(LX2V_ERR_BAD_ARG, "%s: an F32 or BF16 buffer is needed", what);
    if (off + dim < off || off + dim > b->len)
        return fail(LX2V_ERR_BAD_SHAPE, "%s: elements [%zu, +%zu) of a buffer of %zu", what, off, dim, b->len);
    if (b->dtype == LX2V_DTYPE_F32) {
        *out = (const float *)b->ptr + off;
        return LX2V_OK;
    }
    void *st;
    if (int rc = stage_for(ctx, 3 * dim * 4, &st)) return rc;
    float *dst = (float *)st + (size_t)slot * dim;
    if (int rc = run(ctx, "convert", [&] {
            launch_convert(ctx->stream, (const uint16_t *)b->ptr + off, LX2V_DTYPE_BF16, dst, LX2V_DTYPE_F32, dim);
        }))
        return rc;
    *out = dst;
    return LX2V_OK;
}

// Shared body of layer_norm / residual_norm: x (h), a (null for layer_norm).
static int norm_common(lx2v_hip_ctx *ctx, lx2v_hip_buf *x, const lx2v_hip_buf *a, size_t rows, size_t dim,
                       const lx2v_hip_buf *mods, const size_t *gate, const lx2v_hip_norm_t *norm, float eps,
                       lx2v_hip_buf *out, const char *what) {
    NEED(ctx, "ctx");
    NEED(x, "x");
    NEED(norm, "norm");
    NEED(out, "out");
    if (x->quantized() || (a && a->quantized()))
        return fail(LX2V_ERR_BAD_ARG, "%s reads F32 or BF16 activations", what);
    if (a && a->dtype != x->dtype) return fail(LX2V_ERR_BAD_ARG, "%s: h and a differ in dtype", what);
    if (dim && rows > x->len / dim) return fail(LX2V_ERR_BAD_SHAPE, "%s: %zux%zu rows, buffer has %zu", what, rows, dim, x->len);
    if (a && dim && rows > a->len / dim) return fail(LX2V_ERR_BAD_SHAPE, "%s: a has %zu elements", what, a->len);
    if (norm->kind != LX2V_NORM_AFFINE && norm->kind != LX2V_NORM_MOD)
        return fail(LX2V_ERR_BAD_ARG, "%s: unknown norm kind %d", what, norm->kind);
    const bool q = out->dtype == LX2V_DTYPE_E4M3 || out->dtype == LX2V_DTYPE_MXE4M3;
    if (q) {
        if (out->cols != dim || rows > out->rows)
            return fail(LX2V_ERR_BAD_SHAPE, "%s: %zux%zu into a quantized buffer of %zux%zu", what, rows, dim, out->rows,
                        out->cols);
    } else if (dim && rows > out->len / dim) {
        return fail(LX2V_ERR_BAD_SHAPE, "%s: out has %zu elements, %zux%zu needed", what, out->len, rows, dim);
    }
    const size_t n = rows * dim;
    if (overlap(out->ptr, std::max<size_t>(out->bytes(), 1), x->ptr, n * x->elem_bytes()) ||
        (a && overlap(out->ptr, std::max<size_t>(out->bytes(), 1), a->ptr, n * a->elem_bytes())) ||
        (mods && overlap(out->ptr, std::max<size_t>(out->bytes(), 1), mods->ptr, mods->bytes())))
        return fail(LX2V_ERR_ALIAS, "%s: out overlaps an input", what);
    if (a && overlap(x->ptr, n * x->elem_bytes(), a->ptr, n * a->elem_bytes()))
        return fail(LX2V_ERR_ALIAS, "%s: h overlaps a", what);
    if (!n) return ok();
    if (int rc = set_dev(ctx)) return rc;
    const float *g = nullptr, *pm = nullptr, *pa = nullptr;
    if (gate) {
        if (int rc = param_f32(ctx, mods, *gate * dim, dim, 0, &g, "mods (gate)")) return rc;
    }
    if (norm->kind == LX2V_NORM_MOD) {
        if (int rc = param_f32(ctx, mods, norm->scale * dim, dim, 1, &pm, "mods (scale)")) return rc;
        if (int rc = param_f32(ctx, mods, norm->shift * dim, dim, 2, &pa, "mods (shift)")) return rc;
    } else {
        if (int rc = param_f32(ctx, norm->w, 0, dim, 1, &pm, "norm w")) return rc;
        if (int rc = param_f32(ctx, norm->b, 0, dim, 2, &pa, "norm b")) return rc;
    }
    return run(ctx, a ? "residual_norm" : "layer_norm", [&] {
        launch_norm(ctx->stream, x->ptr, a ? a->ptr : nullptr, x->dtype, g, pm, pa, norm->kind == LX2V_NORM_MOD, eps,
                    rows, dim, out->ptr, out->dtype, out->dtype == LX2V_DTYPE_E4M3 ? out->scales : nullptr,
                    out->dtype == LX2V_DTYPE_MXE4M3 ? out->mxs : nullptr, out->srows);
    });
}

int lx2v_hip_layer_norm(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t rows, size_t dim,
                        const lx2v_hip_norm_t *norm, const lx2v_hip_buf *mods, float eps, lx2v_hip_buf *out) {
    return norm_common(ctx, const_cast<lx2v_hip_buf *>(x), nullptr, rows, dim, mods, nullptr, norm, eps, out,
                       "layer_norm");
}

int lx2v_hip_residual_norm(lx2v_hip_ctx *ctx, lx2v_hip_buf *h, const lx2v_hip_buf *a, size_t rows, size_t dim,
                           const lx2v_hip_buf *mods, int has_gate, size_t gate, const lx2v_hip_norm_t *norm, float eps,
                           lx2v_hip_buf *normed) {
    NEED(a, "a");
    return norm_common(ctx, h, a, rows, dim, mods, has_gate ? &gate : nullptr, norm, eps, normed, "residual_norm");
}

int lx2v_hip_gate_residual(lx2v_hip_ctx *ctx, lx2v_hip_buf *h, const lx2v_hip_buf *a, size_t rows, size_t dim,
                           const lx2v_hip_buf *mods, size_t gate) {
    NEED(ctx, "ctx");
    NEED(h, "h");
    NEED(a, "a");
    if (h->quantized() || a->quantized() || h->dtype != a->dtype)
        return fail(LX2V_ERR_BAD_ARG, "gate_residual reads h and a of one F32 or BF16 dtype");
    if (dim && (rows > h->len / dim || rows > a->len / dim))
        return fail(LX2V_ERR_BAD_SHAPE, "gate_residual: %zux%zu, h has %zu, a %zu elements", rows, dim, h->len, a->len);
    const size_t n = rows * dim;
    if (overlap(h->ptr, n * h->elem_bytes(), a->ptr, n * a->elem_bytes()))
        return fail(LX2V_ERR_ALIAS, "gate_residual: h overlaps a");
    if (!n) return ok();
    if (int rc = set_dev(ctx)) return rc;
    const float *g = nullptr;
    if (int rc = param_f32(ctx, mods, gate * dim, dim, 0, &g, "mods (gate)")) return rc;
    return run(ctx, "gate_residual",
               [&] { launch_gate_residual(ctx->stream, h->ptr, a->ptr, h->dtype, g, rows, dim); });
}

// Backend::head_split (backend.rs:255-273).
int lx2v_hip_head_split(lx2v_hip_ctx *ctx, const lx2v_hip_buf *src, size_t rows, size_t src_stride, size_t col_off,
                        size_t heads, size_t head_dim, const lx2v_hip_buf *rms_w, const lx2v_hip_buf *rope_cos,
                        const lx2v_hip_buf *rope_sin, float eps, lx2v_hip_buf *out) {
    NEED(ctx, "ctx");
    NEED(src, "src");
    NEED(out, "out");
    if (src->quantized() || out->quantized() || (rms_w && rms_w->quantized()) ||
        (rope_cos && rope_cos->quantized()) || (rope_sin && rope_sin->quantized()))
        return fail(LX2V_ERR_BAD_ARG, "head_split: F32 or BF16 buffers only");
    if (!rope_cos != !rope_sin) return fail(LX2V_ERR_BAD_ARG, "head_split: rope_cos and rope_sin go together");
    const size_t d = heads * head_dim;
    if (!rows || !d) return ok();
    if (col_off + d < col_off || col_off + d > src_stride)
        return fail(LX2V_ERR_BAD_SHAPE, "head_split: columns [%zu, +%zu) outside a row of %zu", col_off, d, src_stride);
    if ((rows - 1) * src_stride + col_off + d > src->len)
        return fail(LX2V_ERR_BAD_SHAPE, "head_split: src has %zu elements, %zu rows of stride %zu need %zu", src->len,
                    rows, src_stride, (rows - 1) * src_stride + col_off + d);
    if (rows * d > out->len)
        return fail(LX2V_ERR_BAD_SHAPE, "head_split: out has %zu elements, needs %zu", out->len, rows * d);
    if (rms_w && rms_w->len < d)
        return fail(LX2V_ERR_BAD_SHAPE, "head_split: rms_w has %zu elements, needs %zu", rms_w->len, d);
    if (rope_cos && (rope_cos->len < rows * (head_dim / 2) || rope_sin->len < rows * (head_dim / 2)))
        return fail(LX2V_ERR_BAD_SHAPE, "head_split: rope tables need %zu elements each", rows * (head_dim / 2));
    if (overlap(out->ptr, rows * d * out->elem_bytes(), src->ptr, src->bytes()))
        return fail(LX2V_ERR_ALIAS, "head_split: out overlaps src");
    for (const lx2v_hip_buf *b : {rms_w, rope_cos, rope_sin})
        if (b && overlap(out->ptr, rows * d * out->elem_bytes(), b->ptr, b->bytes()))
            return fail(LX2V_ERR_ALIAS, "head_split: out overlaps a parameter");
    if (int rc = set_dev(ctx)) return rc;
    return run(ctx, "head_split", [&] {
        launch_head_split(ctx->stream, src->ptr, src->dtype, rows, src_stride, col_off, heads, head_dim,
                          rms_w ? rms_w->ptr : nullptr, rms_w ? rms_w->dtype : LX2V_DTYPE_F32,
                          rope_cos ? rope_cos->ptr : nullptr, rope_sin ? rope_sin->ptr : nullptr,
                          rope_cos ? rope_cos->dtype : LX2V_DTYPE_F32, eps, out->ptr, out->dtype);
    });
}

// ---- attention ------------------------------------------------------------------

struct lx2v_hip_mask {
    uint8_t *bytes = nullptr;  // [sq, sk], then the bits, then the tile summary
    uint32_t *bits = nullptr;
    uint8_t *tiles = nullptr;
    size_t sq = 0, sk = 0;
};

static int attn_check(lx2v_hip_ctx *ctx, const lx2v_hip_buf *q, const lx2v_hip_buf *k, const lx2v_hip_buf *v,
                      size_t heads, size_t sq, size_t sk, size_t d, const lx2v_hip_buf *out) {
    NEED(ctx, "ctx");
    NEED(q, "q");
    NEED(k, "k");
    NEED(v, "v");
    NEED(out, "out");
    if (q->quantized() || k->quantized() || v->quantized() || out->dtype == LX2V_DTYPE_E4M3)
        return fail(LX2V_ERR_BAD_ARG, "attention reads F32 or BF16 buffers and writes F32, BF16 or MXE4M3 ones");
    if (out->dtype == LX2V_DTYPE_MXE4M3 && (!attention_mfma_supported(d) || out->cols != heads * d || out->rows < sq))
        return fail(LX2V_ERR_BAD_SHAPE,
                    "attention: MXE4M3 output needs head_dim 64 or 128 and a [>= sq, heads * head_dim] buffer "
                    "(head_dim %zu; buffer %zu x %zu; sq %zu, %zu heads)",
                    d, out->rows, out->cols, sq, heads);
    if (q->dtype != k->dtype || q->dtype != v->dtype) return fail(LX2V_ERR_BAD_ARG, "attention: q, k, v differ in dtype");
    if (d == 0 || d > 256) return fail(LX2V_ERR_UNSUPPORTED, "attention: head_dim %zu (1..256)", d);
    if (sq >= (1u << 30) || sk >= (1u << 30) || heads >= (1u << 16))
        return fail(LX2V_ERR_BAD_SHAPE, "attention: %zu heads, sq %zu, sk %zu too large", heads, sq, sk);
    if (sk * d * k->elem_bytes() >= (1ull << 31) || sq * ((sk + 31) / 32) * 4 >= (1ull << 31))
        return fail(LX2V_ERR_BAD_SHAPE, "attention: one head's keys or the mask bits pass 2 GiB (sk %zu)", sk);
    const size_t nq = heads * sq * d, nk = heads * sk * d;
    if (q->len < nq || k->len < nk || v->len < nk || out->len < nq)
        return fail(LX2V_ERR_BAD_SHAPE, "attention: q %zu / k %zu / v %zu / out %zu elements, need %zu, %zu, %zu, %zu",
                    q->len, k->len, v->len, out->len, nq, nk, nk, nq);
    const size_t ob = nq * out->elem_bytes();
    if (overlap(out->ptr, ob, q->ptr, nq * q->elem_bytes()) || overlap(out->ptr, ob, k->ptr, nk * k->elem_bytes()) ||
        overlap(out->ptr, ob, v->ptr, nk * v->elem_bytes()))
        return fail(LX2V_ERR_ALIAS, "attention: out overlaps q, k or v");
    return set_dev(ctx);
}

// The split mode's piece count and partial-sum workspace for this call
// (1 and null where the one-pass kernel runs).
static int attn_part(lx2v_hip_ctx *ctx, size_t heads, size_t sq, size_t sk, size_t d, float **part, int *nsplit) {
    *part = nullptr;
    size_t need = 0;
    *nsplit = attention_split(heads, sq, sk, d, ctx->num_cu, &need);
    if (*nsplit <= 1) return LX2V_OK;
    if (int rc = ensure(ctx, &ctx->attn.ptr, &ctx->attn.bytes, need, "attention workspace alloc")) return rc;
    *part = (float *)ctx->attn.ptr;
    return LX2V_OK;
}

static int attn_run(lx2v_hip_ctx *ctx, const lx2v_hip_buf *q, const lx2v_hip_buf *k, const lx2v_hip_buf *v,
                    size_t heads, size_t sq, size_t sk, size_t d, const lx2v_hip_mask *mask, lx2v_hip_buf *out) {
    if (!heads || !sq) return ok();
    float *part = nullptr;
    int nsplit = 1;
    if (int rc = attn_part(ctx, heads, sq, sk, d, &part, &nsplit)) return rc;
    return run(ctx, mask ? "causal_attention" : "attention", [&] {
        launch_attention(ctx->stream, q->ptr, k->ptr, v->ptr, q->dtype, heads, sq, sk, sk, d,
                         mask ? mask->bytes : nullptr, mask ? mask->bits : nullptr, mask ? mask->tiles : nullptr,
                         out->ptr, out->dtype, out->mxs, out->srows, part, nsplit);
    });
}

int lx2v_hip_attention(lx2v_hip_ctx *ctx, const lx2v_hip_buf *q, const lx2v_hip_buf *k, const lx2v_hip_buf *v,
                       size_t heads, size_t sq, size_t sk, size_t head_dim, lx2v_hip_buf *out) {
    if (int rc = attn_check(ctx, q, k, v, heads, sq, sk, head_dim, out)) return rc;
    return attn_run(ctx, q, k, v, heads, sq, sk, head_dim, nullptr, out);
}

// The mask bytes, bits and tile summary in device memory at `base` (mask_bytes).
static size_t mask_bytes(size_t sq, size_t sk) {
    return ((sq * sk + 255) & ~(size_t)255) + mask_word_count(sq, sk) * 4 + mask_tile_count(sq, sk);
}

static int mask_fill(lx2v_hip_ctx *ctx, const uint8_t *host, size_t sq, size_t sk, uint8_t *base, lx2v_hip_mask *m) {
    const size_t nb = sq * sk;
    m->bytes = base;
    m->bits = (uint32_t *)(base + ((nb + 255) & ~(size_t)255));
    m->tiles = (uint8_t *)(m->bits + mask_word_count(sq, sk));
    m->sq = sq;
    m->sk = sk;
    HIP_TRY(hipMemcpyAsync(base, host, nb, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync(mask)");
    return run(ctx, "mask_tiles", [&] {
        launch_mask_pack(ctx->stream, base, sq, sk, m->bits);
        launch_mask_tiles_bits(ctx->stream, m->bits, sq, sk, m->tiles);
    });
}

int lx2v_hip_causal_attention(lx2v_hip_ctx *ctx, const lx2v_hip_buf *q, const lx2v_hip_buf *k, const lx2v_hip_buf *v,
                              size_t heads, size_t sq, size_t sk, size_t head_dim, const uint8_t *mask,
                              lx2v_hip_buf *out) {
    if (!mask) return lx2v_hip_attention(ctx, q, k, v, heads, sq, sk, head_dim, out);
    if (int rc = attn_check(ctx, q, k, v, heads, sq, sk, head_dim, out)) return rc;
    if (int rc = not_capturing(ctx, "causal_attention with a host mask")) return rc;
    if (!heads || !sq || !sk) return attn_run(ctx, q, k, v, heads, sq, sk, head_dim, nullptr, out);  // sk = 0: zeros
    auto &mb = ctx->mask;
    if (int rc = ensure(ctx, &mb.ptr, &mb.bytes, mask_bytes(sq, sk), "mask alloc")) return rc;
    lx2v_hip_mask m;
    if (int rc = mask_fill(ctx, mask, sq, sk, (uint8_t *)mb.ptr, &m)) return rc;
    if (int rc = attn_run(ctx, q, k, v, heads, sq, sk, head_dim, &m, out)) return rc;
    // the host mask is the caller's again when the call returns
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(causal_attention)");
    return ok();
}

int lx2v_hip_mask_upload(lx2v_hip_ctx *ctx, const uint8_t *mask, size_t sq, size_t sk, lx2v_hip_mask **out) {
    NEED(ctx, "ctx");
    NEED(out, "out");
    if (sq * sk) NEED(mask, "mask");
    if (int rc = not_capturing(ctx, "mask_upload")) return rc;
    if (sq >= (1u << 30) || sk >= (1u << 30)) return fail(LX2V_ERR_BAD_SHAPE, "mask %zux%zu too large", sq, sk);
    if (int rc = set_dev(ctx)) return rc;
    auto *m = new lx2v_hip_mask;
    m->sq = sq;
    m->sk = sk;
    uint8_t *base = nullptr;
    hipError_t e = hipMalloc((void **)&base, std::max<size_t>(mask_bytes(sq, sk), 4));
    if (e != hipSuccess) {
        delete m;
        return hip_fail(e, "hipMalloc(mask)");
    }
    m->bytes = base;
    int rc = sq * sk ? mask_fill(ctx, mask, sq, sk, base, m) : LX2V_OK;
    if (!rc) {
        hipError_t e2 = hipStreamSynchronize(ctx->stream);
        if (e2 != hipSuccess) rc = hip_fail(e2, "mask_upload");
    }
    if (rc) {
        (void)hipFree(m->bytes);
        delete m;
        return rc;
    }
    *out = m;
    return ok();
}

int lx2v_hip_mask_temporal(lx2v_hip_ctx *ctx, const size_t *tq, size_t sq, const size_t *tk, size_t sk,
                           lx2v_hip_mask **out) {
    NEED(ctx, "ctx");
    NEED(out, "out");
    if (sq) NEED(tq, "tq");
    if (sk) NEED(tk, "tk");
    if (int rc = not_capturing(ctx, "mask_temporal")) return rc;
    if (sq >= (1u << 30) || sk >= (1u << 30) || sq * sk >= (1ull << 40))
        return fail(LX2V_ERR_BAD_SHAPE, "mask %zux%zu too large", sq, sk);
    if (int rc = set_dev(ctx)) return rc;
    auto *m = new lx2v_hip_mask;
    m->sq = sq;
    m->sk = sk;
    // [bytes | bits | tiles] as mask_fill lays them out, then tq and tk
    const size_t nb = sq * sk, body = mask_bytes(sq, sk), toff = (body + 255) & ~(size_t)255;
    uint8_t *base = nullptr;
    hipError_t e = hipMalloc((void **)&base, std::max<size_t>(toff + (sq + sk) * 8, 4));
    if (e != hipSuccess) {
        delete m;
        return hip_fail(e, "hipMalloc(mask)");
    }
    m->bytes = base;
    m->bits = (uint32_t *)(base + ((nb + 255) & ~(size_t)255));
    m->tiles = (uint8_t *)(m->bits + mask_word_count(sq, sk));
    uint64_t *dq = (uint64_t *)(base + toff), *dk = dq + sq;
    int rc = LX2V_OK;
    static_assert(sizeof(size_t) == sizeof(uint64_t), "temporal indices are 64-bit");
    if (sq) e = hipMemcpyAsync(dq, tq, sq * 8, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess && sk) e = hipMemcpyAsync(dk, tk, sk * 8, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) rc = hip_fail(e, "mask_temporal upload");
    if (!rc)
        rc = run(ctx, "mask_temporal", [&] {
            launch_mask_temporal(ctx->stream, dq, sq, dk, sk, m->bytes, m->bits, m->tiles);
        });
    if (!rc) {
        hipError_t e2 = hipStreamSynchronize(ctx->stream);  // tq / tk are the caller's again
        if (e2 != hipSuccess) rc = hip_fail(e2, "mask_temporal");
    }
    if (rc) {
        (void)hipFree(base);
        delete m;
        return rc;
    }
    *out = m;
    return ok();
}

int lx2v_hip_mask_free(lx2v_hip_ctx *ctx, lx2v_hip_mask *m) {
    NEED(ctx, "ctx");
    if (!m) return ok();
    if (int rc = not_capturing(ctx, "mask_free")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(mask_free)");
    (void)hipFree(m->bytes);
    delete m;
    return ok();
}

int lx2v_hip_attention_masked(lx2v_hip_ctx *ctx, const lx2v_hip_buf *q, const lx2v_hip_buf *k, const lx2v_hip_buf *v,
                              size_t heads, size_t sq, size_t sk, size_t head_dim, const lx2v_hip_mask *mask,
                              lx2v_hip_buf *out) {
    if (int rc = attn_check(ctx, q, k, v, heads, sq, sk, head_dim, out)) return rc;
    if (mask && (mask->sq != sq || mask->sk != sk))
        return fail(LX2V_ERR_BAD_SHAPE, "attention: mask is %zux%zu, scores are %zux%zu", mask->sq, mask->sk, sq, sk);
    return attn_run(ctx, q, k, v, heads, sq, sk, head_dim, mask && sq * sk ? mask : nullptr, out);
}

// ---- KV cache / MemRoPE (backend.rs:333-392) ------------------------------------
//
// Device: K and V as [heads, cap, d] in one allocation (K first), the
// context's activation dtype at creation.  Host: the temporal index and slot
// kind of every row, as the reference's KvCache (crates/lightx2v-cpu/src/
// lib.rs:126-146); every append / overwrite / evict decision is made on them.

struct lx2v_hip_kv {
    size_t heads = 0, d = 0, cap = 0;
    int dtype = LX2V_DTYPE_F32;
    void *buf = nullptr;  // [2][heads][cap][d]
    size_t bytes = 0;
    std::vector<size_t> temporal;
    std::vector<uint8_t> kinds;
    // the MemRoPE plan: pinned host staging, its device copy, and the event
    // after which the staging may be rewritten
    int *plan_host = nullptr, *plan_dev = nullptr;
    size_t plan_cap = 0;
    hipEvent_t plan_done = nullptr;
    size_t eb() const { return dtype == LX2V_DTYPE_BF16 ? 2 : 4; }
    void *k() const { return buf; }
    void *v() const { return (uint8_t *)buf + heads * cap * d * eb(); }
    size_t rows() const { return temporal.size(); }
};

namespace {

size_t kv_cap_of(const lx2v_hip_kv *kv, size_t bytes) { return bytes / (2 * kv->heads * kv->d * kv->eb()); }

// Reallocate for at least `need` rows per head, keeping the live rows.
int kv_grow(lx2v_hip_ctx *ctx, lx2v_hip_kv *kv, size_t need) {
    if (need <= kv->cap) return LX2V_OK;
    if (int rc = not_capturing(ctx, "kv_cache growth")) return rc;
    const size_t cap = std::max(need, kv->cap + kv->cap / 2), bytes = 2 * kv->heads * cap * kv->d * kv->eb();
    void *nb = nullptr;
    HIP_TRY(hipMalloc(&nb, bytes), "hipMalloc(kv_cache)");
    if (kv->buf && kv->rows()) {
        const size_t w = kv->rows() * kv->d * kv->eb();
        hipError_t e = hipMemcpy2DAsync(nb, cap * kv->d * kv->eb(), kv->buf, kv->cap * kv->d * kv->eb(), w,
                                        2 * kv->heads, hipMemcpyDeviceToDevice, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            (void)hipFree(nb);
            return hip_fail(e, "kv_cache growth copy");
        }
    } else if (kv->buf) {
        HIP_TRY(hipStreamSynchronize(ctx->stream), "kv_cache growth");
    }
    if (kv->buf) (void)hipFree(kv->buf);
    kv->buf = nb;
    kv->bytes = bytes;
    kv->cap = cap;
    return LX2V_OK;
}

int kv_src_check(const lx2v_hip_kv *kv, const lx2v_hip_buf *k, const lx2v_hip_buf *v, size_t rows,
                 const size_t *temporal) {
    NEED(k, "k");
    NEED(v, "v");
    if (rows) NEED(temporal, "temporal");
    if (!valid_dtype(k->dtype) || !valid_dtype(v->dtype))
        return fail(LX2V_ERR_BAD_ARG, "kv_cache: k and v are F32 or BF16 buffers");
    const size_t n = kv->heads * rows * kv->d;
    if (k->len < n || v->len < n)
        return fail(LX2V_ERR_BAD_SHAPE, "kv_cache: k %zu / v %zu elements, [%zu heads, %zu rows, %zu] needs %zu",
                    k->len, v->len, kv->heads, rows, kv->d, n);
    if ((kv->rows() + rows) * kv->d >= (1u << 31))
        return fail(LX2V_ERR_BAD_SHAPE, "kv_cache: %zu + %zu rows of %zu pass 2^31 elements per head", kv->rows(), rows,
                    kv->d);
    return LX2V_OK;
}

// k, v [heads, rows, d] into cache rows [row0, row0 + rows).
int kv_write_rows(lx2v_hip_ctx *ctx, lx2v_hip_kv *kv, const lx2v_hip_buf *k, const lx2v_hip_buf *v, size_t rows,
                  size_t row0) {
    return run(ctx, "kv_cache_put", [&] {
        launch_kv_copy(ctx->stream, k->ptr, k->dtype, rows, 0, kv->k(), kv->dtype, kv->cap, row0, kv->heads, rows,
                       kv->d);
        launch_kv_copy(ctx->stream, v->ptr, v->dtype, rows, 0, kv->v(), kv->dtype, kv->cap, row0, kv->heads, rows,
                       kv->d);
    });
}

int kv_append(lx2v_hip_ctx *ctx, lx2v_hip_kv *kv, const lx2v_hip_buf *k, const lx2v_hip_buf *v, size_t rows,
              const size_t *temporal) {
    const size_t at = kv->rows();
    if (int rc = kv_grow(ctx, kv, at + rows)) return rc;
    if (int rc = kv_write_rows(ctx, kv, k, v, rows, at)) return rc;
    kv->temporal.insert(kv->temporal.end(), temporal, temporal + rows);
    kv->kinds.insert(kv->kinds.end(), rows, (uint8_t)LX2V_SLOT_NEW);  // lib.rs:640-642
    return LX2V_OK;
}

}  // namespace

int lx2v_hip_kv_cache_new(lx2v_hip_ctx *ctx, size_t heads, size_t head_dim, size_t capacity_tokens,
                          lx2v_hip_kv **out) {
    NEED(ctx, "ctx");
    NEED(out, "out");
    if (int rc = not_capturing(ctx, "kv_cache_new")) return rc;
    if (!heads || !head_dim || heads >= (1u << 16) || head_dim > 256)
        return fail(LX2V_ERR_BAD_SHAPE, "kv_cache_new: %zu heads of %zu (1..256)", heads, head_dim);
    if (capacity_tokens * head_dim >= (1u << 31))
        return fail(LX2V_ERR_BAD_SHAPE, "kv_cache_new: capacity %zu", capacity_tokens);
    if (int rc = set_dev(ctx)) return rc;
    auto *kv = new lx2v_hip_kv;
    kv->heads = heads;
    kv->d = head_dim;
    kv->dtype = ctx->act_dtype;
    hipError_t e = hipEventCreateWithFlags(&kv->plan_done, hipEventDisableTiming);
    int rc = e == hipSuccess ? kv_grow(ctx, kv, std::max<size_t>(capacity_tokens, 1)) : hip_fail(e, "kv_cache_new");
    if (rc) {
        if (kv->plan_done) (void)hipEventDestroy(kv->plan_done);
        delete kv;
        return rc;
    }
    *out = kv;
    return ok();
}

int lx2v_hip_kv_cache_free(lx2v_hip_ctx *ctx, lx2v_hip_kv *kv) {
    NEED(ctx, "ctx");
    if (!kv) return ok();
    if (int rc = not_capturing(ctx, "kv_cache_free")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(kv_cache_free)");
    if (kv->buf) (void)hipFree(kv->buf);
    if (kv->plan_dev) (void)hipFree(kv->plan_dev);
    if (kv->plan_host) (void)hipHostFree(kv->plan_host);
    (void)hipEventDestroy(kv->plan_done);
    delete kv;
    return ok();
}

int lx2v_hip_kv_cache_append(lx2v_hip_ctx *ctx, lx2v_hip_kv *kv, const lx2v_hip_buf *k, const lx2v_hip_buf *v,
                             size_t rows, const size_t *temporal) {
    NEED(ctx, "ctx");
    NEED(kv, "cache");
    if (int rc = kv_src_check(kv, k, v, rows, temporal)) return rc;
    if (int rc = set_dev(ctx)) return rc;
    if (int rc = kv_append(ctx, kv, k, v, rows, temporal)) return rc;
    return ok();
}

int lx2v_hip_kv_cache_put(lx2v_hip_ctx *ctx, lx2v_hip_kv *kv, const lx2v_hip_buf *k, const lx2v_hip_buf *v,
                          size_t rows, const size_t *temporal) {
    NEED(ctx, "ctx");
    NEED(kv, "cache");
    if (int rc = kv_src_check(kv, k, v, rows, temporal)) return rc;
    if (int rc = set_dev(ctx)) return rc;
    if (rows) {
        // lib.rs:647-678: the first non-EMA row with temporal[0]; overwrite
        // when the next `rows` rows carry exactly `temporal`.
        const auto &T = kv->temporal;
        for (size_t pos = 0; pos < T.size(); pos++) {
            if (T[pos] != temporal[0] || kv->kinds[pos] == LX2V_SLOT_LONG_EMA || kv->kinds[pos] == LX2V_SLOT_SHORT_EMA)
                continue;
            bool same = pos + rows <= T.size();
            for (size_t i = 0; same && i < rows; i++) same = T[pos + i] == temporal[i];
            if (!same) break;
            if (int rc = kv_write_rows(ctx, kv, k, v, rows, pos)) return rc;
            return ok();
        }
    }
    if (int rc = kv_append(ctx, kv, k, v, rows, temporal)) return rc;
    return ok();
}

int lx2v_hip_kv_cache_len(const lx2v_hip_kv *kv, size_t *rows) {
    NEED(kv, "cache");
    NEED(rows, "rows");
    *rows = kv->rows();
    return ok();
}

int lx2v_hip_kv_cache_temporal(const lx2v_hip_kv *kv, size_t *out, size_t cap) {
    NEED(kv, "cache");
    if (cap < kv->rows()) return fail(LX2V_ERR_BAD_SHAPE, "kv_cache_temporal: room for %zu of %zu rows", cap, kv->rows());
    if (kv->rows()) NEED(out, "out");
    std::copy(kv->temporal.begin(), kv->temporal.end(), out);
    return ok();
}

int lx2v_hip_kv_cache_kinds(const lx2v_hip_kv *kv, uint8_t *out, size_t cap) {
    NEED(kv, "cache");
    if (cap < kv->rows()) return fail(LX2V_ERR_BAD_SHAPE, "kv_cache_kinds: room for %zu of %zu rows", cap, kv->rows());
    if (kv->rows()) NEED(out, "out");
    std::copy(kv->kinds.begin(), kv->kinds.end(), out);
    return ok();
}

int lx2v_hip_kv_cache_read(lx2v_hip_ctx *ctx, const lx2v_hip_kv *kv, lx2v_hip_buf *k, lx2v_hip_buf *v) {
    NEED(ctx, "ctx");
    NEED(kv, "cache");
    NEED(k, "k");
    NEED(v, "v");
    const size_t rows = kv->rows(), n = kv->heads * rows * kv->d;
    if (!valid_dtype(k->dtype) || !valid_dtype(v->dtype))
        return fail(LX2V_ERR_BAD_ARG, "kv_cache_kv: k and v are F32 or BF16 buffers");
    if (k->len < n || v->len < n)
        return fail(LX2V_ERR_BAD_SHAPE, "kv_cache_kv: k %zu / v %zu elements, the cache holds %zu", k->len, v->len, n);
    if (k->ptr == v->ptr && n) return fail(LX2V_ERR_ALIAS, "kv_cache_kv: k and v are one buffer");
    if (int rc = set_dev(ctx)) return rc;
    return run(ctx, "kv_cache_kv", [&] {
        launch_kv_copy(ctx->stream, kv->k(), kv->dtype, kv->cap, 0, k->ptr, k->dtype, rows, 0, kv->heads, rows, kv->d);
        launch_kv_copy(ctx->stream, kv->v(), kv->dtype, kv->cap, 0, v->ptr, v->dtype, rows, 0, kv->heads, rows, kv->d);
    });
}

int lx2v_hip_kv_cache_kv(lx2v_hip_ctx *ctx, const lx2v_hip_kv *kv, lx2v_hip_buf **k, lx2v_hip_buf **v) {
    NEED(ctx, "ctx");
    NEED(kv, "cache");
    NEED(k, "k");
    NEED(v, "v");
    if (int rc = not_capturing(ctx, "kv_cache_kv")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    const size_t n = kv->heads * kv->rows() * kv->d;
    lx2v_hip_buf *kb = nullptr, *vb = nullptr;
    if (int rc = alloc_buf(ctx, n, kv->dtype, &kb)) return rc;
    int rc = alloc_buf(ctx, n, kv->dtype, &vb);
    if (!rc) rc = lx2v_hip_kv_cache_read(ctx, kv, kb, vb);
    if (rc) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(kb->ptr);
        delete kb;
        if (vb) {
            (void)hipFree(vb->ptr);
            delete vb;
        }
        return rc;
    }
    *k = kb;
    *v = vb;
    return ok();
}

int lx2v_hip_kv_cache_memrope_update(lx2v_hip_ctx *ctx, lx2v_hip_kv *kv, const lx2v_hip_memrope_t *cfg,
                                     size_t frame_tokens) {
    NEED(ctx, "ctx");
    NEED(kv, "cache");
    NEED(cfg, "cfg");
    if (!frame_tokens || frame_tokens >= (1u << 24))
        return fail(LX2V_ERR_BAD_SHAPE, "memrope_update: frame_tokens %zu", frame_tokens);
    if (int rc = not_capturing(ctx, "kv_cache_memrope_update")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    const size_t ft = frame_tokens;
    // Simulate lib.rs:707-806 on the row metadata, carrying each row's source:
    // an old row (>= 0), zeros (-1), or EMA slot s's output row o (-2 - (s ft + o)).
    std::vector<size_t> T = kv->temporal;
    std::vector<uint8_t> K = kv->kinds;
    std::vector<int64_t> src(T.size());
    for (size_t i = 0; i < src.size(); i++) src[i] = (int64_t)i;
    auto frames = [&] { return T.size() / ft; };
    if (frames() == 0) return ok();
    auto first_frame = [&](uint8_t kind) -> int64_t {
        for (size_t f = 0; f < frames(); f++)
            if (K[f * ft] == kind) return (int64_t)f;
        return -1;
    };
    // seed the zero EMA frames after the sinks: [sink, long, short] (lib.rs:728-752)
    if (first_frame(LX2V_SLOT_LONG_EMA) < 0 && frames() > cfg->sink_frames) {
        const size_t at = cfg->sink_frames * ft, t = T[std::min(at, T.size() - 1)];
        for (uint8_t kind : {(uint8_t)LX2V_SLOT_SHORT_EMA, (uint8_t)LX2V_SLOT_LONG_EMA}) {
            T.insert(T.begin() + at, ft, t);
            K.insert(K.begin() + at, ft, kind);
            src.insert(src.begin() + at, ft, (int64_t)-1);
        }
    }
    // graduate New frames past the window to Recent (lib.rs:754-768; new_frames() = 3, config.rs:298-300)
    {
        std::vector<size_t> nf;
        for (size_t f = 0; f < frames(); f++)
            if (K[f * ft] == LX2V_SLOT_NEW) nf.push_back(f);
        for (size_t i = 0; i + 3 < nf.size(); i++) std::fill(K.begin() + nf[i] * ft, K.begin() + (nf[i] + 1) * ft, (uint8_t)LX2V_SLOT_RECENT);
    }
    // fold and evict while over capacity (lib.rs:769-799)
    const uint8_t slot_kind[2] = {LX2V_SLOT_LONG_EMA, LX2V_SLOT_SHORT_EMA};
    std::vector<int64_t> init[2];
    std::vector<std::vector<int64_t>> evs[2];
    while (frames() > cfg->cache_frames) {
        int64_t f = first_frame(LX2V_SLOT_RECENT);
        if (f < 0) f = first_frame(LX2V_SLOT_NEW);
        if (f < 0) break;
        const size_t r0 = (size_t)f * ft;
        for (int s = 0; s < 2; s++) {
            const int64_t sf = first_frame(slot_kind[s]);
            if (sf < 0) continue;
            if (init[s].empty()) {  // the slot's rows before its first fold; from now on they are its output
                init[s].assign(src.begin() + sf * ft, src.begin() + (sf + 1) * ft);
                for (size_t o = 0; o < ft; o++) src[sf * ft + o] = -2 - (int64_t)(s * ft + o);
            }
            evs[s].emplace_back(src.begin() + r0, src.begin() + r0 + ft);
        }
        T.erase(T.begin() + r0, T.begin() + r0 + ft);
        K.erase(K.begin() + r0, K.begin() + r0 + ft);
        src.erase(src.begin() + r0, src.begin() + r0 + ft);
    }
    for (size_t f = 0; f < std::min<size_t>(cfg->sink_frames, frames()); f++)
        std::fill(K.begin() + f * ft, K.begin() + (f + 1) * ft, (uint8_t)LX2V_SLOT_SINK);  // lib.rs:800-805

    bool moved = src.size() != kv->rows();
    for (size_t i = 0; !moved && i < src.size(); i++) moved = src[i] != (int64_t)i;
    if (moved) {
        // plan: map, then per slot its init rows and evicted rows
        std::vector<int> plan(src.begin(), src.end());
        int n_ev[2], init_at[2], ev_at[2];
        float alpha[2] = {cfg->ema_alpha_long, cfg->ema_alpha_short};
        for (int s = 0; s < 2; s++) {
            n_ev[s] = (int)evs[s].size();
            init_at[s] = (int)plan.size();
            if (init[s].empty()) init[s].assign(ft, -1);
            plan.insert(plan.end(), init[s].begin(), init[s].end());
            ev_at[s] = (int)plan.size();
            for (auto &e : evs[s]) plan.insert(plan.end(), e.begin(), e.end());
        }
        if (plan.size() >= (1u << 31)) return fail(LX2V_ERR_BAD_SHAPE, "memrope_update: plan too large");
        if (plan.size() > kv->plan_cap) {
            HIP_TRY(hipStreamSynchronize(ctx->stream), "memrope_update");
            if (kv->plan_host) (void)hipHostFree(kv->plan_host);
            if (kv->plan_dev) (void)hipFree(kv->plan_dev);
            kv->plan_host = nullptr;
            kv->plan_dev = nullptr;
            kv->plan_cap = 0;
            HIP_TRY(hipHostMalloc((void **)&kv->plan_host, plan.size() * sizeof(int)), "hipHostMalloc(memrope plan)");
            HIP_TRY(hipMalloc((void **)&kv->plan_dev, plan.size() * sizeof(int)), "hipMalloc(memrope plan)");
            kv->plan_cap = plan.size();
        }
        HIP_TRY(hipEventSynchronize(kv->plan_done), "memrope_update");  // the previous plan's copy has run
        std::copy(plan.begin(), plan.end(), kv->plan_host);
        HIP_TRY(hipMemcpyAsync(kv->plan_dev, kv->plan_host, plan.size() * sizeof(int), hipMemcpyHostToDevice,
                               ctx->stream),
                "hipMemcpyAsync(memrope plan)");
        HIP_TRY(hipEventRecord(kv->plan_done, ctx->stream), "memrope_update");
        // gather into the context's spare layout, then swap it with the cache's
        auto &sp = ctx->kv_spare;
        const size_t need = 2 * kv->heads * std::max(src.size(), kv->cap) * kv->d * kv->eb();
        if (int rc = ensure(ctx, &sp.ptr, &sp.bytes, need, "kv_cache spare alloc")) return rc;
        const size_t dcap = kv_cap_of(kv, sp.bytes), rows = src.size();
        uint8_t *dst = (uint8_t *)sp.ptr;
        if (int rc = run(ctx, "kv_cache_memrope_update", [&] {
                launch_kv_remap(ctx->stream, kv->k(), kv->cap, dst, dcap, kv->dtype, kv->heads, rows, kv->d,
                                kv->plan_dev, (int)ft, n_ev, init_at, ev_at, alpha);
                launch_kv_remap(ctx->stream, kv->v(), kv->cap, dst + kv->heads * dcap * kv->d * kv->eb(), dcap,
                                kv->dtype, kv->heads, rows, kv->d, kv->plan_dev, (int)ft, n_ev, init_at, ev_at, alpha);
            }))
            return rc;
        std::swap(kv->buf, sp.ptr);
        std::swap(kv->bytes, sp.bytes);
        kv->cap = dcap;
    }
    kv->temporal = std::move(T);
    kv->kinds = std::move(K);
    return ok();
}

int lx2v_hip_kv_cache_attention(lx2v_hip_ctx *ctx, const lx2v_hip_buf *q, const lx2v_hip_kv *kv, size_t heads,
                                size_t sq, size_t head_dim, const lx2v_hip_mask *mask, lx2v_hip_buf *out) {
    NEED(kv, "cache");
    if (heads != kv->heads || head_dim != kv->d)
        return fail(LX2V_ERR_BAD_SHAPE, "kv_cache_attention: %zu heads of %zu, the cache holds %zu of %zu", heads,
                    head_dim, kv->heads, kv->d);
    const size_t sk = kv->rows();
    lx2v_hip_buf kb, vb;  // views of the cache: [heads, cap, d]
    kb.ptr = kv->k();
    vb.ptr = kv->v();
    kb.len = vb.len = kv->heads * kv->cap * kv->d;
    kb.dtype = vb.dtype = kv->dtype;
    if (int rc = attn_check(ctx, q, &kb, &vb, heads, sq, sk, head_dim, out)) return rc;
    if (mask && (mask->sq != sq || mask->sk != sk))
        return fail(LX2V_ERR_BAD_SHAPE, "kv_cache_attention: mask is %zux%zu, scores are %zux%zu", mask->sq, mask->sk,
                    sq, sk);
    if (!heads || !sq) return ok();
    const lx2v_hip_mask *m = mask && sq * sk ? mask : nullptr;
    float *part = nullptr;
    int nsplit = 1;
    if (int rc = attn_part(ctx, heads, sq, sk, head_dim, &part, &nsplit)) return rc;
    return run(ctx, m ? "causal_attention" : "attention", [&] {
        launch_attention(ctx->stream, q->ptr, kb.ptr, vb.ptr, q->dtype, heads, sq, sk, kv->cap, head_dim,
                         m ? m->bytes : nullptr, m ? m->bits : nullptr, m ? m->tiles : nullptr, out->ptr, out->dtype,
                         out->mxs, out->srows, part, nsplit);
    });
}

int lx2v_hip_fill_normal(lx2v_hip_ctx *ctx, lx2v_hip_buf *buf, uint64_t seed, float std) {
    NEED(ctx, "ctx");
    NEED(buf, "buf");
    if (buf->quantized()) return fail(LX2V_ERR_BAD_ARG, "fill_normal into an E4M3 / MXE4M3 buffer");
    if (int rc = set_dev(ctx)) return rc;
    if (int rc = run(ctx, "fill_normal", [&] {
            launch_fill_normal(ctx->stream, buf->ptr, buf->dtype, buf->len, seed, std);
        }))
        return rc;
    return ok();
}

// ---- pre-quantized activations ------------------------------------------------------

int lx2v_hip_alloc_e4m3(lx2v_hip_ctx *ctx, size_t rows, size_t cols, lx2v_hip_buf **out) {
    NEED(ctx, "ctx");
    NEED(out, "out");
    if (int rc = not_capturing(ctx, "alloc_e4m3")) return rc;
    if (cols && rows > ((size_t)1 << 40) / cols) return fail(LX2V_ERR_BAD_SHAPE, "E4M3 buffer %zux%zu too large", rows, cols);
    if (int rc = set_dev(ctx)) return rc;
    const size_t codes = (rows * cols + 255) & ~(size_t)255;
    auto *b = new lx2v_hip_buf;
    b->len = rows * cols;
    b->dtype = LX2V_DTYPE_E4M3;
    b->rows = rows;
    b->cols = cols;
    const size_t bytes = std::max<size_t>(codes + rows * 4, 4);
    hipError_t e = hipMalloc(&b->ptr, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(b->ptr, 0, bytes, ctx->stream);
    if (e != hipSuccess) {
        if (b->ptr) (void)hipFree(b->ptr);
        delete b;
        return hip_fail(e, "hipMalloc(E4M3 buffer)");
    }
    b->scales = (float *)((uint8_t *)b->ptr + codes);
    *out = b;
    return ok();
}

int lx2v_hip_quantize_act(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows,
                          lx2v_hip_buf *xq) {
    NEED(ctx, "ctx");
    NEED(x, "x");
    NEED(xq, "xq");
    if (xq->dtype != LX2V_DTYPE_E4M3) return fail(LX2V_ERR_BAD_ARG, "quantize_act writes an E4M3 buffer");
    if (x->quantized()) return fail(LX2V_ERR_BAD_ARG, "quantize_act reads an F32 or BF16 buffer");
    const size_t cols = xq->cols;
    if (rows > xq->rows) return fail(LX2V_ERR_BAD_SHAPE, "%zu rows into an E4M3 buffer of %zu", rows, xq->rows);
    if (x_row + rows < x_row || (x_row + rows) * cols > x->len)
        return fail(LX2V_ERR_BAD_SHAPE, "x has %zu elements, rows [%zu,+%zu) x %zu", x->len, x_row, rows, cols);
    if (!rows || !cols) return ok();
    if (int rc = set_dev(ctx)) return rc;
    const char *xp = (const char *)x->ptr + x_row * cols * x->elem_bytes();
    return run(ctx, "act_quant_e4m3",
               [&] { launch_act_quant(ctx->stream, xp, x->dtype, rows, cols, (uint8_t *)xq->ptr, xq->scales); });
}

int lx2v_hip_alloc_mx(lx2v_hip_ctx *ctx, size_t rows, size_t cols, lx2v_hip_buf **out) {
    NEED(ctx, "ctx");
    NEED(out, "out");
    if (int rc = not_capturing(ctx, "alloc_mx")) return rc;
    if (cols % 32) return fail(LX2V_ERR_BAD_SHAPE, "MXE4M3 buffer cols %zu not a multiple of 32", cols);
    if (cols && rows > ((size_t)1 << 40) / cols) return fail(LX2V_ERR_BAD_SHAPE, "MXE4M3 buffer %zux%zu too large", rows, cols);
    if (int rc = set_dev(ctx)) return rc;
    const size_t codes = (rows * cols + 255) & ~(size_t)255;
    const size_t srows = (rows + 15) & ~(size_t)15;
    auto *b = new lx2v_hip_buf;
    b->len = rows * cols;
    b->dtype = LX2V_DTYPE_MXE4M3;
    b->rows = rows;
    b->cols = cols;
    b->srows = srows;
    const size_t bytes = std::max<size_t>(codes + srows * 4 * ((cols + 127) / 128), 4);
    hipError_t e = hipMalloc(&b->ptr, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(b->ptr, 0, bytes, ctx->stream);
    if (e != hipSuccess) {
        if (b->ptr) (void)hipFree(b->ptr);
        delete b;
        return hip_fail(e, "hipMalloc(MXE4M3 buffer)");
    }
    b->mxs = (uint8_t *)b->ptr + codes;
    *out = b;
    return ok();
}

int lx2v_hip_download_mx(lx2v_hip_ctx *ctx, const lx2v_hip_buf *buf, uint8_t *codes, uint8_t *scales) {
    NEED(ctx, "ctx");
    NEED(buf, "buf");
    if (buf->dtype != LX2V_DTYPE_MXE4M3) return fail(LX2V_ERR_BAD_ARG, "download_mx reads an MXE4M3 buffer");
    if (buf->len) {
        NEED(codes, "codes");
        NEED(scales, "scales");
    }
    if (int rc = not_capturing(ctx, "download_mx")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    std::vector<uint8_t> raw(buf->srows * 4 * ((buf->cols + 127) / 128));
    if (buf->len) {
        HIP_TRY(hipMemcpyAsync(codes, buf->ptr, buf->len, hipMemcpyDeviceToHost, ctx->stream), "download_mx codes");
        HIP_TRY(hipMemcpyAsync(raw.data(), buf->mxs, raw.size(), hipMemcpyDeviceToHost, ctx->stream),
                "download_mx scales");
    }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(download_mx)");
    for (size_t b = 0; b < buf->cols / 32; b++)
        for (size_t r = 0; r < buf->rows; r++) scales[b * buf->rows + r] = raw[mx_sidx(r, b, buf->srows)];
    return ok();
}

int lx2v_hip_download_e4m3(lx2v_hip_ctx *ctx, const lx2v_hip_buf *buf, uint8_t *codes, float *scales) {
    NEED(ctx, "ctx");
    NEED(buf, "buf");
    if (buf->dtype != LX2V_DTYPE_E4M3) return fail(LX2V_ERR_BAD_ARG, "download_e4m3 reads an E4M3 buffer");
    if (buf->len) {
        NEED(codes, "codes");
        NEED(scales, "scales");
    }
    if (int rc = not_capturing(ctx, "download_e4m3")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    if (buf->len) {
        HIP_TRY(hipMemcpyAsync(codes, buf->ptr, buf->len, hipMemcpyDeviceToHost, ctx->stream), "download_e4m3 codes");
        HIP_TRY(hipMemcpyAsync(scales, buf->scales, buf->rows * 4, hipMemcpyDeviceToHost, ctx->stream),
                "download_e4m3 scales");
    }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(download_e4m3)");
    return ok();
}

int lx2v_hip_quantize_mx(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows, lx2v_hip_buf *xq) {
    NEED(ctx, "ctx");
    NEED(x, "x");
    NEED(xq, "xq");
    if (xq->dtype != LX2V_DTYPE_MXE4M3) return fail(LX2V_ERR_BAD_ARG, "quantize_mx writes an MXE4M3 buffer");
    if (x->quantized()) return fail(LX2V_ERR_BAD_ARG, "quantize_mx reads an F32 or BF16 buffer");
    const size_t cols = xq->cols;
    if (rows > xq->rows) return fail(LX2V_ERR_BAD_SHAPE, "%zu rows into an MXE4M3 buffer of %zu", rows, xq->rows);
    if (x_row + rows < x_row || (x_row + rows) * cols > x->len)
        return fail(LX2V_ERR_BAD_SHAPE, "x has %zu elements, rows [%zu,+%zu) x %zu", x->len, x_row, rows, cols);
    if (!rows || !cols) return ok();
    if (int rc = set_dev(ctx)) return rc;
    const char *xp = (const char *)x->ptr + x_row * cols * x->elem_bytes();
    return run(ctx, "act_quant_mx", [&] {
        launch_act_quant_mx(ctx->stream, xp, x->dtype, rows, cols, (uint8_t *)xq->ptr, xq->mxs, xq->srows);
    });
}

// ---- HIP graphs ------------------------------------------------------------------------

}  // extern "C"

struct lx2v_hip_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool uses_scratch = false;  // holds linear_noalloc calls: each launch claims the device scratch
};

extern "C" {

int lx2v_hip_graph_begin(lx2v_hip_ctx *ctx) {
    NEED(ctx, "ctx");
    if (ctx->capturing) return fail(LX2V_ERR_BAD_ARG, "graph capture already in progress");
    if (int rc = set_dev(ctx)) return rc;
    prof_harvest(ctx);  // pending profiler events must not straddle the capture
    HIP_TRY(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    ctx->capturing = true;
    ctx->capture_scratch = false;
    return ok();
}

int lx2v_hip_graph_end(lx2v_hip_ctx *ctx, lx2v_hip_graph **out) {
    NEED(ctx, "ctx");
    NEED(out, "out");
    if (!ctx->capturing) return fail(LX2V_ERR_BAD_ARG, "no graph capture in progress");
    if (int rc = set_dev(ctx)) return rc;
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamEndCapture(ctx->stream, &g), "hipStreamEndCapture");
    auto *gr = new lx2v_hip_graph;
    gr->graph = g;
    gr->uses_scratch = ctx->capture_scratch;
    hipError_t e = hipGraphInstantiate(&gr->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        delete gr;
        return hip_fail(e, "hipGraphInstantiate");
    }
    *out = gr;
    return ok();
}

int lx2v_hip_graph_launch(lx2v_hip_ctx *ctx, const lx2v_hip_graph *g) {
    NEED(ctx, "ctx");
    NEED(g, "graph");
    if (int rc = not_capturing(ctx, "graph_launch")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    if (!g->uses_scratch) {
        HIP_TRY(hipGraphLaunch(g->exec, ctx->stream), "hipGraphLaunch");
        return ok();
    }
    hipError_t e = hipSuccess;
    void *p = nullptr;
    switch (scratch_claim(ctx->device, ctx, ctx->scratch_done, &p, &e)) {
        case ScratchClaim::Busy:
            return fail(LX2V_ERR_BUSY, "graph_launch: the graph holds linear_noalloc calls and the device scratch is "
                        "in use by another context's work in flight on device %d", ctx->device);
        case ScratchClaim::Error: return hip_fail(e, "graph_launch: device scratch");
        case ScratchClaim::Held: break;
    }
    e = hipGraphLaunch(g->exec, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(ctx->scratch_done, ctx->stream);
    scratch_unlock(ctx->device);
    if (e != hipSuccess) return hip_fail(e, "hipGraphLaunch");
    return ok();
}

int lx2v_hip_graph_free(lx2v_hip_ctx *ctx, lx2v_hip_graph *g) {
    NEED(ctx, "ctx");
    if (!g) return ok();
    if (int rc = not_capturing(ctx, "graph_free")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(graph_free)");
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
    return ok();
}

// ---- linear ----------------------------------------------------------------------

static int act_quant_into_ws(lx2v_hip_ctx *ctx, const void *x, int dtype, size_t rows, size_t cols,
                             uint8_t **q, float **s) {
    size_t qbytes = (rows * cols + 255) & ~(size_t)255;
    if (int rc = ensure(ctx, &ctx->ws, &ctx->ws_bytes, qbytes + rows * 4, "workspace alloc")) return rc;
    *q = (uint8_t *)ctx->ws;
    *s = (float *)((uint8_t *)ctx->ws + qbytes);
    return run(ctx, "act_quant_e4m3", [&] { launch_act_quant(ctx->stream, x, dtype, rows, cols, *q, *s); });
}

// gate: residual mode (only where linear_fusable says so): y is the
// residual stream, y[r] += out[r] * gate.
// scr: the no-alloc variant -- every workspace comes from this device
// memory (bias staging first, then the activations' e4m3 codes and row
// scales or their bf16 copy), and the call fails cleanly if it is too small.
static int linear_run(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows, const lx2v_hip_weight *w,
                      const lx2v_hip_buf *bias, int act, lx2v_hip_buf *y, size_t y_row, const float *gate,
                      const lx2v::Scratch *scr = nullptr) {
    NEED(ctx, "ctx");
    NEED(x, "x");
    NEED(w, "weight");
    NEED(y, "y");
    if (act != LX2V_ACT_NONE && act != LX2V_ACT_GELU_TANH) return fail(LX2V_ERR_BAD_ARG, "unknown act %d", act);
    const size_t N = w->rows, K = w->cols;
    if (x_row + rows < x_row || (x_row + rows) * K > x->len)
        return fail(LX2V_ERR_BAD_SHAPE, "x has %zu elements, rows [%zu,+%zu) x %zu need %zu", x->len, x_row, rows,
                    K, (x_row + rows) * K);
    if (y_row + rows < y_row || (y_row + rows) * N > y->len)
        return fail(LX2V_ERR_BAD_SHAPE, "y has %zu elements, rows [%zu,+%zu) x %zu need %zu", y->len, y_row, rows,
                    N, (y_row + rows) * N);
    if (bias && bias->len < N) return fail(LX2V_ERR_BAD_SHAPE, "bias has %zu elements, weight has %zu rows", bias->len, N);
    if (y->dtype == LX2V_DTYPE_E4M3 || (bias && bias->quantized()))
        return fail(LX2V_ERR_BAD_ARG, "linear writes F32, BF16 or MXE4M3 and reads an F32 or BF16 bias");
    if (x->quantized()) {
        if (x->cols != K) return fail(LX2V_ERR_BAD_SHAPE, "E4M3 / MXE4M3 x has %zu cols, weight has %zu", x->cols, K);
        if (w->fmt != LX2V_WFMT_FP8)
            return fail(LX2V_ERR_UNSUPPORTED, "E4M3 / MXE4M3 activations need an FP8 weight");
    }
    const bool x_mx = x->dtype == LX2V_DTYPE_MXE4M3, y_mx = y->dtype == LX2V_DTYPE_MXE4M3;
    if (y_mx && y->cols != N) return fail(LX2V_ERR_BAD_SHAPE, "MXE4M3 y has %zu cols, weight has %zu rows", y->cols, N);
    // FP8 weights the fp8 MFMA takes: one scale per channel, or per 128 columns.
    const bool fp8_grouped = w->fmt == LX2V_WFMT_FP8 && w->group != K && w->gratio_ok &&
                             gemm_fp8_grouped_supported(rows, N, K, w->group);
    const bool fp8_mfma = w->fmt == LX2V_WFMT_FP8 && (w->group == K ? gemm_fp8_supported(rows, N, K) : fp8_grouped);
    if ((x_mx || y_mx) && (!fp8_mfma || K % 128 || (x_mx && x_row % 16)))
        return fail(LX2V_ERR_UNSUPPORTED,
                    "MXE4M3 operands need an FP8 weight with cols %% 128 == 0 and one scale per channel or per 128 "
                    "columns, and an MX input row offset %% 16 == 0 (weight %zux%zu group %zu, x_row %zu)",
                    N, K, w->group, x_row);
    const char *xp = (const char *)x->ptr + x_row * K * x->elem_bytes();
    char *yp = (char *)y->ptr + y_row * N * y->elem_bytes();
    if (overlap(yp, rows * N * y->elem_bytes(), xp, rows * K * x->elem_bytes()) ||
        (x->scales && overlap(yp, rows * N * y->elem_bytes(), x->scales + x_row, rows * 4)))
        return fail(LX2V_ERR_ALIAS, "linear output overlaps its input");
    if (bias && overlap(yp, rows * N * y->elem_bytes(), bias->ptr, N * bias->elem_bytes()))
        return fail(LX2V_ERR_ALIAS, "linear output overlaps its bias");
    if (!rows) return ok();

    // The e4m3 path: quantized activations, MX output, or (per-token e4m3
    // mode) an FP8 weight the fp8 MFMA takes or no bf16 GEMM tiles (the
    // scalar kernel on e4m3 activations).  FP8 weights with other groups
    // that the bf16 GEMM takes run it below (the weight dequantized to bf16
    // in its loader, bf16 activations).
    const bool w16_ok = gemm_w16_dma_supported(w, rows) ||
                        (gemm_w16_supported(w) && rows * K * x->elem_bytes() < (1ull << 31));
    const bool e4m3_path = w->fmt == LX2V_WFMT_FP8 &&
                           (x->quantized() || y_mx || (ctx->fp8_act == LX2V_FP8_ACT_E4M3 && (fp8_mfma || !w16_ok)));
    // Native f32 weights on the bf16 MFMA (their bf16 copy, bf16 activations).
    const bool native_bf16 = w->fmt == LX2V_WFMT_F32 && w->wbf16 && ctx->native_mode == LX2V_NATIVE_BF16 &&
                             gemm_bf16_supported(rows, N, K);
    // The fp8 MFMA's plan, made before anything is enqueued: a call refused
    // below leaves nothing on the stream.
    Fp8Plan plan;
    if (e4m3_path && fp8_mfma) {
        plan = plan_gemm_fp8(ctx->num_cu, rows, N, K, x_mx || y_mx, x_mx, fp8_grouped, y->dtype, act, gate != nullptr,
                             true);
        if (fp8_grouped && plan.kernel != 0 && plan.kernel != 1 && plan.kernel != 6 && plan.kernel != 7 &&
            plan.kernel != 10)  // built with grouped scales
            return fail(LX2V_ERR_UNSUPPORTED, "no grouped-scale fp8 kernel for configuration %d", plan.kernel);
    }
    // Workspaces, each piece 256-byte aligned: a bf16 bias's f32 copy; the
    // activations' e4m3 codes and row scales, or their bf16 copy; split K's
    // f32 partial sums.  The no-alloc variant lays them out in that order in
    // the device scratch; `linear` keeps them in context workspaces, all
    // grown here, before the first launch.
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t s_bias = bias && bias->dtype != LX2V_DTYPE_F32 ? al(N * 4) : 0;
    const size_t s_act = e4m3_path ? (x->quantized() ? 0 : al(rows * K) + al(rows * 4))
                                   : ((gemm_w16_dma_supported(w, rows) || native_bf16) && x->dtype == LX2V_DTYPE_F32
                                          ? al(rows * K * 2)
                                          : 0);
    const size_t s_part = plan.splits > 1 ? al((size_t)plan.splits * rows * N * 4) : 0;
    if (scr && s_bias + s_act + s_part > scr->bytes)
        return fail(LX2V_ERR_UNSUPPORTED,
                    "linear_noalloc: this call needs %zu bytes of scratch (rows %zu x cols %zu -> %zu), the maximum "
                    "is %zu",
                    s_bias + s_act + s_part, rows, K, N, scr->bytes);
    if (int rc = set_dev(ctx)) return rc;
    uint8_t *p_bias = nullptr, *p_act = nullptr;
    float *p_part = nullptr;
    if (scr) {
        p_bias = scr->ptr;
        p_act = scr->ptr + s_bias;
        p_part = (float *)(scr->ptr + s_bias + s_act);
    } else {
        void *st = nullptr;
        if (s_bias)  // slot 0 of the staging (linear_residual's gate is in slot 2)
            if (int rc = stage_for(ctx, N * 4, &st)) return rc;
        if (s_act)
            if (int rc = ensure(ctx, &ctx->ws, &ctx->ws_bytes, s_act, "workspace alloc")) return rc;
        if (s_part)
            if (int rc = ensure(ctx, &ctx->splitk.ptr, &ctx->splitk.bytes, s_part, "split-K workspace alloc"))
                return rc;
        p_bias = (uint8_t *)st;
        p_act = (uint8_t *)ctx->ws;
        p_part = (float *)ctx->splitk.ptr;
    }

    // The epilogue reads an f32 bias.
    const float *bp = nullptr;
    if (bias) {
        if (bias->dtype == LX2V_DTYPE_F32) {
            bp = (const float *)bias->ptr;
        } else {
            if (int rc = run(ctx, "convert", [&] {
                    launch_convert(ctx->stream, bias->ptr, LX2V_DTYPE_BF16, p_bias, LX2V_DTYPE_F32, N);
                }))
                return rc;
            bp = (const float *)p_bias;
        }
    }

    if (e4m3_path) {
        const uint8_t *q;
        const float *s = nullptr;
        Fp8Mx mx;
        if (x->dtype == LX2V_DTYPE_E4M3) {
            q = (const uint8_t *)xp;
            s = x->scales + x_row;
        } else if (x_mx) {
            q = (const uint8_t *)xp;
            mx.a = x->mxs + 4 * x_row;
            mx.a_rows = x->srows;
            mx.a_len = x->srows * 4 * (K / 128) - 4 * x_row;
        } else {
            uint8_t *wq = p_act;
            float *ws = (float *)(p_act + al(rows * K));
            if (int rc = run(ctx, "act_quant_e4m3", [&] { launch_act_quant(ctx->stream, xp, x->dtype, rows, K, wq, ws); }))
                return rc;
            q = wq;
            s = ws;
        }
        if (y_mx) {
            mx.y = y->mxs + 4 * y_row;
            mx.y_rows = y->srows;
        }
        mx.gate = gate;
        if (fp8_mfma) {
            if (fp8_grouped) mx.wgs = w->gratio;
            if (plan.splits > 1) mx.part = p_part;
            // Profile name: the kernel configuration and the operand forms,
            // e.g. "gemm_fp8_e4m3.c0.g128.mxout".
            char pname[64];
            char cfg[8] = "creg";  // the register-staged kernel (K % 128 != 0)
            if (plan.kernel >= 0) snprintf(cfg, sizeof cfg, plan.splits > 1 ? "c%dk%d" : "c%d", plan.kernel, plan.splits);
            snprintf(pname, sizeof pname, "gemm_fp8_e4m3.%s%s%s%s%s", cfg, fp8_grouped ? ".g128" : "", x_mx ? ".mxin" : "", y_mx ? ".mxout" : "", gate ? ".res" : "");
            if (int rc = run(ctx, pname, [&] {
                    launch_gemm_fp8(ctx->stream, ctx->num_cu, plan, q, s, (const uint8_t *)w->codes,
                                    fp8_grouped ? w->glast : w->scales, bp, act, yp, y->dtype, rows, N, K, mx);
                }))
                return rc;
        } else {
            if ((rows + 15) / 16 > 65535)
                return fail(LX2V_ERR_UNSUPPORTED, "rows %zu too many for the generic kernel", rows);
            if (int rc = run(ctx, "gemm_generic", [&] {
                    launch_gemm_generic(ctx->stream, q, A_E4M3, s, w, bp, act, yp, y->dtype, rows);
                }))
                return rc;
        }
        return ok();
    }
    // bf16 activations for the direct-to-LDS kernels: f32 ones rounded (RNE,
    // as the register-staged loader would) into the workspace.
    auto bf16_x = [&](const uint16_t **xb) -> int {
        *xb = (const uint16_t *)xp;
        if (x->dtype != LX2V_DTYPE_F32) return LX2V_OK;
        if (int rc = run(ctx, "convert", [&] {
                launch_convert(ctx->stream, xp, LX2V_DTYPE_F32, p_act, LX2V_DTYPE_BF16, rows * K);
            }))
            return rc;
        *xb = (const uint16_t *)p_act;
        return LX2V_OK;
    };
    if (native_bf16) {
        const uint16_t *xb;
        if (int rc = bf16_x(&xb)) return rc;
        if (int rc = run(ctx, "gemm_bf16_native", [&] {
                launch_gemm_bf16(ctx->stream, ctx->num_cu, xb, w->wbf16, bp, act, yp, y->dtype, rows, N, K);
            }))
            return rc;
        return ok();
    }
    const char *name = w->fmt == LX2V_WFMT_Q8 ? "gemm_w16_q8" : w->fmt == LX2V_WFMT_Q4 ? "gemm_w16_q4" : "gemm_w16_fp8";
    if (gemm_w16_dma_supported(w, rows)) {
        const uint16_t *xb;
        if (int rc = bf16_x(&xb)) return rc;
        const int cfg = plan_gemm_w16_dma(ctx->num_cu, rows, N);
        char pname[40];  // e.g. "gemm_w16_q8.c2": the tile configuration
        snprintf(pname, sizeof pname, "%s.c%d", name, cfg);
        if (int rc = run(ctx, pname, [&] {
                launch_gemm_w16_dma(ctx->stream, cfg, xb, w, bp, act, yp, y->dtype, rows);
            }))
            return rc;
        return ok();
    }
    // The tile loaders address X with 32-bit buffer offsets.
    if (w->fmt != LX2V_WFMT_F32 && gemm_w16_supported(w) && rows * K * x->elem_bytes() < (1ull << 31)) {
        if (int rc = run(ctx, name, [&] {
                launch_gemm_w16(ctx->stream, ctx->num_cu, xp, x->dtype, w, bp, act, yp, y->dtype, rows);
            }))
            return rc;
        return ok();
    }
    if ((rows + 15) / 16 > 65535) return fail(LX2V_ERR_UNSUPPORTED, "rows %zu too many for the generic kernel", rows);
    int amode = x->dtype == LX2V_DTYPE_BF16 ? A_BF16 : A_F32;
    if (int rc = run(ctx, "gemm_generic", [&] {
            launch_gemm_generic(ctx->stream, xp, amode, nullptr, w, bp, act, yp, y->dtype, rows);
        }))
        return rc;
    return ok();
}

int lx2v_hip_linear(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows,
                    const lx2v_hip_weight *w, const lx2v_hip_buf *bias, int act, lx2v_hip_buf *y,
                    size_t y_row) {
    return linear_run(ctx, x, x_row, rows, w, bias, act, y, y_row, nullptr);
}

// No counterpart in the reference: `linear` for callers that cannot
// allocate.  The workspaces come from the device scratch array of
// lx2v_scratch.hip (kScratchBytes per device); no hipMalloc / hipFree, no
// profiler events.  The array is held by one context at a time: while
// another context's work on it is still in flight the call fails with
// LX2V_ERR_BUSY and enqueues nothing.
int lx2v_hip_linear_noalloc(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows,
                            const lx2v_hip_weight *w, const lx2v_hip_buf *bias, int act, lx2v_hip_buf *y,
                            size_t y_row) {
    NEED(ctx, "ctx");
    if (int rc = set_dev(ctx)) return rc;
    hipError_t e = hipSuccess;
    void *p = nullptr;
    if (ctx->capturing) {
        // Nothing runs until the graph is launched, and each launch claims
        // the array (lx2v_hip_graph_launch); no event may be queried here.
        p = scratch_address(ctx->device, &e);
        if (!p) return hip_fail(e, "linear_noalloc: device scratch");
    } else {
        switch (scratch_claim(ctx->device, ctx, ctx->scratch_done, &p, &e)) {
            case ScratchClaim::Busy:
                return fail(LX2V_ERR_BUSY,
                            "linear_noalloc: the device scratch is in use by another context's work in flight on "
                            "device %d", ctx->device);
            case ScratchClaim::Error: return hip_fail(e, "linear_noalloc: device scratch");
            case ScratchClaim::Held: break;
        }
    }
    const lx2v::Scratch scr{(uint8_t *)p, kScratchBytes};
    const bool prof = ctx->prof.on;
    ctx->prof.on = false;  // no event creation inside this call
    int rc = linear_run(ctx, x, x_row, rows, w, bias, act, y, y_row, nullptr, &scr);
    ctx->prof.on = prof;
    if (ctx->capturing) {
        ctx->capture_scratch = true;
        return rc;
    }
    const hipError_t er = hipEventRecord(ctx->scratch_done, ctx->stream);
    if (er != hipSuccess && rc == LX2V_OK) rc = hip_fail(er, "hipEventRecord(linear_noalloc)");
    scratch_unlock(ctx->device);
    return rc;
}

// The residual add can ride in the GEMM's epilogue: FP8 weight with one scale
// per channel on the e4m3 path, a bf16 / f32 output, and a direct-to-LDS
// configuration (K % 128 == 0; not the 256 x 256 ping-pong tile), where
// linear itself would not split K (its sums would then be added in another
// order than the fused kernel's; the pair keeps the two equal).
static bool linear_fusable(const lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t rows, const lx2v_hip_weight *w,
                           const lx2v_hip_buf *h) {
    const size_t N = w->rows, K = w->cols;
    const bool x_mx = x->dtype == LX2V_DTYPE_MXE4M3;
    const bool grouped = w->group != K;
    if (w->fmt != LX2V_WFMT_FP8 || h->quantized() || !gemm_fp8_supported(rows, N, K)) return false;
    if (grouped && !(w->gratio_ok && gemm_fp8_grouped_supported(rows, N, K, w->group))) return false;
    if (!(ctx->fp8_act == LX2V_FP8_ACT_E4M3 || x->quantized())) return false;
    if (plan_gemm_fp8(ctx->num_cu, rows, N, K, x_mx, x_mx, grouped, h->dtype, LX2V_ACT_NONE, false, true).splits > 1)
        return false;
    return gemm_fp8_residual_ok(plan_gemm_fp8(ctx->num_cu, rows, N, K, x_mx, x_mx, grouped, h->dtype, LX2V_ACT_NONE, true));
}

int lx2v_hip_linear_residual(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows,
                             const lx2v_hip_weight *w, const lx2v_hip_buf *bias, int act, lx2v_hip_buf *h,
                             size_t h_row, const lx2v_hip_buf *mods, size_t gate) {
    NEED(ctx, "ctx");
    NEED(x, "x");
    NEED(w, "weight");
    NEED(h, "h");
    if (h->quantized()) return fail(LX2V_ERR_BAD_ARG, "linear_residual: h is an F32 or BF16 buffer");
    const size_t N = w->rows;
    if (h_row + rows < h_row || (h_row + rows) * N > h->len)
        return fail(LX2V_ERR_BAD_SHAPE, "h has %zu elements, rows [%zu,+%zu) x %zu need %zu", h->len, h_row, rows, N,
                    (h_row + rows) * N);
    if (mods && overlap(mods->ptr, mods->bytes(), (char *)h->ptr + h_row * N * h->elem_bytes(), rows * N * h->elem_bytes()))
        return fail(LX2V_ERR_ALIAS, "linear_residual: h overlaps mods");
    if (!rows) return ok();
    if (int rc = set_dev(ctx)) return rc;
    const float *g = nullptr;  // slot 2 of the staging: linear's bias conversion uses slot 0
    if (int rc = param_f32(ctx, mods, gate * N, N, 2, &g, "mods (gate)")) return rc;
    if (linear_fusable(ctx, x, rows, w, h)) return linear_run(ctx, x, x_row, rows, w, bias, act, h, h_row, g);
    // Elsewhere: the linear into a workspace of h's dtype, then the add.
    auto &st = ctx->resid;
    if (int rc = ensure(ctx, &st.ptr, &st.bytes, rows * N * h->elem_bytes(), "residual workspace alloc")) return rc;
    lx2v_hip_buf yb;
    yb.ptr = st.ptr;
    yb.len = rows * N;
    yb.dtype = h->dtype;
    if (int rc = linear_run(ctx, x, x_row, rows, w, bias, act, &yb, 0, nullptr)) return rc;
    return run(ctx, "gate_residual", [&] {
        launch_gate_residual(ctx->stream, (char *)h->ptr + h_row * N * h->elem_bytes(), yb.ptr, h->dtype, g, rows, N);
    });
}

int lx2v_hip_act_quant(lx2v_hip_ctx *ctx, const lx2v_hip_buf *x, size_t x_row, size_t rows, size_t cols,
                       uint8_t *q, float *s) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "act_quant")) return rc;
    NEED(x, "x");
    if (rows) {
        NEED(q, "q");
        NEED(s, "s");
    }
    if ((x_row + rows) * cols > x->len)
        return fail(LX2V_ERR_BAD_SHAPE, "x has %zu elements, rows [%zu,+%zu) x %zu", x->len, x_row, rows, cols);
    if (!rows || !cols) return ok();
    if (int rc = set_dev(ctx)) return rc;
    uint8_t *dq;
    float *ds;
    const char *xp = (const char *)x->ptr + x_row * cols * x->elem_bytes();
    if (int rc = act_quant_into_ws(ctx, xp, x->dtype, rows, cols, &dq, &ds)) return rc;
    HIP_TRY(hipMemcpyAsync(q, dq, rows * cols, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync(act_quant)");
    HIP_TRY(hipMemcpyAsync(s, ds, rows * 4, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync(act_quant)");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(act_quant)");
    return ok();
}

// ---- sync / profile ----------------------------------------------------------------

int lx2v_hip_sync(lx2v_hip_ctx *ctx) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "sync")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return ok();
}

int lx2v_hip_profile_enable(lx2v_hip_ctx *ctx, int on) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "profile_enable")) return rc;
    if (!on) prof_harvest(ctx);
    ctx->prof.on = on != 0;
    return ok();
}

int lx2v_hip_profile_report(lx2v_hip_ctx *ctx, char *out, size_t cap) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "profile_report")) return rc;
    NEED(out, "out");
    if (!cap) return fail(LX2V_ERR_BAD_ARG, "cap is 0");
    if (int rc = set_dev(ctx)) return rc;
    prof_harvest(ctx);
    std::string s;
    if (!ctx->prof.stats.empty()) {
        std::vector<std::pair<std::string, std::pair<uint64_t, double>>> rows(ctx->prof.stats.begin(),
                                                                              ctx->prof.stats.end());
        std::sort(rows.begin(), rows.end(), [](auto &a, auto &b) { return a.second.second > b.second.second; });
        double total = 0;
        for (auto &r : rows) total += r.second.second;
        char line[256];
        s += "hip profile (HIP events per kernel on the context stream):\n";
        s += "kernel              calls      total_ms   mean_us   share\n";
        for (auto &r : rows) {
            snprintf(line, sizeof line, "%-18s %8llu %12.3f %9.1f %6.1f%%\n", r.first.c_str(),
                     (unsigned long long)r.second.first, r.second.second, r.second.second * 1e3 / r.second.first,
                     total > 0 ? r.second.second / total * 100.0 : 0.0);
            s += line;
        }
        snprintf(line, sizeof line, "profile total: %.3f ms\n", total);
        s += line;
    }
    snprintf(out, cap, "%s", s.c_str());
    return ok();
}

int lx2v_hip_profile_reset(lx2v_hip_ctx *ctx) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "profile_reset")) return rc;
    prof_harvest(ctx);
    ctx->prof.stats.clear();
    return ok();
}

int lx2v_hip_profile_region(lx2v_hip_ctx *ctx, const char *name, int begin) {
    NEED(ctx, "ctx");
    NEED(name, "name");
    if (int rc = not_capturing(ctx, "profile_region")) return rc;
    if (int rc = set_dev(ctx)) return rc;
    auto &p = ctx->prof;
    auto it = p.open_regions.find(name);
    if (begin) {
        if (it != p.open_regions.end()) return fail(LX2V_ERR_BAD_ARG, "region %s is already open", name);
        hipEvent_t a;
        HIP_TRY(hipEventCreate(&a), "hipEventCreate(region)");
        hipError_t e = hipEventRecord(a, ctx->stream);
        if (e != hipSuccess) {
            (void)hipEventDestroy(a);
            return hip_fail(e, "hipEventRecord(region)");
        }
        p.open_regions[name] = a;
        return ok();
    }
    if (it == p.open_regions.end()) return fail(LX2V_ERR_BAD_ARG, "region %s was not opened", name);
    hipEvent_t b;
    HIP_TRY(hipEventCreate(&b), "hipEventCreate(region)");
    hipError_t e = hipEventRecord(b, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, it->second, b);
    (void)hipEventDestroy(it->second);
    (void)hipEventDestroy(b);
    p.open_regions.erase(it);
    if (e != hipSuccess) return hip_fail(e, "region timing");
    auto &st = p.stats[name];
    st.first += 1;
    st.second += ms;
    return ok();
}

int lx2v_hip_profile_kernel(lx2v_hip_ctx *ctx, const char *name, uint64_t *calls, double *total_ms) {
    NEED(ctx, "ctx");
    if (int rc = not_capturing(ctx, "profile_kernel")) return rc;
    NEED(name, "name");
    NEED(calls, "calls");
    NEED(total_ms, "total_ms");
    if (int rc = set_dev(ctx)) return rc;
    prof_harvest(ctx);
    auto it = ctx->prof.stats.find(name);
    *calls = it == ctx->prof.stats.end() ? 0 : it->second.first;
    *total_ms = it == ctx->prof.stats.end() ? 0.0 : it->second.second;
    return ok();
}

}  // extern "C"

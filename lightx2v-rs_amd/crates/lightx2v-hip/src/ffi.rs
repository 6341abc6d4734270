//! The C ABI of liblightx2v_hip.so, one declaration per entry point of
//! include/lightx2v_hip.h (tests/test_rust_ffi.py checks names, arity and
//! argument kinds against the header).  Every function returns an `int`
//! status (OK = 0); the message of a failed call is `lx2v_hip_last_error()`
//! (per thread).

#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_double, c_float, c_int, c_void};

#[repr(C)]
pub struct Ctx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct RawBuf {
    _p: [u8; 0],
}
#[repr(C)]
pub struct RawWeight {
    _p: [u8; 0],
}
#[repr(C)]
pub struct RawMask {
    _p: [u8; 0],
}
#[repr(C)]
pub struct RawKv {
    _p: [u8; 0],
}
#[repr(C)]
pub struct RawGraph {
    _p: [u8; 0],
}

pub const ABI_VERSION: c_int = 3;

pub const OK: c_int = 0;
pub const ERR_NO_DEVICE: c_int = 1;
pub const ERR_BAD_SHAPE: c_int = 2;
pub const ERR_ALIAS: c_int = 3;
pub const ERR_HIP: c_int = 4;
pub const ERR_BAD_ARG: c_int = 5;
pub const ERR_OOM: c_int = 6;
pub const ERR_UNSUPPORTED: c_int = 7;
pub const ERR_BUSY: c_int = 8;

pub const ACT_NONE: c_int = 0;
pub const ACT_GELU_TANH: c_int = 1;

pub const DTYPE_F32: c_int = 0;
pub const DTYPE_BF16: c_int = 1;
pub const DTYPE_E4M3: c_int = 2;
pub const DTYPE_MXE4M3: c_int = 3;

pub const WFMT_F32: c_int = 0;
pub const WFMT_Q8: c_int = 1;
pub const WFMT_Q4: c_int = 2;
pub const WFMT_FP8: c_int = 3;

pub const FP8_ACT_E4M3: c_int = 0;
pub const FP8_ACT_BF16: c_int = 1;
pub const NATIVE_BF16: c_int = 0;
pub const NATIVE_F32: c_int = 1;

pub const NORM_AFFINE: c_int = 0;
pub const NORM_MOD: c_int = 1;

pub const SLOT_SINK: u8 = 0;
pub const SLOT_LONG_EMA: u8 = 1;
pub const SLOT_SHORT_EMA: u8 = 2;
pub const SLOT_RECENT: u8 = 3;
pub const SLOT_NEW: u8 = 4;

#[repr(C)]
#[derive(Debug, Default, Clone, Copy)]
pub struct lx2v_hip_weight_info_t {
    pub fmt: c_int,
    pub rows: usize,
    pub cols: usize,
    pub group: usize,
    pub device_bytes: usize,
    pub canonicalized: usize,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct lx2v_hip_norm_t {
    pub kind: c_int,
    pub w: *const RawBuf,
    pub b: *const RawBuf,
    pub scale: usize,
    pub shift: usize,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct lx2v_hip_memrope_t {
    pub cache_frames: usize,
    pub sink_frames: usize,
    pub ema_alpha_long: c_float,
    pub ema_alpha_short: c_float,
}

extern "C" {
    pub fn lx2v_hip_last_error() -> *const c_char;
    pub fn lx2v_hip_device_count(count: *mut c_int) -> c_int;
    pub fn lx2v_hip_create(device: c_int, out: *mut *mut Ctx) -> c_int;
    pub fn lx2v_hip_destroy(ctx: *mut Ctx) -> c_int;
    pub fn lx2v_hip_name(ctx: *const Ctx, out: *mut c_char, cap: usize) -> c_int;
    pub fn lx2v_hip_set_act_dtype(ctx: *mut Ctx, dtype: c_int) -> c_int;
    pub fn lx2v_hip_set_fp8_act(ctx: *mut Ctx, mode: c_int) -> c_int;
    pub fn lx2v_hip_set_native_mode(ctx: *mut Ctx, mode: c_int) -> c_int;

    // ---- buffers
    pub fn lx2v_hip_alloc(ctx: *mut Ctx, len: usize, out: *mut *mut RawBuf) -> c_int;
    pub fn lx2v_hip_alloc_dtype(ctx: *mut Ctx, len: usize, dtype: c_int, out: *mut *mut RawBuf) -> c_int;
    pub fn lx2v_hip_upload(ctx: *mut Ctx, data: *const c_float, len: usize, out: *mut *mut RawBuf) -> c_int;
    pub fn lx2v_hip_write(ctx: *mut Ctx, buf: *mut RawBuf, data: *const c_float, len: usize) -> c_int;
    pub fn lx2v_hip_download(ctx: *mut Ctx, buf: *const RawBuf, out: *mut c_float, len: usize) -> c_int;
    pub fn lx2v_hip_buf_len(buf: *const RawBuf, len: *mut usize) -> c_int;
    pub fn lx2v_hip_buf_dtype(buf: *const RawBuf, dtype: *mut c_int) -> c_int;
    pub fn lx2v_hip_copy(
        ctx: *mut Ctx,
        src: *const RawBuf,
        src_off: usize,
        dst: *mut RawBuf,
        dst_off: usize,
        len: usize,
    ) -> c_int;
    pub fn lx2v_hip_buf_free(ctx: *mut Ctx, buf: *mut RawBuf) -> c_int;

    // ---- weights
    pub fn lx2v_hip_weight_f32(
        ctx: *mut Ctx,
        data: *const c_float,
        rows: usize,
        cols: usize,
        out: *mut *mut RawWeight,
    ) -> c_int;
    pub fn lx2v_hip_weight_q8(
        ctx: *mut Ctx,
        q: *const i8,
        scales: *const c_float,
        rows: usize,
        cols: usize,
        group: usize,
        out: *mut *mut RawWeight,
    ) -> c_int;
    pub fn lx2v_hip_weight_q4(
        ctx: *mut Ctx,
        codes: *const u8,
        packed: c_int,
        scales: *const c_float,
        zeros: *const c_float,
        rows: usize,
        cols: usize,
        group: usize,
        out: *mut *mut RawWeight,
    ) -> c_int;
    pub fn lx2v_hip_weight_fp8(
        ctx: *mut Ctx,
        q: *const u8,
        scales: *const c_float,
        rows: usize,
        cols: usize,
        group: usize,
        out: *mut *mut RawWeight,
    ) -> c_int;
    pub fn lx2v_hip_weight_free(ctx: *mut Ctx, w: *mut RawWeight) -> c_int;
    pub fn lx2v_hip_weight_info(w: *const RawWeight, info: *mut lx2v_hip_weight_info_t) -> c_int;
    pub fn lx2v_hip_weight_dequantize(ctx: *mut Ctx, w: *const RawWeight, out: *mut c_float, len: usize) -> c_int;
    pub fn lx2v_hip_quantize_q8(
        ctx: *mut Ctx,
        src: *const RawBuf,
        rows: usize,
        cols: usize,
        group: usize,
        out: *mut *mut RawWeight,
    ) -> c_int;
    pub fn lx2v_hip_quantize_q4_sym(
        ctx: *mut Ctx,
        src: *const RawBuf,
        rows: usize,
        cols: usize,
        group: usize,
        out: *mut *mut RawWeight,
    ) -> c_int;
    pub fn lx2v_hip_quantize_fp8(
        ctx: *mut Ctx,
        src: *const RawBuf,
        rows: usize,
        cols: usize,
        group: usize,
        out: *mut *mut RawWeight,
    ) -> c_int;
    pub fn lx2v_hip_quantize_q4(
        ctx: *mut Ctx,
        src: *const RawBuf,
        rows: usize,
        cols: usize,
        group: usize,
        hqq: c_int,
        out: *mut *mut RawWeight,
    ) -> c_int;
    pub fn lx2v_hip_quantize_fp8_ref(
        ctx: *mut Ctx,
        src: *const RawBuf,
        rows: usize,
        cols: usize,
        group: usize,
        out: *mut *mut RawWeight,
    ) -> c_int;
    pub fn lx2v_hip_weight_export(
        ctx: *mut Ctx,
        w: *const RawWeight,
        codes: *mut c_void,
        codes_bytes: usize,
        scales: *mut c_float,
        zeros: *mut c_float,
    ) -> c_int;

    // ---- norms, residuals, head split
    pub fn lx2v_hip_layer_norm(
        ctx: *mut Ctx,
        x: *const RawBuf,
        rows: usize,
        dim: usize,
        norm: *const lx2v_hip_norm_t,
        mods: *const RawBuf,
        eps: c_float,
        out: *mut RawBuf,
    ) -> c_int;
    pub fn lx2v_hip_residual_norm(
        ctx: *mut Ctx,
        h: *mut RawBuf,
        a: *const RawBuf,
        rows: usize,
        dim: usize,
        mods: *const RawBuf,
        has_gate: c_int,
        gate: usize,
        norm: *const lx2v_hip_norm_t,
        eps: c_float,
        normed: *mut RawBuf,
    ) -> c_int;
    pub fn lx2v_hip_linear_residual(
        ctx: *mut Ctx,
        x: *const RawBuf,
        x_row: usize,
        rows: usize,
        w: *const RawWeight,
        bias: *const RawBuf,
        act: c_int,
        h: *mut RawBuf,
        h_row: usize,
        mods: *const RawBuf,
        gate: usize,
    ) -> c_int;
    pub fn lx2v_hip_gate_residual(
        ctx: *mut Ctx,
        h: *mut RawBuf,
        a: *const RawBuf,
        rows: usize,
        dim: usize,
        mods: *const RawBuf,
        gate: usize,
    ) -> c_int;
    pub fn lx2v_hip_head_split(
        ctx: *mut Ctx,
        src: *const RawBuf,
        rows: usize,
        src_stride: usize,
        col_off: usize,
        heads: usize,
        head_dim: usize,
        rms_w: *const RawBuf,
        rope_cos: *const RawBuf,
        rope_sin: *const RawBuf,
        eps: c_float,
        out: *mut RawBuf,
    ) -> c_int;

    // ---- attention and masks
    pub fn lx2v_hip_attention(
        ctx: *mut Ctx,
        q: *const RawBuf,
        k: *const RawBuf,
        v: *const RawBuf,
        heads: usize,
        sq: usize,
        sk: usize,
        head_dim: usize,
        out: *mut RawBuf,
    ) -> c_int;
    pub fn lx2v_hip_causal_attention(
        ctx: *mut Ctx,
        q: *const RawBuf,
        k: *const RawBuf,
        v: *const RawBuf,
        heads: usize,
        sq: usize,
        sk: usize,
        head_dim: usize,
        mask: *const u8,
        out: *mut RawBuf,
    ) -> c_int;
    pub fn lx2v_hip_mask_upload(
        ctx: *mut Ctx,
        mask: *const u8,
        sq: usize,
        sk: usize,
        out: *mut *mut RawMask,
    ) -> c_int;
    pub fn lx2v_hip_mask_temporal(
        ctx: *mut Ctx,
        tq: *const usize,
        sq: usize,
        tk: *const usize,
        sk: usize,
        out: *mut *mut RawMask,
    ) -> c_int;
    pub fn lx2v_hip_mask_free(ctx: *mut Ctx, mask: *mut RawMask) -> c_int;
    pub fn lx2v_hip_attention_masked(
        ctx: *mut Ctx,
        q: *const RawBuf,
        k: *const RawBuf,
        v: *const RawBuf,
        heads: usize,
        sq: usize,
        sk: usize,
        head_dim: usize,
        mask: *const RawMask,
        out: *mut RawBuf,
    ) -> c_int;

    // ---- KV cache
    pub fn lx2v_hip_kv_cache_new(
        ctx: *mut Ctx,
        heads: usize,
        head_dim: usize,
        capacity_tokens: usize,
        out: *mut *mut RawKv,
    ) -> c_int;
    pub fn lx2v_hip_kv_cache_free(ctx: *mut Ctx, cache: *mut RawKv) -> c_int;
    pub fn lx2v_hip_kv_cache_append(
        ctx: *mut Ctx,
        cache: *mut RawKv,
        k: *const RawBuf,
        v: *const RawBuf,
        rows: usize,
        temporal: *const usize,
    ) -> c_int;
    pub fn lx2v_hip_kv_cache_put(
        ctx: *mut Ctx,
        cache: *mut RawKv,
        k: *const RawBuf,
        v: *const RawBuf,
        rows: usize,
        temporal: *const usize,
    ) -> c_int;
    pub fn lx2v_hip_kv_cache_len(cache: *const RawKv, rows: *mut usize) -> c_int;
    pub fn lx2v_hip_kv_cache_temporal(cache: *const RawKv, out: *mut usize, cap: usize) -> c_int;
    pub fn lx2v_hip_kv_cache_kinds(cache: *const RawKv, out: *mut u8, cap: usize) -> c_int;
    pub fn lx2v_hip_kv_cache_kv(
        ctx: *mut Ctx,
        cache: *const RawKv,
        k: *mut *mut RawBuf,
        v: *mut *mut RawBuf,
    ) -> c_int;
    pub fn lx2v_hip_kv_cache_read(ctx: *mut Ctx, cache: *const RawKv, k: *mut RawBuf, v: *mut RawBuf) -> c_int;
    pub fn lx2v_hip_kv_cache_memrope_update(
        ctx: *mut Ctx,
        cache: *mut RawKv,
        cfg: *const lx2v_hip_memrope_t,
        frame_tokens: usize,
    ) -> c_int;
    pub fn lx2v_hip_kv_cache_attention(
        ctx: *mut Ctx,
        q: *const RawBuf,
        cache: *const RawKv,
        heads: usize,
        sq: usize,
        head_dim: usize,
        mask: *const RawMask,
        out: *mut RawBuf,
    ) -> c_int;

    // ---- synthetic data, quantized activations
    pub fn lx2v_hip_fill_normal(ctx: *mut Ctx, buf: *mut RawBuf, seed: u64, std: c_float) -> c_int;
    pub fn lx2v_hip_alloc_e4m3(ctx: *mut Ctx, rows: usize, cols: usize, out: *mut *mut RawBuf) -> c_int;
    pub fn lx2v_hip_quantize_act(
        ctx: *mut Ctx,
        x: *const RawBuf,
        x_row: usize,
        rows: usize,
        xq: *mut RawBuf,
    ) -> c_int;
    pub fn lx2v_hip_alloc_mx(ctx: *mut Ctx, rows: usize, cols: usize, out: *mut *mut RawBuf) -> c_int;
    pub fn lx2v_hip_quantize_mx(
        ctx: *mut Ctx,
        x: *const RawBuf,
        x_row: usize,
        rows: usize,
        xq: *mut RawBuf,
    ) -> c_int;
    pub fn lx2v_hip_download_mx(ctx: *mut Ctx, buf: *const RawBuf, codes: *mut u8, scales: *mut u8) -> c_int;
    pub fn lx2v_hip_download_e4m3(ctx: *mut Ctx, buf: *const RawBuf, codes: *mut u8, scales: *mut c_float) -> c_int;

    // ---- the linear
    pub fn lx2v_hip_linear(
        ctx: *mut Ctx,
        x: *const RawBuf,
        x_row: usize,
        rows: usize,
        w: *const RawWeight,
        bias: *const RawBuf,
        act: c_int,
        y: *mut RawBuf,
        y_row: usize,
    ) -> c_int;
    pub fn lx2v_hip_linear_noalloc(
        ctx: *mut Ctx,
        x: *const RawBuf,
        x_row: usize,
        rows: usize,
        w: *const RawWeight,
        bias: *const RawBuf,
        act: c_int,
        y: *mut RawBuf,
        y_row: usize,
    ) -> c_int;
    pub fn lx2v_hip_act_quant(
        ctx: *mut Ctx,
        x: *const RawBuf,
        x_row: usize,
        rows: usize,
        cols: usize,
        q: *mut u8,
        s: *mut c_float,
    ) -> c_int;

    // ---- graphs, sync, profiling
    pub fn lx2v_hip_graph_begin(ctx: *mut Ctx) -> c_int;
    pub fn lx2v_hip_graph_end(ctx: *mut Ctx, out: *mut *mut RawGraph) -> c_int;
    pub fn lx2v_hip_graph_launch(ctx: *mut Ctx, g: *const RawGraph) -> c_int;
    pub fn lx2v_hip_graph_free(ctx: *mut Ctx, g: *mut RawGraph) -> c_int;
    pub fn lx2v_hip_sync(ctx: *mut Ctx) -> c_int;
    pub fn lx2v_hip_profile_enable(ctx: *mut Ctx, on: c_int) -> c_int;
    pub fn lx2v_hip_profile_report(ctx: *mut Ctx, out: *mut c_char, cap: usize) -> c_int;
    pub fn lx2v_hip_profile_reset(ctx: *mut Ctx) -> c_int;
    pub fn lx2v_hip_profile_region(ctx: *mut Ctx, name: *const c_char, begin: c_int) -> c_int;
    pub fn lx2v_hip_profile_kernel(
        ctx: *mut Ctx,
        name: *const c_char,
        calls: *mut u64,
        total_ms: *mut c_double,
    ) -> c_int;
}

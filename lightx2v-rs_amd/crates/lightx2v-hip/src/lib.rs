//! lightx2v-hip: the MI355X (gfx950) backend of lightx2v-rs.
//!
//! Implements `lightx2v_core::backend::Backend`
//! (crates/lightx2v-core/src/backend.rs:145-307) over the C ABI of
//! liblightx2v_hip.so (`ffi`).  The quantized-weight linear path (the
//! `weight*` ops and `linear`) runs on hand-written gfx950 kernels: FP8
//! weights on the fp8 matrix cores (per-token e4m3 activations, one scale per
//! channel or per 128 columns), Q8 / Q4 / f32 weights dequantized to bf16 in
//! the GEMM's tile loader on the bf16 matrix cores.  The norms, head split,
//! attention and the MemRoPE KV cache around it run on the device too.  The
//! ops outside that path (sparse attention, patchify / unpatchify, the DMD
//! sampler step, the decoder's conv2d and tanh clamp) have no kernels here:
//! they run on the reference's own CPU backend (lightx2v-cpu) over host
//! copies of their buffers, so `lightx2v check`, `bench` and the pipeline
//! run end to end with `--backend hip` (those ops at CPU speed, plus two
//! host transfers each).
//!
//! Activations are bf16 on the device (the trait leaves activation precision
//! to the backend, backend.rs:9-11); `LIGHTX2V_HIP_ACT=f32` keeps them f32.
//! Tables uploaded with `upload_table` (the RoPE cos / sin) stay f32.
//!
//! Errors: construction is fallible (`try_new` returns `None` when no
//! gfx950 device is visible: the CLI's `skip:` path); every other call
//! panics with the library's message on failure, as the trait's ops panic
//! on misuse.
//!
//! Threading: one context is used by one thread at a time; the backend and
//! its handles may move to another thread (`Send`), as the serve engine
//! moves its backend (crates/lightx2v-cli/src/serve.rs:594-607).  Two
//! backends share no host state.

mod ffi;

use lightx2v_core::{
    backend::{Act, Backend, ConvEpilogue, ConvShape, NormKind},
    config::MemRopeConfig,
    quant::{Fp8E4M3, Q4, Q8},
    sparse::SparseSpec,
};
use lightx2v_cpu::CpuBackend;
use std::ffi::{CStr, CString};
use std::os::raw::c_int;
use std::sync::Arc;

fn check(rc: c_int) {
    if rc != ffi::OK {
        let msg = unsafe { CStr::from_ptr(ffi::lx2v_hip_last_error()) };
        panic!("lightx2v-hip (status {rc}): {}", msg.to_string_lossy());
    }
}

/// The context, destroyed when the backend and every handle made from it
/// are gone.
struct Ctx(*mut ffi::Ctx);
unsafe impl Send for Ctx {}
unsafe impl Sync for Ctx {}
impl Drop for Ctx {
    fn drop(&mut self) {
        unsafe { ffi::lx2v_hip_destroy(self.0) };
    }
}

pub struct HipBackend {
    ctx: Arc<Ctx>,
}

/// A device buffer (F32 or BF16, `len` elements).
pub struct HipBuf {
    ctx: Arc<Ctx>,
    raw: *mut ffi::RawBuf,
}
unsafe impl Send for HipBuf {}
impl Drop for HipBuf {
    fn drop(&mut self) {
        unsafe { ffi::lx2v_hip_buf_free(self.ctx.0, self.raw) };
    }
}

/// A weight in its storage format (f32, Q8, Q4 or FP8 codes and scales in
/// the reference's byte layouts).
pub struct HipWeight {
    ctx: Arc<Ctx>,
    raw: *mut ffi::RawWeight,
}
unsafe impl Send for HipWeight {}
impl Drop for HipWeight {
    fn drop(&mut self) {
        unsafe { ffi::lx2v_hip_weight_free(self.ctx.0, self.raw) };
    }
}

/// One layer's KV cache (K / V head-major on the device, temporal indices
/// and slot kinds on the host side of the library).
pub struct HipKv {
    ctx: Arc<Ctx>,
    raw: *mut ffi::RawKv,
}
unsafe impl Send for HipKv {}
impl Drop for HipKv {
    fn drop(&mut self) {
        unsafe { ffi::lx2v_hip_kv_cache_free(self.ctx.0, self.raw) };
    }
}

impl HipBackend {
    /// Device 0, like `WgpuBackend::try_new` (crates/lightx2v-wgpu/src/lib.rs:
    /// 282-287): `None` when no gfx950 device is visible.
    pub fn try_new() -> Option<Self> {
        Self::try_new_on(0)
    }

    pub fn try_new_on(device: i32) -> Option<Self> {
        let mut raw = std::ptr::null_mut();
        match unsafe { ffi::lx2v_hip_create(device, &mut raw) } {
            ffi::OK => {}
            ffi::ERR_NO_DEVICE => return None,
            rc => check(rc),
        }
        let ctx = Arc::new(Ctx(raw));
        let act = match std::env::var("LIGHTX2V_HIP_ACT").as_deref() {
            Ok("f32") => ffi::DTYPE_F32,
            _ => ffi::DTYPE_BF16,
        };
        check(unsafe { ffi::lx2v_hip_set_act_dtype(ctx.0, act) });
        Some(Self { ctx })
    }

    fn c(&self) -> *mut ffi::Ctx {
        self.ctx.0
    }

    fn buf(&self, raw: *mut ffi::RawBuf) -> HipBuf {
        HipBuf { ctx: self.ctx.clone(), raw }
    }

    fn weight_handle(&self, raw: *mut ffi::RawWeight) -> HipWeight {
        HipWeight { ctx: self.ctx.clone(), raw }
    }

    fn opt(b: Option<&HipBuf>) -> *const ffi::RawBuf {
        b.map_or(std::ptr::null(), |b| b.raw as *const _)
    }

    fn norm(norm: &NormKind<'_, HipBuf>) -> ffi::lx2v_hip_norm_t {
        match *norm {
            NormKind::Affine { w, b } => ffi::lx2v_hip_norm_t {
                kind: ffi::NORM_AFFINE,
                w: w.raw,
                b: b.raw,
                scale: 0,
                shift: 0,
            },
            NormKind::Mod { scale, shift } => ffi::lx2v_hip_norm_t {
                kind: ffi::NORM_MOD,
                w: std::ptr::null(),
                b: std::ptr::null(),
                scale,
                shift,
            },
        }
    }

    fn act(act: Act) -> c_int {
        match act {
            Act::None => ffi::ACT_NONE,
            Act::GeluTanh => ffi::ACT_GELU_TANH,
        }
    }

    // ---- host delegation of the ops outside this backend's path ----------
    // The reference's CPU backend (a unit struct) runs the op on host copies:
    // each input downloaded, the CPU op, then the op's own output extent
    // written back over the start of the device buffer (`write` overwrites
    // a prefix, backend.rs:221-222), the rest of the buffer untouched.
    fn to_cpu(&self, b: &HipBuf) -> <CpuBackend as Backend>::Buf {
        CpuBackend.upload(&self.download(b))
    }

    fn from_cpu(&self, out: &HipBuf, b: &<CpuBackend as Backend>::Buf, n: usize) {
        let v = CpuBackend.download(b);
        self.write(out, &v[..n]);
    }

    /// A weight's dequantized f32 values as a CPU-backend weight.
    fn weight_to_cpu(&self, w: &HipWeight) -> <CpuBackend as Backend>::Weight {
        let mut info = ffi::lx2v_hip_weight_info_t::default();
        check(unsafe { ffi::lx2v_hip_weight_info(w.raw, &mut info) });
        let mut data = vec![0.0f32; info.rows * info.cols];
        check(unsafe { ffi::lx2v_hip_weight_dequantize(self.c(), w.raw, data.as_mut_ptr(), data.len()) });
        CpuBackend.weight(&data, info.rows, info.cols)
    }
}

impl Backend for HipBackend {
    type Buf = HipBuf;
    type Sparse = SparseSpec;
    type Weight = HipWeight;
    type KvCache = HipKv;

    fn name(&self) -> String {
        let mut b = vec![0u8; 256];
        check(unsafe { ffi::lx2v_hip_name(self.c(), b.as_mut_ptr().cast(), b.len()) });
        let n = b.iter().position(|&c| c == 0).unwrap_or(b.len());
        String::from_utf8_lossy(&b[..n]).into_owned()
    }

    // ---- memory ----------------------------------------------------------
    fn alloc(&self, len: usize) -> HipBuf {
        let mut r = std::ptr::null_mut();
        check(unsafe { ffi::lx2v_hip_alloc(self.c(), len, &mut r) });
        self.buf(r)
    }

    fn upload(&self, data: &[f32]) -> HipBuf {
        let mut r = std::ptr::null_mut();
        check(unsafe { ffi::lx2v_hip_upload(self.c(), data.as_ptr(), data.len(), &mut r) });
        self.buf(r)
    }

    fn upload_table(&self, data: &[f32]) -> HipBuf {
        let mut r = std::ptr::null_mut();
        check(unsafe { ffi::lx2v_hip_alloc_dtype(self.c(), data.len(), ffi::DTYPE_F32, &mut r) });
        let b = self.buf(r);
        check(unsafe { ffi::lx2v_hip_write(self.c(), b.raw, data.as_ptr(), data.len()) });
        b
    }

    fn write(&self, buf: &HipBuf, data: &[f32]) {
        check(unsafe { ffi::lx2v_hip_write(self.c(), buf.raw, data.as_ptr(), data.len()) });
    }

    fn download(&self, buf: &HipBuf) -> Vec<f32> {
        let mut out = vec![0.0f32; self.buf_len(buf)];
        check(unsafe { ffi::lx2v_hip_download(self.c(), buf.raw, out.as_mut_ptr(), out.len()) });
        out
    }

    fn buf_len(&self, buf: &HipBuf) -> usize {
        let mut n = 0usize;
        check(unsafe { ffi::lx2v_hip_buf_len(buf.raw, &mut n) });
        n
    }

    fn copy(&self, src: &HipBuf, src_off: usize, dst: &HipBuf, dst_off: usize, len: usize) {
        check(unsafe { ffi::lx2v_hip_copy(self.c(), src.raw, src_off, dst.raw, dst_off, len) });
    }

    fn weight(&self, data: &[f32], rows: usize, cols: usize) -> HipWeight {
        let mut r = std::ptr::null_mut();
        check(unsafe { ffi::lx2v_hip_weight_f32(self.c(), data.as_ptr(), rows, cols, &mut r) });
        self.weight_handle(r)
    }

    fn weight_q8(&self, q: &Q8) -> HipWeight {
        let mut r = std::ptr::null_mut();
        check(unsafe {
            ffi::lx2v_hip_weight_q8(self.c(), q.q.as_ptr(), q.scales.as_ptr(), q.rows, q.cols, q.group, &mut r)
        });
        self.weight_handle(r)
    }

    fn weight_q4(&self, q: &Q4) -> HipWeight {
        // the packed bytes (element 2i in the low nibble, quant.rs:305-311)
        let packed = q.packed();
        let mut r = std::ptr::null_mut();
        check(unsafe {
            ffi::lx2v_hip_weight_q4(
                self.c(),
                packed.as_ptr(),
                1,
                q.scales.as_ptr(),
                q.zeros.as_ptr(),
                q.rows,
                q.cols,
                q.group,
                &mut r,
            )
        });
        self.weight_handle(r)
    }

    fn weight_fp8(&self, q: &Fp8E4M3) -> HipWeight {
        let mut r = std::ptr::null_mut();
        check(unsafe {
            ffi::lx2v_hip_weight_fp8(self.c(), q.q.as_ptr(), q.scales.as_ptr(), q.rows, q.cols, q.group, &mut r)
        });
        self.weight_handle(r)
    }

    fn sync(&self) {
        check(unsafe { ffi::lx2v_hip_sync(self.c()) });
    }

    fn profile_report(&self) -> Option<String> {
        let mut b = vec![0u8; 1 << 16];
        check(unsafe { ffi::lx2v_hip_profile_report(self.c(), b.as_mut_ptr().cast(), b.len()) });
        let n = b.iter().position(|&c| c == 0).unwrap_or(b.len());
        (n > 0).then(|| String::from_utf8_lossy(&b[..n]).into_owned())
    }

    fn profile_reset(&self) {
        check(unsafe { ffi::lx2v_hip_profile_reset(self.c()) });
    }

    // ---- transformer -----------------------------------------------------
    fn linear(
        &self,
        x: &HipBuf,
        x_row: usize,
        rows: usize,
        w: &HipWeight,
        bias: Option<&HipBuf>,
        act: Act,
        y: &HipBuf,
        y_row: usize,
    ) {
        check(unsafe {
            ffi::lx2v_hip_linear(
                self.c(),
                x.raw,
                x_row,
                rows,
                w.raw,
                Self::opt(bias),
                Self::act(act),
                y.raw,
                y_row,
            )
        });
    }

    fn layer_norm(
        &self,
        x: &HipBuf,
        rows: usize,
        dim: usize,
        norm: NormKind<'_, HipBuf>,
        mods: &HipBuf,
        eps: f32,
        out: &HipBuf,
    ) {
        let n = Self::norm(&norm);
        check(unsafe { ffi::lx2v_hip_layer_norm(self.c(), x.raw, rows, dim, &n, mods.raw, eps, out.raw) });
    }

    fn residual_norm(
        &self,
        h: &HipBuf,
        a: &HipBuf,
        rows: usize,
        dim: usize,
        mods: &HipBuf,
        gate: Option<usize>,
        norm: NormKind<'_, HipBuf>,
        eps: f32,
        normed: &HipBuf,
    ) {
        let n = Self::norm(&norm);
        check(unsafe {
            ffi::lx2v_hip_residual_norm(
                self.c(),
                h.raw,
                a.raw,
                rows,
                dim,
                mods.raw,
                gate.is_some() as c_int,
                gate.unwrap_or(0),
                &n,
                eps,
                normed.raw,
            )
        });
    }

    fn gate_residual(&self, h: &HipBuf, a: &HipBuf, rows: usize, dim: usize, mods: &HipBuf, gate: usize) {
        check(unsafe { ffi::lx2v_hip_gate_residual(self.c(), h.raw, a.raw, rows, dim, mods.raw, gate) });
    }

    fn head_split(
        &self,
        src: &HipBuf,
        rows: usize,
        src_stride: usize,
        col_off: usize,
        heads: usize,
        head_dim: usize,
        rms_w: Option<&HipBuf>,
        rope: Option<(&HipBuf, &HipBuf)>,
        eps: f32,
        out: &HipBuf,
    ) {
        let (c, s) = rope.map_or((std::ptr::null(), std::ptr::null()), |(c, s)| {
            (c.raw as *const ffi::RawBuf, s.raw as *const ffi::RawBuf)
        });
        check(unsafe {
            ffi::lx2v_hip_head_split(
                self.c(),
                src.raw,
                rows,
                src_stride,
                col_off,
                heads,
                head_dim,
                Self::opt(rms_w),
                c,
                s,
                eps,
                out.raw,
            )
        });
    }

    fn attention(
        &self,
        q: &HipBuf,
        k: &HipBuf,
        v: &HipBuf,
        heads: usize,
        sq: usize,
        sk: usize,
        head_dim: usize,
        out: &HipBuf,
    ) {
        check(unsafe { ffi::lx2v_hip_attention(self.c(), q.raw, k.raw, v.raw, heads, sq, sk, head_dim, out.raw) });
    }

    fn causal_attention(
        &self,
        q: &HipBuf,
        k: &HipBuf,
        v: &HipBuf,
        heads: usize,
        sq: usize,
        sk: usize,
        head_dim: usize,
        mask: Option<&[bool]>,
        out: &HipBuf,
    ) {
        if let Some(m) = mask {
            assert_eq!(m.len(), sq * sk, "mask is [sq, sk]");
        }
        // bool is one byte, 0 or 1: the library's byte-per-pair mask
        let mp = mask.map_or(std::ptr::null(), |m| m.as_ptr() as *const u8);
        check(unsafe {
            ffi::lx2v_hip_causal_attention(self.c(), q.raw, k.raw, v.raw, heads, sq, sk, head_dim, mp, out.raw)
        });
    }

    // Sparse attention on the CPU backend (host delegation, above); the
    // dense `attention` is this backend's own.
    fn sparse_supported(&self, _head_dim: usize) -> bool {
        true
    }

    fn sparse_prepare(&self, spec: &SparseSpec) -> SparseSpec {
        CpuBackend.sparse_prepare(spec)
    }

    fn sparse_attention(
        &self,
        q: &HipBuf,
        k: &HipBuf,
        v: &HipBuf,
        gate: &HipBuf,
        sparse: &SparseSpec,
        out: &HipBuf,
    ) {
        let (qc, kc, vc, gc) = (self.to_cpu(q), self.to_cpu(k), self.to_cpu(v), self.to_cpu(gate));
        let n = self.buf_len(out);
        let oc = CpuBackend.alloc(n);
        CpuBackend.sparse_attention(&qc, &kc, &vc, &gc, sparse, &oc);
        self.from_cpu(out, &oc, n);
    }

    // ---- KV cache / MemRoPE ----------------------------------------------
    fn kv_cache_new(&self, heads: usize, head_dim: usize, capacity_tokens: usize) -> HipKv {
        let mut r = std::ptr::null_mut();
        check(unsafe { ffi::lx2v_hip_kv_cache_new(self.c(), heads, head_dim, capacity_tokens, &mut r) });
        HipKv { ctx: self.ctx.clone(), raw: r }
    }

    fn kv_cache_append(&self, cache: &mut HipKv, k: &HipBuf, v: &HipBuf, rows: usize, temporal: &[usize]) {
        assert_eq!(temporal.len(), rows, "one temporal index per row");
        check(unsafe { ffi::lx2v_hip_kv_cache_append(self.c(), cache.raw, k.raw, v.raw, rows, temporal.as_ptr()) });
    }

    fn kv_cache_put(&self, cache: &mut HipKv, k: &HipBuf, v: &HipBuf, rows: usize, temporal: &[usize]) {
        assert_eq!(temporal.len(), rows, "one temporal index per row");
        check(unsafe { ffi::lx2v_hip_kv_cache_put(self.c(), cache.raw, k.raw, v.raw, rows, temporal.as_ptr()) });
    }

    fn kv_cache_len(&self, cache: &HipKv) -> usize {
        let mut n = 0usize;
        check(unsafe { ffi::lx2v_hip_kv_cache_len(cache.raw, &mut n) });
        n
    }

    fn kv_cache_temporal(&self, cache: &HipKv) -> Vec<usize> {
        let mut out = vec![0usize; self.kv_cache_len(cache)];
        check(unsafe { ffi::lx2v_hip_kv_cache_temporal(cache.raw, out.as_mut_ptr(), out.len()) });
        out
    }

    fn kv_cache_kv(&self, cache: &HipKv) -> (HipBuf, HipBuf) {
        let (mut k, mut v) = (std::ptr::null_mut(), std::ptr::null_mut());
        check(unsafe { ffi::lx2v_hip_kv_cache_kv(self.c(), cache.raw, &mut k, &mut v) });
        (self.buf(k), self.buf(v))
    }

    fn kv_cache_memrope_update(&self, cache: &mut HipKv, cfg: &MemRopeConfig, frame_tokens: usize) {
        let c = ffi::lx2v_hip_memrope_t {
            cache_frames: cfg.cache_frames,
            sink_frames: cfg.sink_frames,
            ema_alpha_long: cfg.ema_alpha_long,
            ema_alpha_short: cfg.ema_alpha_short,
        };
        check(unsafe { ffi::lx2v_hip_kv_cache_memrope_update(self.c(), cache.raw, &c, frame_tokens) });
    }

    // ---- outside this backend's path: host delegation to the CPU backend ----
    fn patchify(&self, latent: &HipBuf, c: usize, t: usize, h: usize, w: usize, p: usize, out: &HipBuf) {
        let n = t * (h / p) * (w / p) * c * p * p;
        let (lc, oc) = (self.to_cpu(latent), CpuBackend.alloc(n));
        CpuBackend.patchify(&lc, c, t, h, w, p, &oc);
        self.from_cpu(out, &oc, n);
    }

    fn unpatchify(&self, x: &HipBuf, c: usize, t: usize, h: usize, w: usize, p: usize, out: &HipBuf) {
        let n = c * t * h * w;
        let (xc, oc) = (self.to_cpu(x), CpuBackend.alloc(n));
        CpuBackend.unpatchify(&xc, c, t, h, w, p, &oc);
        self.from_cpu(out, &oc, n);
    }

    fn dmd_step(
        &self,
        x: &HipBuf,
        v: &HipBuf,
        noise: Option<&HipBuf>,
        sigma_t: f32,
        sigma_next: f32,
        n: usize,
    ) {
        let (xc, vc) = (self.to_cpu(x), self.to_cpu(v));
        let nc = noise.map(|b| self.to_cpu(b));
        CpuBackend.dmd_step(&xc, &vc, nc.as_ref(), sigma_t, sigma_next, n);
        self.from_cpu(x, &xc, n);
    }

    fn conv2d(
        &self,
        a: &HipBuf,
        b: Option<&HipBuf>,
        shape: &ConvShape,
        w: &HipWeight,
        bias: Option<&HipBuf>,
        epilogue: ConvEpilogue<'_, HipBuf>,
        out: &HipBuf,
    ) {
        let ac = self.to_cpu(a);
        let bc = b.map(|x| self.to_cpu(x));
        let wc = self.weight_to_cpu(w);
        let biasc = bias.map(|x| self.to_cpu(x));
        let ec = match &epilogue {
            ConvEpilogue::AddRelu(r) | ConvEpilogue::Prelu(r) => Some(self.to_cpu(r)),
            _ => None,
        };
        let epi = match epilogue {
            ConvEpilogue::None => ConvEpilogue::None,
            ConvEpilogue::Relu => ConvEpilogue::Relu,
            ConvEpilogue::AddRelu(_) => ConvEpilogue::AddRelu(ec.as_ref().unwrap()),
            ConvEpilogue::Prelu(_) => ConvEpilogue::Prelu(ec.as_ref().unwrap()),
        };
        let n = shape.out_len();
        let oc = CpuBackend.alloc(n);
        CpuBackend.conv2d(&ac, bc.as_ref(), shape, &wc, biasc.as_ref(), epi, &oc);
        self.from_cpu(out, &oc, n);
    }

    fn tanh_clamp(&self, x: &HipBuf, n: usize, s: f32) {
        let xc = self.to_cpu(x);
        CpuBackend.tanh_clamp(&xc, n, s);
        self.from_cpu(x, &xc, n);
    }
}

impl HipBackend {
    /// `linear` followed by `gate_residual(h, y, mods, gate)` in one launch
    /// where the GEMM's epilogue can do the add (bit-identical to the pair).
    #[allow(clippy::too_many_arguments)]
    pub fn linear_residual(
        &self,
        x: &HipBuf,
        x_row: usize,
        rows: usize,
        w: &HipWeight,
        bias: Option<&HipBuf>,
        act: Act,
        h: &HipBuf,
        h_row: usize,
        mods: &HipBuf,
        gate: usize,
    ) {
        check(unsafe {
            ffi::lx2v_hip_linear_residual(
                self.c(),
                x.raw,
                x_row,
                rows,
                w.raw,
                Self::opt(bias),
                Self::act(act),
                h.raw,
                h_row,
                mods.raw,
                gate,
            )
        });
    }

    /// `linear` with no allocation (its workspaces in the library's 48 MiB
    /// per-device scratch): for callers under graph capture or in loops that
    /// must not allocate.  One context at a time holds a device's scratch:
    /// `Err(status)` with `ffi::ERR_BUSY` while another context's work on it
    /// is in flight (nothing was enqueued; retry later); any other failure
    /// panics like `linear`.
    #[allow(clippy::too_many_arguments)]
    pub fn linear_noalloc(
        &self,
        x: &HipBuf,
        x_row: usize,
        rows: usize,
        w: &HipWeight,
        bias: Option<&HipBuf>,
        act: Act,
        y: &HipBuf,
        y_row: usize,
    ) -> Result<(), c_int> {
        let rc = unsafe {
            ffi::lx2v_hip_linear_noalloc(
                self.c(),
                x.raw,
                x_row,
                rows,
                w.raw,
                Self::opt(bias),
                Self::act(act),
                y.raw,
                y_row,
            )
        };
        if rc == ffi::ERR_BUSY {
            return Err(rc);
        }
        check(rc);
        Ok(())
    }

    /// Native f32 weights on the bf16 MFMA through their bf16 copy
    /// (default), or in f32 like the CPU reference (`exact_f32 = true`).
    pub fn set_native_f32(&self, exact_f32: bool) {
        let mode = if exact_f32 { ffi::NATIVE_F32 } else { ffi::NATIVE_BF16 };
        check(unsafe { ffi::lx2v_hip_set_native_mode(self.c(), mode) });
    }

    /// Profile every kernel launch with HIP events (the CPU backend's
    /// LIGHTX2V_PROFILE switch is honoured at creation too).
    pub fn profile_enable(&self, on: bool) {
        check(unsafe { ffi::lx2v_hip_profile_enable(self.c(), on as c_int) });
    }

    /// Time everything enqueued between `region(name, true)` and
    /// `region(name, false)` (reported by `profile_report`).
    pub fn region(&self, name: &str, begin: bool) {
        let n = CString::new(name).expect("region name without NUL");
        check(unsafe { ffi::lx2v_hip_profile_region(self.c(), n.as_ptr(), begin as c_int) });
    }
}

#[cfg(test)]
mod tests {
    //! Against the CPU reference backend on the same inputs (as
    //! crates/lightx2v-wgpu/tests/conformance.rs does); skipped without a
    //! gfx950 device.
    use super::*;
    use lightx2v_core::rng::Rng;
    use lightx2v_cpu::CpuBackend;

    fn rel_l2(a: &[f32], b: &[f32]) -> f64 {
        let num: f64 = a.iter().zip(b).map(|(x, y)| ((x - y) as f64).powi(2)).sum();
        let den: f64 = b.iter().map(|y| (*y as f64).powi(2)).sum();
        (num / den.max(1e-30)).sqrt()
    }

    #[test]
    fn fp8_linear_matches_cpu() {
        let Some(hip) = HipBackend::try_new() else {
            eprintln!("skip: no gfx950 device");
            return;
        };
        let cpu = CpuBackend;
        let (m, k, n) = (200, 1536, 384);
        let x = Rng::new(1001).normal(m * k);
        let w: Vec<f32> = Rng::new(1002).normal(n * k).iter().map(|v| v * 0.02).collect();
        let b: Vec<f32> = Rng::new(1003).normal(n).iter().map(|v| v * 0.01).collect();
        let q = Fp8E4M3::quantize(&w, n, k);
        let y_cpu = {
            let (xb, bb, yb) = (cpu.upload(&x), cpu.upload(&b), cpu.alloc(m * n));
            cpu.linear(&xb, 0, m, &cpu.weight_fp8(&q), Some(&bb), Act::GeluTanh, &yb, 0);
            cpu.download(&yb)
        };
        let y_hip = {
            let (xb, bb, yb) = (hip.upload(&x), hip.upload(&b), hip.alloc(m * n));
            hip.linear(&xb, 0, m, &hip.weight_fp8(&q), Some(&bb), Act::GeluTanh, &yb, 0);
            hip.download(&yb)
        };
        // e4m3 activations (3 mantissa bits) against the f32 reference
        assert!(rel_l2(&y_hip, &y_cpu) < 4e-2);
    }
}

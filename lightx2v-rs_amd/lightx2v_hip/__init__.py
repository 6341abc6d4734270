"""Python binding of the gfx950 quantized-linear backend (liblightx2v_hip.so).

``HipBackend`` mirrors the lightx2v-rs ``Backend`` trait's linear path
(crates/lightx2v-core/src/backend.rs:145-212) method for method, over the C
ABI declared in include/lightx2v_hip.h, the same surface a ``lightx2v-hip``
Rust crate binds.  Misuse raises ``HipError`` (the trait panics);
``HipBackend.try_new`` returns None when no gfx950 device answers, like
``WgpuBackend::try_new`` (crates/lightx2v-wgpu/src/lib.rs:282-287).

There is no fallback: if the shared library is missing, importing this module
raises, and every op runs the library's HIP kernels.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblightx2v_hip.so")

OK, ERR_NO_DEVICE, ERR_BAD_SHAPE, ERR_ALIAS, ERR_HIP, ERR_BAD_ARG, ERR_OOM, ERR_UNSUPPORTED, ERR_BUSY = range(9)
ACT_NONE, ACT_GELU_TANH = 0, 1
DTYPE_F32, DTYPE_BF16, DTYPE_E4M3, DTYPE_MXE4M3 = 0, 1, 2, 3
WFMT_F32, WFMT_Q8, WFMT_Q4, WFMT_FP8 = 0, 1, 2, 3
FP8_ACT_E4M3, FP8_ACT_BF16 = 0, 1
NATIVE_BF16, NATIVE_F32 = 0, 1

# Every entry point include/lightx2v_hip.h declares (checked by the tests).
EXPORTS = [
    "lx2v_hip_last_error", "lx2v_hip_device_count", "lx2v_hip_create", "lx2v_hip_destroy",
    "lx2v_hip_name", "lx2v_hip_set_act_dtype", "lx2v_hip_set_fp8_act", "lx2v_hip_set_native_mode", "lx2v_hip_alloc",
    "lx2v_hip_alloc_dtype", "lx2v_hip_upload", "lx2v_hip_write", "lx2v_hip_download",
    "lx2v_hip_buf_len", "lx2v_hip_buf_dtype", "lx2v_hip_copy", "lx2v_hip_buf_free",
    "lx2v_hip_weight_f32", "lx2v_hip_weight_q8", "lx2v_hip_weight_q4", "lx2v_hip_weight_fp8",
    "lx2v_hip_weight_free", "lx2v_hip_weight_info", "lx2v_hip_weight_dequantize",
    "lx2v_hip_quantize_q8", "lx2v_hip_quantize_q4_sym", "lx2v_hip_quantize_fp8",
    "lx2v_hip_fill_normal", "lx2v_hip_linear", "lx2v_hip_act_quant", "lx2v_hip_sync",
    "lx2v_hip_profile_enable", "lx2v_hip_profile_report", "lx2v_hip_profile_reset",
    "lx2v_hip_profile_kernel", "lx2v_hip_alloc_e4m3", "lx2v_hip_quantize_act", "lx2v_hip_graph_begin",
    "lx2v_hip_graph_end", "lx2v_hip_graph_launch", "lx2v_hip_graph_free", "lx2v_hip_profile_region",
    "lx2v_hip_alloc_mx", "lx2v_hip_quantize_mx", "lx2v_hip_download_mx",
    "lx2v_hip_quantize_q4", "lx2v_hip_quantize_fp8_ref", "lx2v_hip_weight_export",
    "lx2v_hip_layer_norm", "lx2v_hip_residual_norm", "lx2v_hip_gate_residual", "lx2v_hip_download_e4m3",
    "lx2v_hip_attention", "lx2v_hip_causal_attention", "lx2v_hip_mask_upload", "lx2v_hip_mask_free",
    "lx2v_hip_attention_masked", "lx2v_hip_kv_cache_new", "lx2v_hip_kv_cache_free", "lx2v_hip_kv_cache_append",
    "lx2v_hip_kv_cache_put", "lx2v_hip_kv_cache_len", "lx2v_hip_kv_cache_temporal", "lx2v_hip_kv_cache_kinds",
    "lx2v_hip_kv_cache_kv", "lx2v_hip_kv_cache_read", "lx2v_hip_kv_cache_memrope_update",
    "lx2v_hip_kv_cache_attention", "lx2v_hip_mask_temporal", "lx2v_hip_linear_residual", "lx2v_hip_head_split",
    "lx2v_hip_linear_noalloc",
]


class HipError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"lightx2v-hip status {status}: {msg}")
        self.status = status


NORM_AFFINE, NORM_MOD = 0, 1

# SlotKind (crates/lightx2v-core/src/memrope.rs:31-37)
SLOT_SINK, SLOT_LONG_EMA, SLOT_SHORT_EMA, SLOT_RECENT, SLOT_NEW = range(5)


class MemRopeConfig(ctypes.Structure):
    """The MemRopeConfig fields the cache update reads (config.rs:265-295;
    defaults = default_memrope())."""

    _fields_ = [("cache_frames", ctypes.c_size_t), ("sink_frames", ctypes.c_size_t),
                ("ema_alpha_long", ctypes.c_float), ("ema_alpha_short", ctypes.c_float)]

    def __init__(self, cache_frames=12, sink_frames=3, ema_alpha_long=0.01, ema_alpha_short=0.1):
        super().__init__(cache_frames, sink_frames, ema_alpha_long, ema_alpha_short)


class _Norm(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("w", ctypes.c_void_p), ("b", ctypes.c_void_p),
                ("scale", ctypes.c_size_t), ("shift", ctypes.c_size_t)]


class NormKind:
    """``NormKind`` (backend.rs:47-52): ``affine(w, b)`` is LN(x) * w + b,
    ``mod(scale, shift)`` is LN(x) * (1 + mods[scale]) + mods[shift]."""

    def __init__(self, kind: int, w=None, b=None, scale: int = 0, shift: int = 0):
        self.kind, self.w, self.b, self.scale, self.shift = kind, w, b, scale, shift

    @staticmethod
    def affine(w: "Buf", b: "Buf") -> "NormKind":
        return NormKind(NORM_AFFINE, w=w, b=b)

    @staticmethod
    def mod(scale: int, shift: int) -> "NormKind":
        return NormKind(NORM_MOD, scale=scale, shift=shift)

    def _c(self) -> _Norm:
        return _Norm(self.kind, self.w.h if self.w is not None else None, self.b.h if self.b is not None else None,
                     self.scale, self.shift)


class _WeightInfo(ctypes.Structure):
    _fields_ = [("fmt", ctypes.c_int), ("rows", ctypes.c_size_t), ("cols", ctypes.c_size_t),
                ("group", ctypes.c_size_t), ("device_bytes", ctypes.c_size_t),
                ("canonicalized", ctypes.c_size_t)]


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built (run __graft_entry__.build() or make -C lightx2v-rs_amd)")
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, ip = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    pp = ctypes.POINTER(ctypes.c_void_p)
    sig = {
        "lx2v_hip_last_error": (ctypes.c_char_p, []),
        "lx2v_hip_device_count": (ip, [ctypes.POINTER(ctypes.c_int)]),
        "lx2v_hip_create": (ip, [ip, pp]),
        "lx2v_hip_destroy": (ip, [vp]),
        "lx2v_hip_name": (ip, [vp, ctypes.c_char_p, sz]),
        "lx2v_hip_set_act_dtype": (ip, [vp, ip]),
        "lx2v_hip_set_fp8_act": (ip, [vp, ip]),
        "lx2v_hip_set_native_mode": (ip, [vp, ip]),
        "lx2v_hip_alloc": (ip, [vp, sz, pp]),
        "lx2v_hip_alloc_dtype": (ip, [vp, sz, ip, pp]),
        "lx2v_hip_upload": (ip, [vp, vp, sz, pp]),
        "lx2v_hip_write": (ip, [vp, vp, vp, sz]),
        "lx2v_hip_download": (ip, [vp, vp, vp, sz]),
        "lx2v_hip_buf_len": (ip, [vp, ctypes.POINTER(ctypes.c_size_t)]),
        "lx2v_hip_buf_dtype": (ip, [vp, ctypes.POINTER(ctypes.c_int)]),
        "lx2v_hip_copy": (ip, [vp, vp, sz, vp, sz, sz]),
        "lx2v_hip_buf_free": (ip, [vp, vp]),
        "lx2v_hip_weight_f32": (ip, [vp, vp, sz, sz, pp]),
        "lx2v_hip_weight_q8": (ip, [vp, vp, vp, sz, sz, sz, pp]),
        "lx2v_hip_weight_q4": (ip, [vp, vp, ip, vp, vp, sz, sz, sz, pp]),
        "lx2v_hip_weight_fp8": (ip, [vp, vp, vp, sz, sz, sz, pp]),
        "lx2v_hip_weight_free": (ip, [vp, vp]),
        "lx2v_hip_weight_info": (ip, [vp, ctypes.POINTER(_WeightInfo)]),
        "lx2v_hip_weight_dequantize": (ip, [vp, vp, vp, sz]),
        "lx2v_hip_quantize_q8": (ip, [vp, vp, sz, sz, sz, pp]),
        "lx2v_hip_quantize_q4_sym": (ip, [vp, vp, sz, sz, sz, pp]),
        "lx2v_hip_quantize_fp8": (ip, [vp, vp, sz, sz, sz, pp]),
        "lx2v_hip_quantize_q4": (ip, [vp, vp, sz, sz, sz, ip, pp]),
        "lx2v_hip_quantize_fp8_ref": (ip, [vp, vp, sz, sz, sz, pp]),
        "lx2v_hip_weight_export": (ip, [vp, vp, vp, sz, vp, vp]),
        "lx2v_hip_layer_norm": (ip, [vp, vp, sz, sz, ctypes.POINTER(_Norm), vp, ctypes.c_float, vp]),
        "lx2v_hip_residual_norm": (ip, [vp, vp, vp, sz, sz, vp, ip, sz, ctypes.POINTER(_Norm), ctypes.c_float,
                                        vp]),
        "lx2v_hip_gate_residual": (ip, [vp, vp, vp, sz, sz, vp, sz]),
        "lx2v_hip_head_split": (ip, [vp, vp, sz, sz, sz, sz, sz, vp, vp, vp, ctypes.c_float, vp]),
        "lx2v_hip_linear_noalloc": (ip, [vp, vp, sz, sz, vp, vp, ip, vp, sz]),
        "lx2v_hip_attention": (ip, [vp, vp, vp, vp, sz, sz, sz, sz, vp]),
        "lx2v_hip_causal_attention": (ip, [vp, vp, vp, vp, sz, sz, sz, sz, vp, vp]),
        "lx2v_hip_mask_upload": (ip, [vp, vp, sz, sz, pp]),
        "lx2v_hip_mask_free": (ip, [vp, vp]),
        "lx2v_hip_mask_temporal": (ip, [vp, vp, sz, vp, sz, pp]),
        "lx2v_hip_attention_masked": (ip, [vp, vp, vp, vp, sz, sz, sz, sz, vp, vp]),
        "lx2v_hip_kv_cache_new": (ip, [vp, sz, sz, sz, pp]),
        "lx2v_hip_kv_cache_free": (ip, [vp, vp]),
        "lx2v_hip_kv_cache_append": (ip, [vp, vp, vp, vp, sz, vp]),
        "lx2v_hip_kv_cache_put": (ip, [vp, vp, vp, vp, sz, vp]),
        "lx2v_hip_kv_cache_len": (ip, [vp, ctypes.POINTER(ctypes.c_size_t)]),
        "lx2v_hip_kv_cache_temporal": (ip, [vp, vp, sz]),
        "lx2v_hip_kv_cache_kinds": (ip, [vp, vp, sz]),
        "lx2v_hip_kv_cache_kv": (ip, [vp, vp, pp, pp]),
        "lx2v_hip_kv_cache_read": (ip, [vp, vp, vp, vp]),
        "lx2v_hip_kv_cache_memrope_update": (ip, [vp, vp, ctypes.POINTER(MemRopeConfig), sz]),
        "lx2v_hip_kv_cache_attention": (ip, [vp, vp, vp, sz, sz, sz, vp, vp]),
        "lx2v_hip_fill_normal": (ip, [vp, vp, ctypes.c_uint64, ctypes.c_float]),
        "lx2v_hip_linear": (ip, [vp, vp, sz, sz, vp, vp, ip, vp, sz]),
        "lx2v_hip_linear_residual": (ip, [vp, vp, sz, sz, vp, vp, ip, vp, sz, vp, sz]),
        "lx2v_hip_act_quant": (ip, [vp, vp, sz, sz, sz, vp, vp]),
        "lx2v_hip_sync": (ip, [vp]),
        "lx2v_hip_profile_enable": (ip, [vp, ip]),
        "lx2v_hip_profile_report": (ip, [vp, ctypes.c_char_p, sz]),
        "lx2v_hip_profile_reset": (ip, [vp]),
        "lx2v_hip_profile_kernel": (ip, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64),
                                         ctypes.POINTER(ctypes.c_double)]),
        "lx2v_hip_alloc_e4m3": (ip, [vp, sz, sz, pp]),
        "lx2v_hip_quantize_act": (ip, [vp, vp, sz, sz, vp]),
        "lx2v_hip_alloc_mx": (ip, [vp, sz, sz, pp]),
        "lx2v_hip_quantize_mx": (ip, [vp, vp, sz, sz, vp]),
        "lx2v_hip_download_mx": (ip, [vp, vp, vp, vp]),
        "lx2v_hip_download_e4m3": (ip, [vp, vp, vp, vp]),
        "lx2v_hip_graph_begin": (ip, [vp]),
        "lx2v_hip_graph_end": (ip, [vp, pp]),
        "lx2v_hip_graph_launch": (ip, [vp, vp]),
        "lx2v_hip_graph_free": (ip, [vp, vp]),
        "lx2v_hip_profile_region": (ip, [vp, ctypes.c_char_p, ip]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


lib = _load()


def _check(rc: int):
    if rc != OK:
        raise HipError(rc, lib.lx2v_hip_last_error().decode())


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(lib.lx2v_hip_device_count(ctypes.byref(n)))
    return n.value


class Buf:
    """The trait's ``Buf``: a flat device buffer of activations."""

    def __init__(self, be: "HipBackend", h: int):
        self._be, self.h = be, h

    def __len__(self) -> int:
        n = ctypes.c_size_t(0)
        _check(lib.lx2v_hip_buf_len(self.h, ctypes.byref(n)))
        return n.value

    @property
    def dtype(self) -> int:
        d = ctypes.c_int(0)
        _check(lib.lx2v_hip_buf_dtype(self.h, ctypes.byref(d)))
        return d.value

    def free(self):
        if self.h and self._be.ctx:
            lib.lx2v_hip_buf_free(self._be.ctx, self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    """The trait's ``Weight``: a quantized (or f32) matrix resident in HBM."""

    def __init__(self, be: "HipBackend", h: int):
        self._be, self.h = be, h

    def info(self) -> dict:
        i = _WeightInfo()
        _check(lib.lx2v_hip_weight_info(self.h, ctypes.byref(i)))
        return {f: getattr(i, f) for f, _ in _WeightInfo._fields_}

    def free(self):
        if self.h and self._be.ctx:
            lib.lx2v_hip_weight_free(self._be.ctx, self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Mask:
    """A [sq, sk] attention mask resident in HBM (with its tile summary)."""

    def __init__(self, be: "HipBackend", h: int, sq: int, sk: int):
        self._be, self.h, self.sq, self.sk = be, h, sq, sk

    def free(self):
        if self.h and self._be.ctx:
            lib.lx2v_hip_mask_free(self._be.ctx, self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class KvCache:
    """One layer's KV cache (the trait's ``KvCache``, backend.rs:333-392):
    K / V rows in HBM, temporal index and slot kind per row on the host."""

    def __init__(self, be: "HipBackend", h: int, heads: int, head_dim: int):
        self._be, self.h, self.heads, self.head_dim = be, h, heads, head_dim

    @staticmethod
    def _temporal(temporal, rows: int) -> np.ndarray:
        t = np.ascontiguousarray(temporal, np.uint64).ravel()
        if t.size != rows:
            raise HipError(ERR_BAD_SHAPE, f"{t.size} temporal indices for {rows} rows")
        return t

    def append(self, k: Buf, v: Buf, rows: int, temporal):
        t = self._temporal(temporal, rows)
        _check(lib.lx2v_hip_kv_cache_append(self._be.ctx, self.h, k.h, v.h, rows, _ptr(t)))

    def put(self, k: Buf, v: Buf, rows: int, temporal):
        t = self._temporal(temporal, rows)
        _check(lib.lx2v_hip_kv_cache_put(self._be.ctx, self.h, k.h, v.h, rows, _ptr(t)))

    def __len__(self) -> int:
        n = ctypes.c_size_t(0)
        _check(lib.lx2v_hip_kv_cache_len(self.h, ctypes.byref(n)))
        return n.value

    def temporal(self) -> list:
        t = np.zeros(len(self), np.uint64)
        _check(lib.lx2v_hip_kv_cache_temporal(self.h, _ptr(t), t.size))
        return [int(x) for x in t]

    def kinds(self) -> list:
        k = np.zeros(len(self), np.uint8)
        _check(lib.lx2v_hip_kv_cache_kinds(self.h, _ptr(k), k.size))
        return [int(x) for x in k]

    def kv(self):
        """(K, V) as new [heads, rows, head_dim] buffers in the cache's dtype."""
        kh, vh = ctypes.c_void_p(), ctypes.c_void_p()
        _check(lib.lx2v_hip_kv_cache_kv(self._be.ctx, self.h, ctypes.byref(kh), ctypes.byref(vh)))
        return Buf(self._be, kh.value), Buf(self._be, vh.value)

    def read(self, k: Buf, v: Buf):
        _check(lib.lx2v_hip_kv_cache_read(self._be.ctx, self.h, k.h, v.h))

    def memrope_update(self, cfg: MemRopeConfig, frame_tokens: int):
        _check(lib.lx2v_hip_kv_cache_memrope_update(self._be.ctx, self.h, ctypes.byref(cfg), frame_tokens))

    def attention(self, q: Buf, sq: int, mask: Optional[Mask], out: Buf):
        """causal_attention of q [heads, sq, d] over every cached row, in place."""
        _check(lib.lx2v_hip_kv_cache_attention(self._be.ctx, q.h, self.h, self.heads, sq, self.head_dim,
                                               mask.h if mask is not None else None, out.h))

    def free(self):
        if self.h and self._be.ctx:
            lib.lx2v_hip_kv_cache_free(self._be.ctx, self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Graph:
    """A captured sequence of device work, replayed with one launch."""

    def __init__(self, be: "HipBackend", h: int):
        self._be, self.h = be, h

    def launch(self):
        _check(lib.lx2v_hip_graph_launch(self._be.ctx, self.h))

    def free(self):
        if self.h and self._be.ctx:
            lib.lx2v_hip_graph_free(self._be.ctx, self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipBackend:
    """lightx2v-rs ``Backend`` (linear path) on one gfx950 device."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_create(device, ctypes.byref(h)))
        self.ctx = h.value
        self.act_dtype = DTYPE_F32  # the context's default (lx2v_hip_create)

    @classmethod
    def try_new(cls, device: int = 0) -> Optional["HipBackend"]:
        try:
            return cls(device)
        except HipError as e:
            if e.status == ERR_NO_DEVICE:
                return None
            raise

    def close(self):
        if self.ctx:
            lib.lx2v_hip_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- backend.rs:158-196 ----
    def name(self) -> str:
        b = ctypes.create_string_buffer(256)
        _check(lib.lx2v_hip_name(self.ctx, b, 256))
        return b.value.decode()

    def set_act_dtype(self, dtype: int):
        _check(lib.lx2v_hip_set_act_dtype(self.ctx, dtype))
        self.act_dtype = dtype

    def set_fp8_act(self, mode: int):
        _check(lib.lx2v_hip_set_fp8_act(self.ctx, mode))

    def set_native_mode(self, mode: int):
        """NATIVE_BF16 (default): native f32 weights through their bf16 copy on
        the bf16 MFMA; NATIVE_F32: f32 operands (the scalar kernel)."""
        _check(lib.lx2v_hip_set_native_mode(self.ctx, mode))

    def _out(self):
        return ctypes.c_void_p()

    def alloc(self, n: int, dtype: Optional[int] = None) -> Buf:
        h = ctypes.c_void_p()
        if dtype is None:
            _check(lib.lx2v_hip_alloc(self.ctx, n, ctypes.byref(h)))
        else:
            _check(lib.lx2v_hip_alloc_dtype(self.ctx, n, dtype, ctypes.byref(h)))
        return Buf(self, h.value)

    def upload(self, data) -> Buf:
        a = np.ascontiguousarray(data, np.float32).ravel()
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_upload(self.ctx, _ptr(a), a.size, ctypes.byref(h)))
        return Buf(self, h.value)

    def write(self, buf: Buf, data):
        a = np.ascontiguousarray(data, np.float32).ravel()
        _check(lib.lx2v_hip_write(self.ctx, buf.h, _ptr(a), a.size))

    def download(self, buf: Buf) -> np.ndarray:
        out = np.empty(len(buf), np.float32)
        _check(lib.lx2v_hip_download(self.ctx, buf.h, _ptr(out), out.size))
        return out

    def buf_len(self, buf: Buf) -> int:
        return len(buf)

    def copy(self, src: Buf, src_off: int, dst: Buf, dst_off: int, n: int):
        _check(lib.lx2v_hip_copy(self.ctx, src.h, src_off, dst.h, dst_off, n))

    def weight(self, data, rows: int, cols: int) -> Weight:
        a = np.ascontiguousarray(data, np.float32).ravel()
        if a.size != rows * cols:
            raise HipError(ERR_BAD_SHAPE, f"weight has {a.size} elements, {rows}x{cols} expected")
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_weight_f32(self.ctx, _ptr(a), rows, cols, ctypes.byref(h)))
        return Weight(self, h.value)

    def weight_q8(self, q, scales, rows: int, cols: int, group: int) -> Weight:
        qa = np.ascontiguousarray(q, np.int8).ravel()
        sa = np.ascontiguousarray(scales, np.float32).ravel()
        if qa.size != rows * cols or sa.size != rows * cols // group:
            raise HipError(ERR_BAD_SHAPE, "q8 codes/scales do not match the shape")
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_weight_q8(self.ctx, _ptr(qa), _ptr(sa), rows, cols, group, ctypes.byref(h)))
        return Weight(self, h.value)

    def weight_q4(self, codes, scales, zeros, rows: int, cols: int, group: int,
                  packed: bool = False) -> Weight:
        ca = np.ascontiguousarray(codes, np.uint8).ravel()
        sa = np.ascontiguousarray(scales, np.float32).ravel()
        za = np.ascontiguousarray(zeros, np.float32).ravel()
        need = (rows * cols + 1) // 2 if packed else rows * cols
        if ca.size != need or sa.size != rows * cols // group or za.size != sa.size:
            raise HipError(ERR_BAD_SHAPE, "q4 codes/scales/zeros do not match the shape")
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_weight_q4(self.ctx, _ptr(ca), int(packed), _ptr(sa), _ptr(za), rows, cols,
                                      group, ctypes.byref(h)))
        return Weight(self, h.value)

    def weight_fp8(self, q, scales, rows: int, cols: int, group: int) -> Weight:
        qa = np.ascontiguousarray(q, np.uint8).ravel()
        sa = np.ascontiguousarray(scales, np.float32).ravel()
        if qa.size != rows * cols or sa.size != rows * cols // group:
            raise HipError(ERR_BAD_SHAPE, "fp8 codes/scales do not match the shape")
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_weight_fp8(self.ctx, _ptr(qa), _ptr(sa), rows, cols, group, ctypes.byref(h)))
        return Weight(self, h.value)

    def dequantize(self, w: Weight) -> np.ndarray:
        i = w.info()
        out = np.empty(i["rows"] * i["cols"], np.float32)
        _check(lib.lx2v_hip_weight_dequantize(self.ctx, w.h, _ptr(out), out.size))
        return out.reshape(i["rows"], i["cols"])

    def quantize_q8(self, src: Buf, rows: int, cols: int, group: int) -> Weight:
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_quantize_q8(self.ctx, src.h, rows, cols, group, ctypes.byref(h)))
        return Weight(self, h.value)

    def quantize_q4_sym(self, src: Buf, rows: int, cols: int, group: int) -> Weight:
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_quantize_q4_sym(self.ctx, src.h, rows, cols, group, ctypes.byref(h)))
        return Weight(self, h.value)

    def quantize_fp8(self, src: Buf, rows: int, cols: int, group: int) -> Weight:
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_quantize_fp8(self.ctx, src.h, rows, cols, group, ctypes.byref(h)))
        return Weight(self, h.value)

    def quantize_q4(self, src: Buf, rows: int, cols: int, group: int, hqq: bool) -> Weight:
        """Q4::quantize (quant.rs:226-292) on the device: affine, optional HQQ, f16 scale / zero."""
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_quantize_q4(self.ctx, src.h, rows, cols, group, int(bool(hqq)), ctypes.byref(h)))
        return Weight(self, h.value)

    def quantize_fp8_ref(self, src: Buf, rows: int, cols: int, group: int) -> Weight:
        """Fp8E4M3::quantize (quant.rs:423-447) with the reference's encoder, verbatim."""
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_quantize_fp8_ref(self.ctx, src.h, rows, cols, group, ctypes.byref(h)))
        return Weight(self, h.value)

    def weight_export(self, w: Weight) -> dict:
        """The weight in the reference's host layouts: ``q`` (Q8 int8 [rows, cols], Q4 packed
        uint8 [rows, cols / 2], FP8 the reference's code bytes [rows, cols], F32 values),
        ``scales`` / ``zeros`` f32 [rows, cols / group]."""
        i = w.info()
        rows, cols, fmt = i["rows"], i["cols"], i["fmt"]
        if fmt == WFMT_F32:
            q = np.empty((rows, cols), np.float32)
        elif fmt == WFMT_Q4:
            q = np.empty((rows * cols + 1) // 2, np.uint8)
        else:
            q = np.empty((rows, cols), np.int8 if fmt == WFMT_Q8 else np.uint8)
        ng = cols // i["group"] if fmt != WFMT_F32 else 0
        s = np.empty((rows, ng), np.float32)
        z = np.empty((rows, ng), np.float32)
        _check(lib.lx2v_hip_weight_export(self.ctx, w.h, _ptr(q), q.nbytes, _ptr(s) if ng else None,
                                          _ptr(z) if fmt == WFMT_Q4 else None))
        if fmt == WFMT_Q4 and cols % 2 == 0:
            q = q.reshape(rows, cols // 2)
        out = {"fmt": fmt, "rows": rows, "cols": cols, "group": i["group"], "q": q}
        if fmt != WFMT_F32:
            out["scales"] = s
        if fmt == WFMT_Q4:
            out["zeros"] = z
        return out

    def fill_normal(self, buf: Buf, seed: int, std: float):
        _check(lib.lx2v_hip_fill_normal(self.ctx, buf.h, ctypes.c_uint64(seed), ctypes.c_float(std)))

    def linear(self, x: Buf, x_row: int, rows: int, w: Weight, bias: Optional[Buf], act: int,
               y: Buf, y_row: int):
        _check(lib.lx2v_hip_linear(self.ctx, x.h, x_row, rows, w.h, bias.h if bias else None, act, y.h,
                                   y_row))

    def linear_noalloc(self, x: Buf, x_row: int, rows: int, w: Weight, bias: Optional[Buf], act: int, y: Buf,
                       y_row: int):
        """lx2v_hip_linear_noalloc: linear with its workspaces in the device scratch."""
        _check(lib.lx2v_hip_linear_noalloc(self.ctx, x.h, x_row, rows, w.h, bias.h if bias is not None else None,
                                           act, y.h, y_row))

    def linear_residual(self, x: Buf, x_row: int, rows: int, w: Weight, bias: Optional[Buf], act: int, h: Buf,
                        h_row: int, mods: Buf, gate: int):
        """h[h_row + r] += act(x W^T + b)[r] * mods[gate]: linear then gate_residual, fused on the FP8 path."""
        _check(lib.lx2v_hip_linear_residual(self.ctx, x.h, x_row, rows, w.h, bias.h if bias else None, act, h.h,
                                            h_row, mods.h, gate))

    # ---- backend.rs:214-252: the norms around the linears ----
    def layer_norm(self, x: Buf, rows: int, dim: int, norm: NormKind, mods: Optional[Buf], eps: float, out: Buf):
        """out = norm(x); ``out`` may be E4M3 / MXE4M3 (the next FP8 linear's input)."""
        n = norm._c()
        _check(lib.lx2v_hip_layer_norm(self.ctx, x.h, rows, dim, ctypes.byref(n), mods.h if mods else None,
                                       ctypes.c_float(eps), out.h))

    def residual_norm(self, h: Buf, a: Buf, rows: int, dim: int, mods: Optional[Buf], gate: Optional[int],
                      norm: NormKind, eps: float, normed: Buf):
        """h += a * mods[gate] (gate None: h += a), then normed = norm(h)."""
        n = norm._c()
        _check(lib.lx2v_hip_residual_norm(self.ctx, h.h, a.h, rows, dim, mods.h if mods else None,
                                          int(gate is not None), gate or 0, ctypes.byref(n), ctypes.c_float(eps),
                                          normed.h))

    def gate_residual(self, h: Buf, a: Buf, rows: int, dim: int, mods: Buf, gate: int):
        """h += a * mods[gate]."""
        _check(lib.lx2v_hip_gate_residual(self.ctx, h.h, a.h, rows, dim, mods.h, gate))

    # ---- backend.rs:273-305: attention ----
    def head_split(self, src: Buf, rows: int, src_stride: int, col_off: int, heads: int, head_dim: int,
                   rms_w: Optional[Buf], rope: Optional[tuple], eps: float, out: Buf):
        """Backend::head_split: rope = (cos, sin) buffers or None."""
        c, s = rope if rope is not None else (None, None)
        _check(lib.lx2v_hip_head_split(self.ctx, src.h, rows, src_stride, col_off, heads, head_dim,
                                       rms_w.h if rms_w is not None else None, c.h if c is not None else None,
                                       s.h if s is not None else None, ctypes.c_float(eps), out.h))

    def attention(self, q: Buf, k: Buf, v: Buf, heads: int, sq: int, sk: int, head_dim: int, out: Buf):
        """q [heads, sq, d], k / v [heads, sk, d] -> out [sq, heads * d]."""
        _check(lib.lx2v_hip_attention(self.ctx, q.h, k.h, v.h, heads, sq, sk, head_dim, out.h))

    def causal_attention(self, q: Buf, k: Buf, v: Buf, heads: int, sq: int, sk: int, head_dim: int, mask,
                         out: Buf):
        """``mask``: host [sq, sk] bool array (True = allowed), a resident ``Mask``, or None."""
        if isinstance(mask, Mask):
            _check(lib.lx2v_hip_attention_masked(self.ctx, q.h, k.h, v.h, heads, sq, sk, head_dim, mask.h, out.h))
            return
        m = None if mask is None else np.ascontiguousarray(mask, np.uint8).ravel()
        if m is not None and m.size != sq * sk:
            raise HipError(ERR_BAD_SHAPE, f"mask has {m.size} entries, {sq}x{sk} expected")
        _check(lib.lx2v_hip_causal_attention(self.ctx, q.h, k.h, v.h, heads, sq, sk, head_dim,
                                             None if m is None else _ptr(m), out.h))

    def mask_upload(self, mask, sq: int, sk: int) -> Mask:
        m = np.ascontiguousarray(mask, np.uint8).ravel()
        if m.size != sq * sk:
            raise HipError(ERR_BAD_SHAPE, f"mask has {m.size} entries, {sq}x{sk} expected")
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_mask_upload(self.ctx, _ptr(m), sq, sk, ctypes.byref(h)))
        return Mask(self, h.value, sq, sk)

    def mask_temporal(self, tq, tk) -> Mask:
        """Resident mask "tk[j] <= tq[i]" built on the device (dit.rs:643-653)."""
        q = np.ascontiguousarray(tq, np.uint64).ravel()
        k = np.ascontiguousarray(tk, np.uint64).ravel()
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_mask_temporal(self.ctx, _ptr(q), q.size, _ptr(k), k.size, ctypes.byref(h)))
        return Mask(self, h.value, q.size, k.size)

    # ---- backend.rs:333-392: KV cache / MemRoPE ----
    def kv_cache_new(self, heads: int, head_dim: int, capacity_tokens: int) -> KvCache:
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_kv_cache_new(self.ctx, heads, head_dim, capacity_tokens, ctypes.byref(h)))
        return KvCache(self, h.value, heads, head_dim)

    def act_quant(self, x: Buf, x_row: int, rows: int, cols: int):
        q = np.empty((rows, cols), np.uint8)
        s = np.empty(rows, np.float32)
        _check(lib.lx2v_hip_act_quant(self.ctx, x.h, x_row, rows, cols, _ptr(q), _ptr(s)))
        return q, s

    def alloc_e4m3(self, rows: int, cols: int) -> Buf:
        """Per-token e4m3 activations [rows, cols] (codes + row scales)."""
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_alloc_e4m3(self.ctx, rows, cols, ctypes.byref(h)))
        return Buf(self, h.value)

    def quantize_act(self, x: Buf, x_row: int, rows: int, xq: Buf):
        _check(lib.lx2v_hip_quantize_act(self.ctx, x.h, x_row, rows, xq.h))

    def alloc_mx(self, rows: int, cols: int) -> Buf:
        """MX e4m3 activations [rows, cols] (codes + one E8M0 scale per 32 columns of a row)."""
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_alloc_mx(self.ctx, rows, cols, ctypes.byref(h)))
        return Buf(self, h.value)

    def quantize_mx(self, x: Buf, x_row: int, rows: int, xq: Buf):
        _check(lib.lx2v_hip_quantize_mx(self.ctx, x.h, x_row, rows, xq.h))

    def download_mx(self, buf: Buf, rows: int, cols: int):
        """Raw codes [rows, cols] and scale bytes [cols / 32, rows] of an MXE4M3 buffer."""
        q = np.empty((rows, cols), np.uint8)
        s = np.empty((cols // 32, rows), np.uint8)
        _check(lib.lx2v_hip_download_mx(self.ctx, buf.h, _ptr(q), _ptr(s)))
        return q, s

    def download_e4m3(self, buf: Buf, rows: int, cols: int):
        """Raw codes [rows, cols] and row scales [rows] of an E4M3 buffer."""
        q = np.empty((rows, cols), np.uint8)
        s = np.empty(rows, np.float32)
        _check(lib.lx2v_hip_download_e4m3(self.ctx, buf.h, _ptr(q), _ptr(s)))
        return q, s

    def graph_begin(self):
        _check(lib.lx2v_hip_graph_begin(self.ctx))

    def graph_end(self) -> Graph:
        h = ctypes.c_void_p()
        _check(lib.lx2v_hip_graph_end(self.ctx, ctypes.byref(h)))
        return Graph(self, h.value)

    def sync(self):
        _check(lib.lx2v_hip_sync(self.ctx))

    def profile_enable(self, on: bool = True):
        _check(lib.lx2v_hip_profile_enable(self.ctx, int(on)))

    def profile_report(self) -> Optional[str]:
        b = ctypes.create_string_buffer(1 << 16)
        _check(lib.lx2v_hip_profile_report(self.ctx, b, 1 << 16))
        s = b.value.decode()
        return s or None

    def profile_reset(self):
        _check(lib.lx2v_hip_profile_reset(self.ctx))

    def profile_region(self, name: str, begin: bool):
        _check(lib.lx2v_hip_profile_region(self.ctx, name.encode(), int(begin)))

    def profile_stats(self) -> dict:
        """{kernel name: (calls, total_ms)} from profile_report()."""
        out = {}
        for line in (self.profile_report() or "").splitlines():
            f = line.split()
            if len(f) == 5 and f[4].endswith("%") and f[1].isdigit():
                out[f[0]] = (int(f[1]), float(f[2]))
        return out

    def profile_kernel(self, name: str):
        c = ctypes.c_uint64(0)
        t = ctypes.c_double(0.0)
        _check(lib.lx2v_hip_profile_kernel(self.ctx, name.encode(), ctypes.byref(c), ctypes.byref(t)))
        return c.value, t.value

"""CPU oracle for lightx2v-rs's quantized-linear path (TEST INFRASTRUCTURE).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or as the timed
CPU baseline.  The product (``lightx2v-rs_amd/``) never imports it.

Two restatements of the reference live here:

* ``liblx2v_oracle.so`` (``lx2v_oracle.c``): the C restatement with Rust
  semantics, wrapped below with numpy-array functions;
* ``oracle.np_ref``: an independent numpy restatement of the parts that can be
  vectorised exactly (Rng, e4m3 codecs, Q8, the symmetric Q4), used to
  cross-check the C one.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liblx2v_oracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_sz = ctypes.c_size_t


def build() -> str:
    """Compile the C oracle (make -C oracle); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    """The loaded C oracle (built on first use if missing)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_rng_next_u64.restype = ctypes.c_uint64
        L.orc_rng_next_f32.restype = ctypes.c_float
        L.orc_f32_to_e4m3_ref.restype = ctypes.c_uint8
        L.orc_f32_to_e4m3_ref.argtypes = [ctypes.c_float]
        L.orc_f32_to_e4m3_canon.restype = ctypes.c_uint8
        L.orc_f32_to_e4m3_canon.argtypes = [ctypes.c_float]
        L.orc_f32_to_e4m3_ocp_rne.restype = ctypes.c_uint8
        L.orc_f32_to_e4m3_ocp_rne.argtypes = [ctypes.c_float]
        L.orc_e4m3_to_f32_ref.restype = ctypes.c_float
        L.orc_e4m3_to_f32_ref.argtypes = [ctypes.c_uint8]
        L.orc_e4m3_to_f32_ocp.restype = ctypes.c_float
        L.orc_e4m3_to_f32_ocp.argtypes = [ctypes.c_uint8]
        L.orc_f16_round.restype = ctypes.c_float
        L.orc_f16_round.argtypes = [ctypes.c_float]
        L.orc_bf16_round.restype = ctypes.c_float
        L.orc_bf16_round.argtypes = [ctypes.c_float]
        L.orc_gelu_tanh.restype = ctypes.c_float
        L.orc_gelu_tanh.argtypes = [ctypes.c_float]
        L.orc_q8_ref_group.restype = _sz
        L.orc_q8_ref_group.argtypes = [_sz]
        L.orc_fp8_ref_group.restype = _sz
        L.orc_fp8_ref_group.argtypes = [_sz]
        L.orc_mx_exponent.restype = ctypes.c_int
        L.orc_mx_exponent.argtypes = [ctypes.c_float]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


# ---- Rng (rng.rs:8-54) -------------------------------------------------------

class _RngState(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint64)]


class Rng:
    """The reference's SplitMix64 + Box-Muller generator (rng.rs:8-54)."""

    def __init__(self, seed: int):
        self._s = _RngState()
        lib().orc_rng_new(ctypes.byref(self._s), ctypes.c_uint64(seed & (2**64 - 1)))

    def next_u64(self) -> int:
        return lib().orc_rng_next_u64(ctypes.byref(self._s))

    def next_f32(self) -> float:
        return lib().orc_rng_next_f32(ctypes.byref(self._s))

    def uniform(self, n: int, a: float) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().orc_rng_uniform(ctypes.byref(self._s), _p(out, _f32p), _sz(n), ctypes.c_float(a))
        return out

    def normal(self, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().orc_rng_normal(ctypes.byref(self._s), _p(out, _f32p), _sz(n))
        return out


# ---- scalar codecs, mapped over arrays in C ---------------------------------

def _map_f2u(fn, v) -> np.ndarray:
    a = np.ascontiguousarray(v, np.float32).ravel()
    out = np.empty(a.size, np.uint8)
    getattr(lib(), fn)(_p(a, _f32p), _sz(a.size), _p(out, _u8p))
    return out


def _map_u2f(fn, c) -> np.ndarray:
    a = np.ascontiguousarray(c, np.uint8).ravel()
    out = np.empty(a.size, np.float32)
    getattr(lib(), fn)(_p(a, _u8p), _sz(a.size), _p(out, _f32p))
    return out


def _map_f2f(fn, v) -> np.ndarray:
    a = np.ascontiguousarray(v, np.float32)
    flat = a.ravel()
    out = np.empty(flat.size, np.float32)
    getattr(lib(), fn)(_p(flat, _f32p), _sz(flat.size), _p(out, _f32p))
    return out.reshape(a.shape)


def e4m3_encode_ref(v) -> np.ndarray:
    """quant.rs:376-406 verbatim."""
    return _map_f2u("orc_map_e4m3_ref", v)


def e4m3_encode_canon(v) -> np.ndarray:
    return _map_f2u("orc_map_e4m3_canon", v)


def e4m3_encode_ocp(v) -> np.ndarray:
    return _map_f2u("orc_map_e4m3_ocp", v)


def e4m3_decode_ref(codes) -> np.ndarray:
    """quant.rs:409-420 verbatim."""
    return _map_u2f("orc_map_decode_ref", codes)


def e4m3_decode_ocp(codes) -> np.ndarray:
    return _map_u2f("orc_map_decode_ocp", codes)


def gelu_tanh(v) -> np.ndarray:
    """crates/lightx2v-cpu/src/lib.rs:151-153 element-wise (keeps the shape)."""
    return _map_f2f("orc_map_gelu", v)


def f16_round(v) -> np.ndarray:
    return _map_f2f("orc_map_f16_round", v)


def bf16_round(v) -> np.ndarray:
    """bfloat16 round-to-nearest-even (vectorised, same rule as the C)."""
    a = np.ascontiguousarray(v, np.float32)
    b = a.view(np.uint32).astype(np.uint64)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    r = np.where(nan, ((b >> 16) | 0x40) << 16, r)
    return (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32).reshape(a.shape)


# ---- Q8 / Q4 / FP8 -----------------------------------------------------------

def q8_ref_group(cols: int) -> int:
    """quant.rs:156-160: 128 when it divides cols, else cols."""
    return int(lib().orc_q8_ref_group(cols))


def fp8_ref_group(cols: int) -> int:
    """quant.rs:425-429."""
    return int(lib().orc_fp8_ref_group(cols))


def q8_quantize(w: np.ndarray, rows: int, cols: int, group: int):
    w = np.ascontiguousarray(w, np.float32)
    q = np.empty(rows * cols, np.int8)
    s = np.empty(rows * cols // group, np.float32)
    lib().orc_q8_quantize(_p(w, _f32p), _sz(rows), _sz(cols), _sz(group), _p(q, _i8p), _p(s, _f32p))
    return q.reshape(rows, cols), s.reshape(rows, cols // group)


def q8_dequantize(q: np.ndarray, s: np.ndarray, rows: int, cols: int, group: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.int8)
    s = np.ascontiguousarray(s, np.float32)
    out = np.empty(rows * cols, np.float32)
    lib().orc_q8_dequantize(_p(q, _i8p), _p(s, _f32p), _sz(rows), _sz(cols), _sz(group), _p(out, _f32p))
    return out.reshape(rows, cols)


def q4_quantize(w: np.ndarray, rows: int, cols: int, group: int, hqq: bool):
    """quant.rs:226-292 (pass the effective group)."""
    w = np.ascontiguousarray(w, np.float32)
    c = np.empty(rows * cols, np.uint8)
    ng = rows * cols // group
    s = np.empty(ng, np.float32)
    z = np.empty(ng, np.float32)
    lib().orc_q4_quantize(_p(w, _f32p), _sz(rows), _sz(cols), _sz(group), ctypes.c_int(int(hqq)),
                          _p(c, _u8p), _p(s, _f32p), _p(z, _f32p))
    return c.reshape(rows, cols), s.reshape(rows, cols // group), z.reshape(rows, cols // group)


def q4_quantize_sym(w: np.ndarray, rows: int, cols: int, group: int):
    w = np.ascontiguousarray(w, np.float32)
    c = np.empty(rows * cols, np.uint8)
    ng = rows * cols // group
    s = np.empty(ng, np.float32)
    z = np.empty(ng, np.float32)
    lib().orc_q4_quantize_sym(_p(w, _f32p), _sz(rows), _sz(cols), _sz(group),
                              _p(c, _u8p), _p(s, _f32p), _p(z, _f32p))
    return c.reshape(rows, cols), s.reshape(rows, cols // group), z.reshape(rows, cols // group)


def q4_dequantize(c, s, z, rows: int, cols: int, group: int) -> np.ndarray:
    c = np.ascontiguousarray(c, np.uint8)
    s = np.ascontiguousarray(s, np.float32)
    z = np.ascontiguousarray(z, np.float32)
    out = np.empty(rows * cols, np.float32)
    lib().orc_q4_dequantize(_p(c, _u8p), _p(s, _f32p), _p(z, _f32p), _sz(rows), _sz(cols),
                            _sz(group), _p(out, _f32p))
    return out.reshape(rows, cols)


def q4_pack(codes) -> np.ndarray:
    c = np.ascontiguousarray(codes, np.uint8).ravel()
    out = np.empty((c.size + 1) // 2, np.uint8)
    lib().orc_q4_pack(_p(c, _u8p), _sz(c.size), _p(out, _u8p))
    return out


def q4_unpack(packed, n: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, np.uint8).ravel()
    out = np.empty(n, np.uint8)
    lib().orc_q4_unpack(_p(p, _u8p), _sz(n), _p(out, _u8p))
    return out


def fp8_quantize(w: np.ndarray, rows: int, cols: int, group: int, canon: bool):
    w = np.ascontiguousarray(w, np.float32)
    q = np.empty(rows * cols, np.uint8)
    s = np.empty(rows * cols // group, np.float32)
    lib().orc_fp8_quantize(_p(w, _f32p), _sz(rows), _sz(cols), _sz(group), ctypes.c_int(int(canon)),
                           _p(q, _u8p), _p(s, _f32p))
    return q.reshape(rows, cols), s.reshape(rows, cols // group)


def fp8_dequantize(q, s, rows: int, cols: int, group: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.float32)
    out = np.empty(rows * cols, np.float32)
    lib().orc_fp8_dequantize(_p(q, _u8p), _p(s, _f32p), _sz(rows), _sz(cols), _sz(group), _p(out, _f32p))
    return out.reshape(rows, cols)


# ---- linear (crates/lightx2v-cpu/src/lib.rs:296-326) ---------------------------

def linear(x: np.ndarray, w: np.ndarray, bias, act: int, rows: int | None = None,
           x_row: int = 0, y: np.ndarray | None = None, y_row: int = 0,
           nthreads: int = 1) -> np.ndarray:
    """``y[y_row+r] = act(x[x_row+r] . W^T + b)``, the oracle's loop order."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    if rows is None:
        rows = x.size // k - x_row
    if y is None:
        y = np.zeros((y_row + rows, n), np.float32)
    assert y.flags.c_contiguous and y.dtype == np.float32
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_linear(_p(x, _f32p), _sz(x_row), _sz(rows), _p(w, _f32p), _sz(n), _sz(k),
                     None if b is None else _p(b, _f32p), ctypes.c_int(act), _p(y, _f32p),
                     _sz(y_row), ctypes.c_int(nthreads))
    return y


def linear_f64(x: np.ndarray, w: np.ndarray, bias) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    rows = x.size // k
    y = np.empty((rows, n), np.float64)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_linear_f64(_p(x, _f32p), _sz(rows), _p(w, _f32p), _sz(n), _sz(k),
                         None if b is None else _p(b, _f32p), _p(y, _f64p))
    return y


# ---- norms around the linears ------------------------------------------------

def _fp(a):
    return None if a is None else _p(np.ascontiguousarray(a, np.float32), _f32p)


def layer_norm(x: np.ndarray, kind: int, w=None, b=None, mods=None, scale: int = 0, shift: int = 0,
               eps: float = 1e-6) -> np.ndarray:
    """crates/lightx2v-cpu/src/lib.rs:328-361; kind 0 Affine (w, b), 1 Mod (mods rows scale, shift)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, dim = x.shape
    keep = [np.ascontiguousarray(v, np.float32) if v is not None else None for v in (w, b, mods)]
    out = np.empty_like(x)
    lib().orc_layer_norm(_p(x, _f32p), _sz(rows), _sz(dim), ctypes.c_int(kind), _fp(keep[0]), _fp(keep[1]),
                         _fp(keep[2]), _sz(scale), _sz(shift), ctypes.c_float(eps), _p(out, _f32p))
    return out


def residual_norm(h: np.ndarray, a: np.ndarray, mods, gate, kind: int, w=None, b=None, scale: int = 0,
                  shift: int = 0, eps: float = 1e-6):
    """lib.rs:363-388: returns (h after h += a * gate, normed); gate None = 1."""
    h = np.array(h, np.float32, copy=True)
    a = np.ascontiguousarray(a, np.float32)
    rows, dim = h.shape
    keep = [np.ascontiguousarray(v, np.float32) if v is not None else None for v in (w, b, mods)]
    out = np.empty_like(h)
    lib().orc_residual_norm(_p(h, _f32p), _p(a, _f32p), _sz(rows), _sz(dim), _fp(keep[2]),
                            ctypes.c_long(-1 if gate is None else gate), ctypes.c_int(kind), _fp(keep[0]),
                            _fp(keep[1]), _sz(scale), _sz(shift), ctypes.c_float(eps), _p(out, _f32p))
    return h, out


def gate_residual(h: np.ndarray, a: np.ndarray, mods, gate: int) -> np.ndarray:
    """lib.rs:390-400: returns h + a * mods[gate]."""
    h = np.array(h, np.float32, copy=True)
    a = np.ascontiguousarray(a, np.float32)
    m = np.ascontiguousarray(mods, np.float32)
    rows, dim = h.shape
    lib().orc_gate_residual(_p(h, _f32p), _p(a, _f32p), _sz(rows), _sz(dim), _p(m, _f32p), _sz(gate))
    return h


def head_split(src: np.ndarray, col_off: int, heads: int, head_dim: int, rms_w=None, rope=None,
               eps: float = 1e-6, f64: bool = False) -> np.ndarray:
    """crates/lightx2v-cpu/src/lib.rs:406-455: src [rows, stride] -> [heads,
    rows, head_dim]; rms_w [heads * head_dim] or None; rope (cos, sin), each
    [rows, head_dim / 2], or None.  f64=True: the same in double (a pin)."""
    src = np.ascontiguousarray(src, np.float32)
    rows, stride = src.shape
    assert col_off + heads * head_dim <= stride
    w = None if rms_w is None else np.ascontiguousarray(rms_w, np.float32)
    c = s = None
    if rope is not None:
        c, s = (np.ascontiguousarray(t, np.float32) for t in rope)
        assert c.size == rows * (head_dim // 2) and s.size == c.size
    out = np.empty((heads, rows, head_dim), np.float64 if f64 else np.float32)
    fn = lib().orc_head_split_f64 if f64 else lib().orc_head_split
    fn(_p(src, _f32p), _sz(rows), _sz(stride), _sz(col_off), _sz(heads), _sz(head_dim), _fp(w), _fp(c), _fp(s),
       ctypes.c_float(eps), _p(out, _f64p if f64 else _f32p))
    return out


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask=None, nthreads: int = 8) -> np.ndarray:
    """crates/lightx2v-cpu/src/lib.rs:155-203: q [heads, sq, d], k / v [heads,
    sk, d], mask [sq, sk] bool or None -> out [sq, heads * d]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    heads, sq, d = q.shape
    sk = k.shape[1]
    m = None if mask is None else np.ascontiguousarray(mask, np.uint8)
    out = np.empty((sq, heads * d), np.float32)
    lib().orc_attention(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), _sz(heads), _sz(sq), _sz(sk), _sz(d),
                        None if m is None else _p(m, _u8p), _p(out, _f32p), ctypes.c_int(nthreads))
    return out


def act_quant_e4m3(x: np.ndarray):
    """Build-defined per-token e4m3 activation quantization."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty(rows, np.float32)
    lib().orc_act_quant_e4m3(_p(x, _f32p), _sz(rows), _sz(cols), _p(q, _u8p), _p(s, _f32p))
    return q, s


def act_quant_mx(x: np.ndarray):
    """Build-defined MX e4m3 quantization: codes [rows, cols] and E8M0 scale
    bytes, block-major [cols / 32, rows] (one per 32 columns of a row)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    assert cols % 32 == 0
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((cols // 32, rows), np.uint8)
    lib().orc_act_quant_mx(_p(x, _f32p), _sz(rows), _sz(cols), _p(q, _u8p), _p(s, _u8p))
    return q, s


def dequant_mx(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """Values of MX e4m3 codes: e4m3(q) * 2^(s - 127)."""
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.uint8)
    rows, cols = q.shape
    out = np.empty((rows, cols), np.float32)
    lib().orc_dequant_mx(_p(q, _u8p), _p(s, _u8p), _sz(rows), _sz(cols), _p(out, _f32p))
    return out


def mx_exponent(amax: float) -> int:
    return int(lib().orc_mx_exponent(ctypes.c_float(amax)))


# ---- decode tables -------------------------------------------------------------

def e4m3_table_ref() -> np.ndarray:
    """All 256 codes through quant.rs:409-420."""
    return e4m3_decode_ref(np.arange(256, dtype=np.uint8))


def e4m3_table_ocp() -> np.ndarray:
    return e4m3_decode_ocp(np.arange(256, dtype=np.uint8))

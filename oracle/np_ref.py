"""Independent numpy restatement of parts of the oracle (TEST INFRASTRUCTURE).

Written separately from ``lx2v_oracle.c`` so the two can be checked against
each other: vectorised, float32 throughout, no shared code.  Covers the
Rng (rng.rs:8-54), the e4m3 codecs (quant.rs:376-420), Q8 (quant.rs:154-186)
and the FP8 weight quantizer (quant.rs:423-455), plus the build-defined
canonical e4m3 encoder, the OCP e4m3fn RNE encoder and bf16 rounding.
"""

from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
F32 = np.float32


def rng_u64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Draws start..start+n of SplitMix64 seeded as rng.rs:13-27."""
    with np.errstate(over="ignore"):
        k = np.arange(start + 2, start + n + 2, dtype=np.uint64)
        z = np.uint64(seed & (2**64 - 1)) + k * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def rng_f32(seed: int, n: int) -> np.ndarray:
    """rng.rs:29-31: (u >> 40) / 2^24, both exact in f32."""
    return (rng_u64(seed, n) >> np.uint64(40)).astype(F32) / F32(1 << 24)


def rng_uniform(seed: int, n: int, a: float) -> np.ndarray:
    """rng.rs:34-36."""
    return (rng_f32(seed, n) * F32(2.0) - F32(1.0)) * F32(a)


def rng_normal(seed: int, n: int) -> np.ndarray:
    """rng.rs:39-54 (numpy's float32 log/cos/sin may differ from glibc's by
    an ulp, so compare this one with a tolerance)."""
    pairs = (n + 1) // 2
    f = rng_f32(seed, 2 * pairs).reshape(pairs, 2)
    u1 = np.maximum(f[:, 0], F32(1e-7))
    u2 = f[:, 1]
    r = np.sqrt(F32(-2.0) * np.log(u1))
    t = F32(2.0 * np.float32(np.pi)) * u2
    out = np.stack([r * np.cos(t), r * np.sin(t)], axis=1).ravel()
    return out[:n].astype(F32)


def _round_away(x: np.ndarray) -> np.ndarray:
    """f32::round: half away from zero (exact: the fraction of |x| is
    computed exactly, so 0.49999997 stays 0)."""
    x = np.asarray(x, F32)
    a = np.abs(x)
    f = np.floor(a)
    with np.errstate(invalid="ignore"):
        r = np.where(a - f >= F32(0.5), f + F32(1.0), f)
    return np.copysign(r, x).astype(F32)


def _as_u8(x: np.ndarray) -> np.ndarray:
    """float -> u8 `as`: saturating, truncating, NaN -> 0."""
    x = np.nan_to_num(x, nan=0.0)
    return np.clip(np.trunc(x), 0, 255).astype(np.uint8)


def e4m3_encode_ref(v) -> np.ndarray:
    """quant.rs:376-406 with Rust integer semantics."""
    v = np.asarray(v, F32).ravel()
    sign = np.where(np.signbit(v), 0x80, 0x00).astype(np.int64)
    a = np.abs(v)
    out = np.zeros(v.shape, np.int64)
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(a))
    zero = v == 0
    sat = ~np.isfinite(a) | (a >= F32(464.0))
    e = np.where(zero | sat, 0, e).astype(np.int64)
    sub = ~zero & ~sat & (e < -9)
    big = ~zero & ~sat & (e > 8)
    mid = ~zero & ~sat & ~sub & ~big
    # subnormal branch: (a / 2^-12).round() as u8, min 7
    m_sub = np.minimum(_as_u8(_round_away(a * F32(4096.0))).astype(np.int64), 7)
    # main branch
    exp = (e + 7) & 0xFF  # `as u8` wraps
    p = np.ldexp(F32(1.0), np.clip(e, -30, 30)).astype(F32)
    mant = _as_u8(_round_away((a / p - F32(1.0)) * F32(8.0))).astype(np.int64)
    carry = mant >= 8
    code_mid = np.where(carry, np.where(exp >= 15, 0x7E, ((exp + 1) << 3) & 0xFF),
                        ((exp << 3) & 0xFF) | mant)
    out = np.where(zero, 0, out)
    out = np.where(sat | big, 0x7E, out)
    out = np.where(sub, m_sub, out)
    out = np.where(mid, code_mid, out)
    return (out | sign).astype(np.uint8)


def e4m3_encode_canon(v) -> np.ndarray:
    """Build-defined weight encoder: quant.rs:376-406 for |v| >= 2^-6, 0x08
    for 2^-7 < |v| < 2^-6, signed zero below."""
    v = np.asarray(v, F32).ravel()
    a = np.abs(v)
    sign = np.where(np.signbit(v), 0x80, 0x00)
    code = e4m3_encode_ref(v).astype(np.int64)
    code = np.where(a < F32(2.0**-6), np.where(a > F32(2.0**-7), sign | 0x08, sign), code)
    return code.astype(np.uint8)


def e4m3_decode_ref(codes) -> np.ndarray:
    """quant.rs:409-420."""
    c = np.asarray(codes, np.uint8).astype(np.int64).ravel()
    sign = np.where(c & 0x80, F32(-1.0), F32(1.0))
    exp = (c >> 3) & 0xF
    mant = (c & 7).astype(F32)
    sub = sign * (mant / F32(8.0)) * F32(2.0**-9)
    norm = sign * (F32(1.0) + mant / F32(8.0)) * np.ldexp(F32(1.0), exp - 7).astype(F32)
    out = np.where(exp == 0, sub, norm).astype(F32)
    return np.where((exp == 15) & (c & 7 == 7), F32(np.nan), out).astype(F32)


def e4m3_decode_ocp(codes) -> np.ndarray:
    c = np.asarray(codes, np.uint8).astype(np.int64).ravel()
    sign = np.where(c & 0x80, F32(-1.0), F32(1.0))
    exp = (c >> 3) & 0xF
    mant = (c & 7).astype(F32)
    sub = sign * mant * F32(2.0**-9)
    norm = sign * (F32(1.0) + mant / F32(8.0)) * np.ldexp(F32(1.0), exp - 7).astype(F32)
    out = np.where(exp == 0, sub, norm).astype(F32)
    return np.where((exp == 15) & (c & 7 == 7), F32(np.nan), out).astype(F32)


def e4m3_encode_ocp_rne(v) -> np.ndarray:
    """OCP e4m3fn, round-to-nearest-even, by exhaustive nearest search over
    the 126 non-negative finite codes (a different method from the C)."""
    v = np.asarray(v, F32).ravel()
    table = e4m3_decode_ocp(np.arange(0, 127, dtype=np.uint8)).astype(np.float64)
    a = np.abs(v).astype(np.float64)
    idx = np.searchsorted(table, a)  # first table value >= a
    idx = np.clip(idx, 1, 126)
    lo, hi = table[idx - 1], table[idx]
    pick_hi = (a - lo > hi - a) | ((a - lo == hi - a) & (idx % 2 == 0))
    code = np.where(pick_hi, idx, idx - 1)
    code = np.where(a >= table[126], 126, code)
    code = np.where(a == 0, 0, code)
    out = code | np.where(np.signbit(v), 0x80, 0)
    return np.where(np.isnan(v), 0x7F, out).astype(np.uint8)


def q8_quantize(w: np.ndarray, group: int):
    """quant.rs:154-178 (group parameterised)."""
    w = np.asarray(w, F32)
    rows, cols = w.shape
    g = w.reshape(-1, group)
    amax = np.max(np.abs(g), axis=1)
    s = np.where(amax > 0, amax / F32(127.0), F32(1.0)).astype(F32)
    q = np.clip(_round_away(g / s[:, None]), -127, 127).astype(np.int8)
    return q.reshape(rows, cols), s.reshape(rows, cols // group)


def fp8_quantize(w: np.ndarray, group: int, canon: bool):
    """quant.rs:423-447 (group parameterised)."""
    w = np.asarray(w, F32)
    rows, cols = w.shape
    g = w.reshape(-1, group)
    amax = np.max(np.abs(g), axis=1)
    s = np.where(amax > 0, amax / F32(448.0), F32(1.0)).astype(F32)
    scaled = (g / s[:, None]).astype(F32)
    enc = e4m3_encode_canon if canon else e4m3_encode_ref
    return enc(scaled).reshape(rows, cols), s.reshape(rows, cols // group)


def bf16_round(v) -> np.ndarray:
    a = np.ascontiguousarray(v, F32)
    b = a.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    r = np.where((b & 0x7FFFFFFF) > 0x7F800000, ((b >> 16) | 0x40) << 16, r)
    return (r & 0xFFFFFFFF).astype(np.uint32).view(F32).reshape(a.shape)


def act_quant_mx(x) -> tuple:
    """MX e4m3 quantization restated with numpy (independent of the C):
    the scale exponent is found by search -- the smallest k in [-127, 127]
    with amax * 2^-k <= 448, over float64 -- and the codes by the
    nearest-value search of e4m3_encode_ocp_rne."""
    x = np.asarray(x, F32)
    rows, cols = x.shape
    blocks = np.abs(x.reshape(rows, cols // 32, 32)).max(axis=2).astype(np.float64)
    ks = np.arange(-127, 128)
    ok = blocks[..., None] * np.ldexp(1.0, -ks)[None, None, :] <= 448.0
    k = np.where(ok.any(axis=2), ks[np.argmax(ok, axis=2)], 127)
    scaled = (x.reshape(rows, cols // 32, 32).astype(np.float64) * np.ldexp(1.0, -k)[..., None]).astype(F32)
    q = e4m3_encode_ocp_rne(np.clip(scaled, F32(-448.0), F32(448.0))).reshape(rows, cols)
    return q, (k + 127).astype(np.uint8).T.copy()

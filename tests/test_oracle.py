"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each function of the oracle is held here to something other than its own
formula: the reference's known-answer vectors and its published run output
(tests/golden/quant_kats.json), an independent numpy restatement, torch's
IEEE / OCP conversions, closed forms, and f64 brute force.
"""

import json
import math
import os

import numpy as np
import pytest

import oracle as O
from oracle import np_ref as N

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "quant_kats.json")))


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---- e4m3 codecs (quant.rs:376-420) ------------------------------------------------

def test_e4m3_reference_kats():
    for e in GOLD["e4m3_encode"]:
        assert O.e4m3_encode_ref([e["v"]])[0] == e["code"], e
        assert N.e4m3_encode_ref([e["v"]])[0] == e["code"], e
    for e in GOLD["e4m3_decode"]:
        assert abs(O.e4m3_decode_ref([e["code"]])[0] - e["value"]) < e["tol"], e


def test_e4m3_derived_quirk_kats():
    for e in GOLD["e4m3_encode_derived"]:
        assert O.e4m3_encode_ref([e["v"]])[0] == e["code"], e
        assert N.e4m3_encode_ref([e["v"]])[0] == e["code"], e


def test_e4m3_decode_table_closed_form():
    """All 256 codes against sign * 2^(e-7) * (1 + m/8), exponent 0 as m * 2^-12
    (quant.rs:413-414), e=15/m=7 NaN; C and numpy bit-identical."""
    c = O.e4m3_table_ref()
    n = N.e4m3_decode_ref(np.arange(256))
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e, m = (code >> 3) & 15, code & 7
        if e == 15 and m == 7:
            assert np.isnan(c[code]) and np.isnan(n[code])
            continue
        want = s * m * 2.0**-12 if e == 0 else s * (1 + m / 8) * 2.0 ** (e - 7)
        assert c[code] == want and n[code] == want
        assert u32(c[code : code + 1])[0] == u32(n[code : code + 1])[0]  # signed zeros too
    assert u32(c[0x7F:0x80])[0] == 0x7FC00000 == u32(c[0xFF:0x100])[0]


def test_e4m3_ocp_against_torch():
    """The OCP e4m3fn decoder/encoder against torch.float8_e4m3fn (RNE)."""
    torch = pytest.importorskip("torch")
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    mine = O.e4m3_table_ocp()
    both_nan = np.isnan(codes) & np.isnan(mine)
    assert np.all(both_nan | (codes == mine))
    rng = np.random.default_rng(1)
    v = (rng.standard_normal(20000) * np.exp2(rng.uniform(-12, 9, 20000))).astype(np.float32)
    v = np.clip(v, -448, 448)
    v = np.concatenate([v, O.e4m3_table_ocp()[np.isfinite(O.e4m3_table_ocp())]])
    # midpoints between neighbouring codes: ties to even
    t = np.sort(np.unique(O.e4m3_table_ocp()[:127]))
    v = np.concatenate([v, ((t[1:] + t[:-1]) / 2).astype(np.float32)]).astype(np.float32)
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.e4m3_encode_ocp(v), want)
    assert np.array_equal(N.e4m3_encode_ocp_rne(v), want)


def test_e4m3_encoders_c_vs_numpy_dense():
    """C (glibc log2f) and numpy encoders agree on a dense sample spanning
    every binade of the encoder, plus the 64 floats below and above each
    power of two in [2^-12, 2^9] (where floor(log2f) can round)."""
    rng = np.random.default_rng(2)
    v = (rng.standard_normal(300000) * np.exp2(rng.uniform(-14, 10, 300000))).astype(np.float32)
    edges = []
    for e in range(-12, 10):
        b = np.float32(2.0**e).view(np.uint32)
        edges.append((np.arange(b - 64, b + 64, dtype=np.uint32)).view(np.float32))
    v = np.concatenate([v, -v[:1000]] + edges + [np.array([0.0, -0.0, 463.9, 464.0, 1e30, np.inf, -np.inf], np.float32)])
    assert np.array_equal(O.e4m3_encode_ref(v), N.e4m3_encode_ref(v))
    assert np.array_equal(O.e4m3_encode_canon(v), N.e4m3_encode_canon(v))


def test_e4m3_ref_roundtrips_its_own_grid():
    """Every decodable code value with exponent field >= 1 encodes back to
    itself (the normal range has no quirk)."""
    codes = np.array([c for c in range(256) if (c >> 3) & 15 and not ((c & 0x7F) == 0x7F)], np.uint8)
    vals = O.e4m3_decode_ref(codes)
    assert np.array_equal(O.e4m3_encode_ref(vals), codes)


def test_e4m3_canon_properties():
    """The canonical encoder never emits exponent-0 non-zero codes or NaN,
    equals the reference encoder for |v| >= 2^-6, and rounds below that to
    the nearer of 0 and 2^-6."""
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(200000) * np.exp2(rng.uniform(-12, 9, 200000))).astype(np.float32)
    c = O.e4m3_encode_canon(v)
    assert not np.any(((c & 0x78) == 0) & ((c & 7) != 0))
    assert not np.any((c & 0x7F) == 0x7F)
    big = np.abs(v) >= 2.0**-6
    assert np.array_equal(c[big], O.e4m3_encode_ref(v[big]))
    small = ~big
    want = np.where(np.abs(v[small]) > 2.0**-7, 0x08, 0x00) | np.where(np.signbit(v[small]), 0x80, 0)
    assert np.array_equal(c[small], want.astype(np.uint8))


# ---- Rng (rng.rs:8-54) --------------------------------------------------------------

def test_rng_deterministic_and_gaussian():  # rng.rs:59-69
    a = O.Rng(7).normal(1000)
    assert np.array_equal(a, O.Rng(7).normal(1000))
    assert not np.array_equal(O.Rng(8).normal(16), O.Rng(7).normal(16))
    assert abs(a.mean()) < 0.1 and abs(a.var() - 1.0) < 0.15


def test_rng_c_vs_numpy():
    r = O.Rng(12345)
    u = np.array([r.next_u64() for _ in range(1000)], np.uint64)
    assert np.array_equal(u, N.rng_u64(12345, 1000))
    assert np.array_equal(O.Rng(99).uniform(5001, 0.5), N.rng_uniform(99, 5001, 0.5))
    a, b = O.Rng(3).normal(4001), N.rng_normal(3, 4001)
    assert np.max(np.abs(a - b)) < 1e-5  # libm ulps only


def test_splitmix_known_values():
    """SplitMix64 from seed 0: published first outputs of the generator
    (state advanced before mixing, as rng.rs:20-27 does) -- Rng::new(s)
    adds one more golden step, so Rng::new(0) is SplitMix64 seeded with phi."""
    z = N.rng_u64(2**64 - 0x9E3779B97F4A7C15, 3)  # Rng state == 0 at start
    assert [int(x) for x in z] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


# ---- Q8 / Q4 / FP8 (quant.rs:142-460) --------------------------------------------------

def _ref_data(rows, cols, f):
    return np.array([f(i) for i in range(rows * cols)], np.float32)


def test_q8_round_trip_half_step():  # quant.rs:467-479
    rows, cols = 8, 256
    w = _ref_data(rows, cols, lambda i: (np.float32(i * 7919 % 1000) / np.float32(500.0) - np.float32(1.0)) * np.float32(1 + i // cols))
    g = O.q8_ref_group(cols)
    assert g == 128
    q, s = O.q8_quantize(w, rows, cols, g)
    assert s.size == rows * 2
    d = O.q8_dequantize(q, s, rows, cols, g).ravel()
    sc = np.repeat(s.ravel(), 128)
    assert np.all(np.abs(w - d) <= sc * 0.5 + 1e-6)
    qn, sn = N.q8_quantize(w.reshape(rows, cols), g)
    assert np.array_equal(q, qn) and np.array_equal(u32(s), u32(sn))


def test_q8_dequant_closed_form():
    rng = np.random.default_rng(4)
    q = rng.integers(-127, 128, (16, 96)).astype(np.int8)
    s = rng.uniform(0.001, 2, (16, 3)).astype(np.float32)
    d = O.q8_dequantize(q, s, 16, 96, 32)
    want = (q.astype(np.float32) * np.repeat(s, 32, axis=1)).astype(np.float32)
    assert np.array_equal(u32(d), u32(want))


def test_q4_round_trip_and_hqq_not_worse():  # quant.rs:482-526
    rows, cols = 16, 256

    def f(i):
        u = np.float32(i * 7919 % 1009) / np.float32(1009.0) - np.float32(0.5)
        return u * np.float32(8.0) if i % 97 == 0 else u * np.float32(0.3)

    w = _ref_data(rows, cols, f)
    c, s, z = O.q4_quantize(w, rows, cols, 64, False)
    assert c.max() <= 15
    d = O.q4_dequantize(c, s, z, rows, cols, 64).ravel()
    assert np.all(np.abs(w - d) <= np.repeat(s.ravel(), 64) * 0.52 + 1e-5)
    ch, sh, zh = O.q4_quantize(w, rows, cols, 64, True)
    assert ch.max() <= 15
    err = lambda cc, ss, zz: float(np.sum((w - O.q4_dequantize(cc, ss, zz, rows, cols, 64).ravel()) ** 2))
    assert err(ch, sh, zh) <= err(c, s, z) * 1.05
    # scale and zero are f16-rounded (quant.rs:280-281)
    assert np.array_equal(sh, sh.astype(np.float16).astype(np.float32))
    assert np.array_equal(zh, zh.astype(np.float16).astype(np.float32))


def test_q4_pack_layout():  # quant.rs:305-336
    codes = np.arange(16, dtype=np.uint8).repeat(3)[:47]
    p = O.q4_pack(codes)
    assert p.size == 24
    assert p[0] == (codes[0] | (codes[1] << 4)) and p[-1] == codes[46]
    assert np.array_equal(O.q4_unpack(p, 47), codes)


def test_q4_sym_layout():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((8, 64)) * 0.02).astype(np.float32)
    c, s, z = O.q4_quantize_sym(w, 8, 64, 32)
    assert c.max() <= 15 and np.all(z == 8.0)
    d = O.q4_dequantize(c, s, z, 8, 64, 32)
    q = c.astype(np.int32) - 8
    assert np.array_equal(u32(d), u32(q.astype(np.float32) * np.repeat(s, 32, axis=1)))
    amax = np.abs(w).reshape(-1, 32).max(1)
    assert np.array_equal(u32(s.ravel()), u32((amax / np.float32(7.0)).astype(np.float32)))


def test_fp8_round_trip_bound():  # quant.rs:541-554
    rows, cols = 4, 256
    w = _ref_data(rows, cols, lambda i: (np.float32(i * 7919 % 1000) / np.float32(500.0) - np.float32(1.0)) * np.float32(0.7))
    g = O.fp8_ref_group(cols)
    q, s = O.fp8_quantize(w, rows, cols, g, False)
    d = O.fp8_dequantize(q, s, rows, cols, g).ravel()
    tol = np.abs(w) * 0.0625 + np.repeat(s.ravel(), 128) * 0.5 + 1e-6
    assert np.all(np.abs(w - d) <= tol)
    qn, sn = N.fp8_quantize(w.reshape(rows, cols), g, False)
    assert np.array_equal(q, qn) and np.array_equal(u32(s), u32(sn))


def test_check_quant_published_value():
    """check.rs:294-320 reproduces the reference's printed 6.552e-2
    (docs/benchmarks.md:268): pins Rng::uniform, Q8, Q4+HQQ (f16 scale/zero,
    glibc powf) and the FP8 codec together."""
    g = GOLD["check_quant"]
    w = O.Rng(g["seed"]).uniform(g["rows"] * g["cols"], g["uniform_a"])
    rows, cols = g["rows"], g["cols"]
    q8, s8 = O.q8_quantize(w, rows, cols, O.q8_ref_group(cols))
    e8 = np.max(np.abs(w - O.q8_dequantize(q8, s8, rows, cols, 128).ravel()))
    c4, s4, z4 = O.q4_quantize(w, rows, cols, g["q4_group"], g["hqq"])
    e4 = np.max(np.abs(w - O.q4_dequantize(c4, s4, z4, rows, cols, g["q4_group"]).ravel()))
    qf, sf = O.fp8_quantize(w, rows, cols, O.fp8_ref_group(cols), False)
    df = O.fp8_dequantize(qf, sf, rows, cols, 128).ravel()
    ef = np.max(np.abs(w - df) / (np.abs(w) + np.float32(1e-6)))
    got = max(e8, e4, ef)
    mant, exp = f"{got:.3e}".split("e")
    assert f"{mant}e{int(exp)}" == g["printed"]
    assert got <= g["tolerance"]


def test_f16_and_bf16_rounding_vs_numpy_torch():
    rng = np.random.default_rng(6)
    v = (rng.standard_normal(50000) * np.exp2(rng.uniform(-30, 17, 50000))).astype(np.float32)
    f16 = O.f16_round(v[:20000])
    assert np.array_equal(f16, v[:20000].astype(np.float16).astype(np.float32))
    torch = pytest.importorskip("torch")
    want = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(u32(O.bf16_round(v)), u32(want))
    assert np.array_equal(u32(N.bf16_round(v)), u32(want))


# ---- gelu / linear (crates/lightx2v-cpu/src/lib.rs:151-153, 296-326) ------------------------

def test_gelu_tanh_closed_form():
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    got = O.gelu_tanh(x).astype(np.float64)
    xd = x.astype(np.float64)
    want = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd**3)))
    assert np.max(np.abs(got - want)) < 4e-6


def test_check_linear_kat():
    g = GOLD["check_linear"]
    y = O.linear(np.array(g["x"]), np.array(g["w"]).reshape(g["n"], g["k"]), np.array(g["b"]), 0)
    assert np.max(np.abs(y.ravel() - np.array(g["want"]))) <= g["tolerance"]
    assert np.array_equal(y.ravel(), np.array(g["want"], np.float32))


def test_linear_vs_f64_and_offsets_and_threads():
    rng = np.random.default_rng(7)
    M, N_, K = 37, 29, 130
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N_, K)) * 0.05).astype(np.float32)
    b = (rng.standard_normal(N_) * 0.01).astype(np.float32)
    y = O.linear(x, w, b, 0)
    y64 = O.linear_f64(x, w, b)
    assert np.max(np.abs(y - y64)) < 1e-5 * (1 + np.max(np.abs(y64)))
    # the sequential f32 sum order: element (0, 0) recomputed by hand
    acc = np.float32(0)
    for i in range(K):
        acc = np.float32(acc + np.float32(x[0, i] * w[0, i]))
    assert y[0, 0] == np.float32(acc + b[0])
    # threads: bit-identical
    assert np.array_equal(u32(O.linear(x, w, b, 1, nthreads=4)), u32(O.linear(x, w, b, 1)))
    # row offsets (backend.rs:199-212)
    yy = np.full((M + 5, N_), 7.0, np.float32)
    O.linear(x, w, b, 0, rows=10, x_row=3, y=yy, y_row=5)
    assert np.array_equal(yy[5:15], y[3:13]) and np.all(yy[:5] == 7.0)
    # GELU epilogue
    assert np.array_equal(u32(O.linear(x, w, b, 1)), u32(O.gelu_tanh(y).reshape(y.shape)))


def test_act_quant_oracle_properties():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((6, 96)).astype(np.float32)
    x[2] = 0.0
    x[3] *= 1e-3
    q, s = O.act_quant_e4m3(x)
    assert s[2] == 1.0 and np.all(q[2] == 0)
    d = O.e4m3_decode_ocp(q.ravel()).reshape(q.shape) * s[:, None]
    for r in (0, 1, 3, 4, 5):
        i = np.argmax(np.abs(x[r]))
        assert (q[r, i] & 0x7F) == 0x7E  # the row's absmax lands on 448
        # within half an e4m3 step (2^-4 relative) or half the subnormal step
        tol = np.maximum(np.abs(x[r]) * 2.0**-4, s[r] * 2.0**-10) + 1e-12
        assert np.all(np.abs(d[r] - x[r]) <= tol)


# ---- MX e4m3 (the FFN hand-off format, build-defined) -------------------------------

def _mx_inputs():
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((41, 320)) * np.exp(rng.uniform(-30, 30, (41, 10))).repeat(32, axis=1)).astype(np.float32)
    x[0, :32] = 0.0                                   # all-zero block
    x[1, :32] = 448.0                                 # amax exactly 448 * 2^0
    x[2, :32] = np.float32(448.0 * 2.0**-60)          # exactly 448 * 2^-60
    x[3, :32] = np.float32(np.nextafter(np.float32(448.0), np.float32(1e9)))  # just above: next scale
    x[4, :32] = np.float32(1e-42)                     # subnormal block
    x[5, :32] = np.float32(3.0e38)                    # near f32 max
    x[6, 32:64] = np.float32(1.75)                    # mantissa exactly 1.75
    x[7, 32:64] = np.float32(np.nextafter(np.float32(1.75), np.float32(2)))
    # an RNE tie on the scaled grid: with k = 0, 1.0625 is halfway between
    # the e4m3 neighbours 1.0 and 1.125 (step 2^-3 in [1, 2)) and goes to 1.0
    x[8, :32] = 448.0
    x[8, 1:32] = np.float32(1.0625)
    return x


def test_mx_quant_c_vs_numpy():
    x = _mx_inputs()
    q, s = O.act_quant_mx(x)
    q2, s2 = N.act_quant_mx(x)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_mx_quant_closed_form():
    x = _mx_inputs()
    q, s = O.act_quant_mx(x)
    rows, cols = x.shape
    k = s.T.astype(np.int64) - 127                    # [rows, blocks]
    assert k[0, 0] == -127 and np.all(q[0, :32] == 0)  # zero block: smallest scale, zero codes
    assert k[1, 0] == 0 and np.all(q[1, :32] == 0x7E)  # 448 = 448 * 2^0
    assert k[2, 0] == -60 and np.all(q[2, :32] == 0x7E)
    assert k[3, 0] == 1                                # 448+ needs 2^1 (then 224 = 0x76)
    assert k[6, 1] == k[7, 1] - 1                      # mantissa 1.75 stays, 1.75+ steps up
    assert k[8, 0] == 0 and np.all(q[8, 1:32] == 0x38)  # the tie went to even (1.0)
    amax = np.abs(x).reshape(rows, cols // 32, 32).max(axis=2).astype(np.float64)
    scaled = amax * np.ldexp(1.0, -k)
    live = (amax > 0) & (k > -127) & (k < 127)
    assert np.all(scaled <= 448.0)                     # no block saturates
    assert np.all(scaled[live] > 224.0)                # and k is the smallest such exponent
    d = O.dequant_mx(q, s)
    ref = (N.e4m3_decode_ocp(q.ravel()).reshape(q.shape).astype(np.float64)
           * np.ldexp(1.0, k).repeat(32, axis=1))
    assert np.array_equal(d.astype(np.float64), ref)  # dequantization is exact
    blk = np.ldexp(1.0, k).repeat(32, axis=1)
    err = np.abs(d.astype(np.float64) - x)
    # half an e4m3 step (2^-4 relative) or half the subnormal step 2^-10 of the block scale
    assert np.all(err <= np.maximum(np.abs(x) * 2.0**-4, blk * 2.0**-10) * (1 + 1e-6) + 1e-45)

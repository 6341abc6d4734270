"""Bit-exact checks of the device decode and encode paths against the oracle:
weight dequantization (the decode every GEMM uses), the device quantizers,
per-token activation quantization, buffer dtype conversion and the
synthetic-data generator."""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import normal, u32

pytestmark = pytest.mark.gpu


# ---- weight dequantization: quant.rs:180-186, 294-303, 449-455 ------------------------

@pytest.mark.parametrize("group", [32, 128, 384])
def test_dequant_q8_bit_exact(be, group):
    rows, cols = 48, 384
    rng = np.random.default_rng(group)
    q = rng.integers(-128, 128, (rows, cols)).astype(np.int8)
    q[0, :256] = np.arange(-128, 128)
    s = rng.uniform(1e-4, 3, (rows, cols // group)).astype(np.float32)
    w = be.weight_q8(q, s, rows, cols, group)
    got = be.dequantize(w)
    want = O.q8_dequantize(q, s, rows, cols, group)
    assert np.array_equal(u32(got), u32(want))


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("group,hqq", [(32, False), (64, True), (256, True)])
def test_dequant_q4_bit_exact(be, packed, group, hqq):
    rows, cols = 40, 256
    wf = normal(7 + group, rows * cols, 0.05).reshape(rows, cols)
    c, s, z = O.q4_quantize(wf, rows, cols, group, hqq)
    c[0, :16] = np.arange(16)
    codes = O.q4_pack(c) if packed else c
    w = be.weight_q4(codes, s, z, rows, cols, group, packed=packed)
    assert np.array_equal(u32(be.dequantize(w)), u32(O.q4_dequantize(c, s, z, rows, cols, group)))


@pytest.mark.parametrize("group", [128, 512])
def test_dequant_fp8_all_codes_bit_exact(be, group):
    """Every one of the 256 codes, including NaN (0x7F/0xFF -> +NaN
    0x7FC00000), exponent-0 codes (m * 2^-12) and the quirk codes."""
    rows, cols = 8, 512
    q = np.tile(np.arange(256, dtype=np.uint8), rows * cols // 256).reshape(rows, cols)
    s = np.exp2(np.random.default_rng(1).integers(-10, 4, (rows, cols // group))).astype(np.float32)
    s[0, 0] = 0.0123
    w = be.weight_fp8(q, s, rows, cols, group)
    assert w.info()["canonicalized"] == int(np.sum(((q & 0x78) == 0) & ((q & 7) != 0)))
    got = be.dequantize(w)
    want = O.fp8_dequantize(q, s, rows, cols, group)
    assert np.array_equal(u32(got), u32(want))


# ---- device quantizers (quant.rs:154-178, 423-447, symmetric Q4) --------------------------

def _weights(seed, rows, cols):
    w = normal(seed, rows * cols, 0.02).reshape(rows, cols)
    w[1] = 0.0                                # all-zero groups: scale 1.0
    w[2, ::7] *= np.float32(40.0)             # heavy tails
    w[3, :5] = np.float32(1e-9)               # far below 2^-7 after scaling
    return w


@pytest.mark.parametrize("group", [32, 128])
def test_quantize_q8_matches_oracle(be, group):
    rows, cols = 64, 512
    w = _weights(11, rows, cols)
    src = be.alloc(rows * cols, H.DTYPE_F32)
    be.write(src, w)
    wq = be.quantize_q8(src, rows, cols, group)
    q, s = O.q8_quantize(w, rows, cols, group)
    assert np.array_equal(u32(be.dequantize(wq)), u32(O.q8_dequantize(q, s, rows, cols, group)))


def test_quantize_q4_sym_matches_oracle(be):
    rows, cols, group = 64, 512, 32
    w = _weights(12, rows, cols)
    src = be.alloc(rows * cols, H.DTYPE_F32)
    be.write(src, w)
    wq = be.quantize_q4_sym(src, rows, cols, group)
    c, s, z = O.q4_quantize_sym(w, rows, cols, group)
    assert np.array_equal(u32(be.dequantize(wq)), u32(O.q4_dequantize(c, s, z, rows, cols, group)))


@pytest.mark.parametrize("group", [128, 512])
def test_quantize_fp8_matches_oracle(be, group):
    rows, cols = 64, 512
    w = _weights(13, rows, cols)
    src = be.alloc(rows * cols, H.DTYPE_F32)
    be.write(src, w)
    wq = be.quantize_fp8(src, rows, cols, group)
    q, s = O.fp8_quantize(w, rows, cols, group, True)
    assert wq.info()["canonicalized"] == 0
    assert np.array_equal(u32(be.dequantize(wq)), u32(O.fp8_dequantize(q, s, rows, cols, group)))


# ---- per-token e4m3 activation quantization ---------------------------------------------

@pytest.mark.parametrize("dtype", [H.DTYPE_F32, H.DTYPE_BF16])
@pytest.mark.parametrize("cols", [512, 1536, 3072, 5120, 8960, 16384, 100, 16400])
def test_act_quant_bit_exact(be, dtype, cols):
    rows = 37
    x = normal(cols, rows * cols).reshape(rows, cols)
    x[3] = 0.0
    x[4] *= np.float32(1e-30)
    x[5, 7] = np.float32(3e4)
    be.set_act_dtype(dtype)
    try:
        xb = be.upload(x)
    finally:
        be.set_act_dtype(H.DTYPE_F32)
    xs = x if dtype == H.DTYPE_F32 else O.bf16_round(x)
    q, s = be.act_quant(xb, 0, rows, cols)
    qw, sw = O.act_quant_e4m3(xs)
    assert np.array_equal(u32(s), u32(sw))
    assert np.array_equal(q, qw)
    # row offset
    q2, s2 = be.act_quant(xb, 5, 3, cols)
    assert np.array_equal(q2, qw[5:8]) and np.array_equal(u32(s2), u32(sw[5:8]))


def test_act_quant_rounding_edges(be):
    """Rows whose absmax is 448 quantize with inv == 1 exactly, so every
    element reaches the e4m3 rounding unchanged: all midpoints between
    adjacent codes (ties to even, subnormal ties at (k + 1/2) 2^-9), their
    float neighbours, and values past 448 that saturate."""
    vals = O.e4m3_decode_ocp(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)  # 0 .. 448
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    up = np.nextafter(mids, np.float32(np.inf))
    dn = np.nextafter(mids, np.float32(0))
    edge = np.concatenate([mids, up, dn, [447.99997, 448.0, 2 ** -10, 2 ** -9, 3 * 2 ** -10]]).astype(np.float32)
    cols = 512
    row = np.zeros(cols, np.float32)
    row[: edge.size] = edge
    row[0] = 448.0
    x = np.stack([row, -row, row[::-1].copy()])
    xb = be.upload(x)
    q, s = be.act_quant(xb, 0, 3, cols)
    qw, sw = O.act_quant_e4m3(x)
    assert np.all(s == 1.0) and np.array_equal(u32(s), u32(sw))
    assert np.array_equal(q, qw)


# ---- buffers, synthetic fill --------------------------------------------------------------

def test_buffers_round_trip_and_dtypes(be):
    v = normal(5, 1000)
    b = be.upload(v)
    assert b.dtype == H.DTYPE_F32 and len(b) == 1000
    assert np.array_equal(u32(be.download(b)), u32(v))
    z = be.alloc(50)
    assert np.all(be.download(z) == 0.0)
    be.write(z, v[:10])
    got = be.download(z)
    assert np.array_equal(got[:10], v[:10]) and np.all(got[10:] == 0)
    hb = be.alloc(1000, H.DTYPE_BF16)
    be.write(hb, v)
    assert np.array_equal(u32(be.download(hb)), u32(O.bf16_round(v)))
    fb = be.alloc(1000, H.DTYPE_F32)
    be.copy(hb, 100, fb, 200, 300)
    assert np.array_equal(be.download(fb)[200:500], O.bf16_round(v)[100:400])
    with pytest.raises(H.HipError) as e:
        be.copy(hb, 900, fb, 0, 200)
    assert e.value.status == H.ERR_BAD_SHAPE


def test_fill_normal_matches_rng(be):
    n = 10001
    b = be.alloc(n, H.DTYPE_F32)
    be.fill_normal(b, 1234, 0.5)
    want = O.Rng(1234).normal(n) * np.float32(0.5)
    assert np.max(np.abs(be.download(b) - want)) < 1e-5  # device vs glibc libm ulps

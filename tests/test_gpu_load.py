"""Load-time quantization on the device and checkpoint ingest, against the
oracle's restatement of the reference's quantizers.

* quantize_fp8_ref (Fp8E4M3::quantize with quant.rs:376-406 verbatim): raw
  codes bit-exact with orc_f32_to_e4m3_ref over a dense sweep of the encoder's
  input range, the exponent-wrap region included, and on N(0, 0.02) rows;
* quantize_q4 (Q4::quantize): round-to-nearest bit-exact (codes, f16 scale and
  zero); HQQ bit-exact except where glibc's powf and the device's
  double-precision pow round apart (counted and bounded);
* load_linear (dit.rs:61-157): f32 rows quantized at load, stored codes of
  every format, fused QKV from three stored parts, the error cases; and the
  reference's stored == load-time check (export.rs:284-363): device-quantized
  weights written in the export layout, read back, give the same codes.
"""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import FP8_TIGHT, W16_TIGHT, assert_close, oracle_w16, rel_l2, u32
from lightx2v_hip.quant import StoredFp8, StoredQ4, StoredQ8, WeightQuant
from lightx2v_hip.weights import (SafetensorsSource, WeightsError, f16_bytes, f32_bytes, load_linear,
                                  quantized_linear_tensors, write_safetensors)

pytestmark = pytest.mark.gpu
WQ = WeightQuant


def _normal(seed, n, std):
    return (O.Rng(seed).normal(n) * np.float32(std)).astype(np.float32)


def _dev_f32(be, w):
    src = be.alloc(w.size, H.DTYPE_F32)
    be.write(src, w)
    return src


def _encoder_sweep():
    """Inputs v/s for the encoder: every 16th f32 of [2^-14, 2^-5] (the
    subnormal, wrap and first normal binades), every f32 within 64 ulps of
    each power of two in [2^-12, 2^9], special values; both signs."""
    lo, hi = np.float32(2.0 ** -14).view(np.uint32), np.float32(2.0 ** -5).view(np.uint32)
    dense = np.arange(lo, hi, 16, dtype=np.uint32).view(np.float32)
    near = []
    for e in range(-12, 10):
        c = np.float32(2.0 ** e).view(np.uint32)
        near.append(np.arange(c - 64, c + 64, dtype=np.uint32).view(np.float32))
    special = np.array([0.0, 1e-30, 1.0, 1.0625, 2.0, 447.9, 448.0, 463.99, 464.0, 1e6, np.inf, np.nan,
                        2.0 ** -10, 1.5 * 2.0 ** -9, 1.9 * 2.0 ** -8, 1.99 * 2.0 ** -8, 0.9 * 2.0 ** -6],
                       np.float32)
    v = np.concatenate([dense] + near + [special])
    return np.concatenate([v, -v]).astype(np.float32)


def test_quantize_fp8_ref_encoder_sweep(be):
    """Rows of 127 sweep values plus one 448: the scale is exactly 1, so the
    device encodes the sweep values themselves."""
    v = _encoder_sweep()
    v = v[np.isfinite(v) & (np.abs(v) < 448.0)]
    per = 127
    v = np.concatenate([v, np.zeros(-v.size % per, np.float32)])
    rows = v.size // per
    w = np.concatenate([v.reshape(rows, per), np.full((rows, 1), 448.0, np.float32)], axis=1)
    wq = be.quantize_fp8_ref(_dev_f32(be, w), rows, 128, 128)
    e = be.weight_export(wq)
    assert np.array_equal(e["scales"].ravel(), np.ones(rows, np.float32))
    want = O.e4m3_encode_ref(w).reshape(rows, 128)
    bad = np.flatnonzero(e["q"].ravel() != want.ravel())
    assert bad.size == 0, f"{bad.size} codes differ, first v={w.ravel()[bad[:4]]}"
    # the wrap region really was exercised: NaN / 448 / huge codes from small inputs
    small = np.abs(w) < 2.0 ** -6
    assert np.any(small & ((want & 0x7F) == 0x7F)) and np.any(small & ((want & 0x7F) >= 0x70))
    canon = ((want & 0x78) == 0) & ((want & 7) != 0)
    assert wq.info()["canonicalized"] == int(canon.sum())


@pytest.mark.parametrize("rows,cols", [(96, 1536), (64, 1000)])  # group 128, and the cols fallback
def test_quantize_fp8_ref_matches_oracle(be, rows, cols):
    w = _normal(31, rows * cols, 0.02).reshape(rows, cols)
    w[1] = 0.0
    w[2, ::5] *= np.float32(30.0)
    group = O.fp8_ref_group(cols)
    wq = be.quantize_fp8_ref(_dev_f32(be, w), rows, cols, group)
    q, s = O.fp8_quantize(w, rows, cols, group, False)
    e = be.weight_export(wq)
    assert np.array_equal(e["q"], q) and np.array_equal(u32(e["scales"]), u32(s))
    assert np.array_equal(u32(be.dequantize(wq)), u32(O.fp8_dequantize(q, s, rows, cols, group)))
    # the GEMMs see the codes weight_fp8 would hold for the same struct
    x = _normal(32, 8 * cols, 1.0).reshape(8, cols)
    xb, y1, y2 = be.upload(x), be.alloc(8 * rows), be.alloc(8 * rows)
    w2 = be.weight_fp8(q, s, rows, cols, group)
    assert w2.info()["canonicalized"] == wq.info()["canonicalized"]
    be.linear(xb, 0, 8, wq, None, H.ACT_NONE, y1, 0)
    be.linear(xb, 0, 8, w2, None, H.ACT_NONE, y2, 0)
    assert np.array_equal(u32(be.download(y1)), u32(be.download(y2)))


@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_q4_rtn_bit_exact(be, group):
    rows, cols = 64, 1024
    w = _normal(41, rows * cols, 0.02).reshape(rows, cols)
    w[1] = 0.25          # constant groups: is = 1
    w[2, ::3] *= np.float32(25.0)
    wq = be.quantize_q4(_dev_f32(be, w), rows, cols, group, False)
    c, s, z = O.q4_quantize(w, rows, cols, group, False)
    e = be.weight_export(wq)
    assert np.array_equal(e["q"].ravel(), O.q4_pack(c))
    assert np.array_equal(u32(e["scales"]), u32(s)) and np.array_equal(u32(e["zeros"]), u32(z))
    assert np.array_equal(u32(be.dequantize(wq)), u32(O.q4_dequantize(c, s, z, rows, cols, group)))


@pytest.mark.parametrize("group", [32, 64])
def test_quantize_q4_hqq_matches_oracle(be, group):
    """HQQ (quant.rs:248-281) on the device: the shrink's a^-0.3 is glibc's
    powf restated (csrc/powf_arm.hpp, bit-identical to the libm on every
    positive f32 at this exponent, tests/test_powf_arm.py), so codes, scales
    and zero points equal the oracle's (which calls the libm) in every
    group, including a heavy-tailed row."""
    rows, cols = 128, 2048
    w = _normal(51, rows * cols, 0.02).reshape(rows, cols)
    w[3, ::7] *= np.float32(20.0)
    wq = be.quantize_q4(_dev_f32(be, w), rows, cols, group, True)
    c, s, z = O.q4_quantize(w, rows, cols, group, True)
    e = be.weight_export(wq)
    assert np.array_equal(O.q4_unpack(e["q"], rows * cols), c.ravel())
    assert np.array_equal(u32(e["scales"]), u32(s))
    assert np.array_equal(u32(e["zeros"]), u32(z))
    assert np.array_equal(u32(be.dequantize(wq)), u32(O.q4_dequantize(c, s, z, rows, cols, group)))


def test_quantize_q4_rejects_odd_group(be):
    src = be.alloc(12, H.DTYPE_F32)
    with pytest.raises(H.HipError):
        be.quantize_q4(src, 4, 3, 3, False)


# ---- load_linear ------------------------------------------------------------------


def _f32_file(tmp_path, keys, shapes, seed):
    tensors, vals = [], {}
    for i, k in enumerate(keys):
        o, c = shapes[f"{k}.weight"]
        w = _normal(seed + i, o * c, 0.02)
        b = _normal(seed + 100 + i, o, 0.01)
        vals[k] = (w.reshape(o, c), b)
        tensors += [(f"{k}.weight", "F32", [o, c], f32_bytes(w)), (f"{k}.bias", "F32", [o], f32_bytes(b))]
    path = str(tmp_path / "f32.safetensors")
    write_safetensors(path, tensors)
    return SafetensorsSource(path), vals


QKV = ["blocks.0.attn1.to_q", "blocks.0.attn1.to_k", "blocks.0.attn1.to_v"]
FFN1 = ["blocks.0.ffn.net.0.proj"]


def _oracle_dequant(fmt, w, rows, cols):
    if fmt.kind == "int8":
        g = O.q8_ref_group(cols)
        return O.q8_dequantize(*O.q8_quantize(w, rows, cols, g), rows, cols, g)
    if fmt.kind == "int4":
        g = fmt.group if cols % fmt.group == 0 else cols
        return O.q4_dequantize(*O.q4_quantize(w, rows, cols, g, fmt.hqq), rows, cols, g)
    g = O.fp8_ref_group(cols)
    return O.fp8_dequantize(*O.fp8_quantize(w, rows, cols, g, False), rows, cols, g)


@pytest.mark.parametrize("quant", ["int8", "fp8", "int4-g32", "int4-hqq-g64-ffn", "native"])
def test_load_linear_quantizes_at_load(be, tmp_path, quant):
    """f32 rows -> for_key -> the reference quantizer on the device; the fused
    QKV stacks three linears by rows (dit.rs:253)."""
    be.set_act_dtype(H.DTYPE_F32)
    q = WQ.parse(quant)
    shapes = {f"{k}.weight": [128, 256] for k in QKV}
    src, vals = _f32_file(tmp_path, QKV, shapes, 61)
    lin = load_linear(be, src, shapes, QKV, q)
    info = lin.w.info()
    assert (info["rows"], info["cols"]) == (384, 256)
    w = np.concatenate([vals[k][0] for k in QKV])
    b = np.concatenate([vals[k][1] for k in QKV])
    fmt = q.for_key(QKV[0])
    got = be.dequantize(lin.w)
    if fmt.kind == "native":
        assert np.array_equal(u32(got), u32(w))
    elif fmt.kind == "int4" and fmt.hqq:
        assert rel_l2(got, _oracle_dequant(fmt, w, 384, 256)) < 1e-3
    else:
        assert np.array_equal(u32(got), u32(_oracle_dequant(fmt, w, 384, 256)))
    assert np.array_equal(be.download(lin.b), b.astype(np.float32))


def _stored_tensors(fmt, key, w, b, group):
    rows, cols = w.shape
    t = [(f"{key}.bias", "F32", [rows], f32_bytes(b))]
    if fmt == "q8":
        q, s = O.q8_quantize(w, rows, cols, group)
        t += [(f"{key}.weight.q8", "I8", [rows, cols], q.tobytes()),
              (f"{key}.weight.scale", "F32", [rows, cols // group], f32_bytes(s))]
        return t, O.q8_dequantize(q, s, rows, cols, group)
    if fmt == "q4":
        c, s, z = O.q4_quantize(w, rows, cols, group, True)
        t += [(f"{key}.weight.q4", "U8", [rows, cols // 2], O.q4_pack(c).tobytes()),
              (f"{key}.weight.scale", "F16", [rows, cols // group], f16_bytes(s)),
              (f"{key}.weight.zero", "F16", [rows, cols // group], f16_bytes(z))]
        return t, O.q4_dequantize(c, s, z, rows, cols, group)
    q, s = O.fp8_quantize(w, rows, cols, group, False)
    t += [(f"{key}.weight.fp8", "U8", [rows, cols], q.tobytes()),
          (f"{key}.weight.scale", "F32", [rows, cols // group], f32_bytes(s))]
    return t, O.fp8_dequantize(q, s, rows, cols, group)


@pytest.mark.parametrize("fmt,group", [("q8", 32), ("q8", 128), ("q4", 32), ("q4", 64), ("fp8", 128), ("fp8", 256)])
def test_load_linear_stored_qkv(be, tmp_path, fmt, group):
    """Stored codes go to the device untouched: three stored parts stacked
    by rows, dequantized bit-exact, and the linear over them matches the
    oracle on the same dequantized weights."""
    be.set_act_dtype(H.DTYPE_F32)
    rows, cols = 96, 256
    tensors, deq, bias = [], [], []
    for i, k in enumerate(QKV):
        w = _normal(71 + i, rows * cols, 0.02).reshape(rows, cols)
        b = _normal(81 + i, rows, 0.01)
        t, d = _stored_tensors(fmt, k, w, b, group)
        tensors += t
        deq.append(d)
        bias.append(b)
    path = str(tmp_path / "stored.safetensors")
    write_safetensors(path, tensors)
    shapes = {f"{k}.weight": [rows, cols] for k in QKV}
    lin = load_linear(be, SafetensorsSource(path), shapes, QKV, WQ.native())  # stored wins over the policy
    want_w = np.concatenate(deq)
    assert np.array_equal(u32(be.dequantize(lin.w)), u32(want_w))
    be.set_act_dtype(H.DTYPE_F32)
    x = _normal(91, 40 * cols, 1.0).reshape(40, cols)
    xb, y = be.upload(x), be.alloc(40 * 3 * rows)
    be.linear(xb, 0, 40, lin.w, lin.b, H.ACT_NONE, y, 0)
    got = be.download(y).reshape(40, 3 * rows)
    b = np.concatenate(bias)
    if fmt == "fp8":  # per-token e4m3 activations (fp8 MFMA per-channel, the generic kernel grouped)
        xq, sx = O.act_quant_e4m3(x)
        xd = (O.e4m3_decode_ocp(xq.ravel()).reshape(40, cols) * sx[:, None]).astype(np.float32)
        assert_close(got, O.linear(xd, want_w, b, H.ACT_NONE), *FP8_TIGHT, what="stored fp8")
    else:  # weight dequantized to bf16 in the GEMM, bf16 MFMA
        assert_close(got, oracle_w16(x, want_w, b, H.ACT_NONE), *W16_TIGHT, what=f"stored {fmt}")


def test_stored_equals_load_time_quantization(be, tmp_path):
    """export.rs:284-363 on the device: f32 checkpoint -> quantized at load ->
    written in the export layout -> read back as stored codes: the same
    codes, scales and zeros as the load-time weights and the oracle's."""
    be.set_act_dtype(H.DTYPE_F32)
    keys = QKV + FFN1 + ["blocks.0.attn2.to_out.0"]
    shapes = {f"{k}.weight": [64, 256] for k in keys}
    shapes["blocks.0.ffn.net.0.proj.weight"] = [128, 256]
    src, vals = _f32_file(tmp_path, keys, shapes, 101)
    for quant in ["int8", "int4-hqq-g16-ffn", "int4-g32", "fp8"]:
        q = WQ.parse(quant)
        tensors = []
        loaded = {}
        for k in keys:
            lin = load_linear(be, src, shapes, [k], q)
            if q.for_key(k).kind == "native":
                continue
            loaded[k] = be.weight_export(lin.w)
            tensors += quantized_linear_tensors(be, f"{k}.weight", lin.w)
        path = str(tmp_path / f"{quant}.safetensors")
        write_safetensors(path, tensors)
        back = SafetensorsSource(path)
        for k, e in loaded.items():
            s = back.stored(k)
            fmt = q.for_key(k)
            w = vals[k][0]
            rows, cols = w.shape
            if fmt.kind == "int8":
                assert isinstance(s, StoredQ8)
                rq, rs = O.q8_quantize(w, rows, cols, O.q8_ref_group(cols))
                assert np.array_equal(s.q, rq.ravel()) and np.array_equal(u32(s.scales), u32(rs).ravel())
            elif fmt.kind == "int4":
                assert isinstance(s, StoredQ4) and s.group == fmt.group
                assert np.array_equal(s.q, O.q4_unpack(e["q"], rows * cols))
                assert np.array_equal(u32(s.scales), u32(e["scales"]).ravel())  # f16 values survive F16 storage
                assert np.array_equal(u32(s.zeros), u32(e["zeros"]).ravel())
                if not fmt.hqq:
                    rc, rs, rz = O.q4_quantize(w, rows, cols, fmt.group, False)
                    assert np.array_equal(s.q, rc.ravel()) and np.array_equal(u32(s.zeros), u32(rz).ravel())
            else:
                assert isinstance(s, StoredFp8)
                rq, rs = O.fp8_quantize(w, rows, cols, O.fp8_ref_group(cols), False)
                assert np.array_equal(s.q, rq.ravel()) and np.array_equal(u32(s.scales), u32(rs).ravel())


def test_load_linear_errors(be, tmp_path):
    rows, cols = 32, 128
    w = _normal(111, rows * cols, 0.02).reshape(rows, cols)
    b = _normal(112, rows, 0.01)
    t_q8, _ = _stored_tensors("q8", QKV[0], w, b, 32)
    t_fp8, _ = _stored_tensors("fp8", QKV[1], w, b, 128)
    t_f32 = [(f"{QKV[2]}.weight", "F32", [rows, cols], f32_bytes(w)), (f"{QKV[2]}.bias", "F32", [rows], f32_bytes(b))]
    path = str(tmp_path / "mixed.safetensors")
    write_safetensors(path, t_q8 + t_fp8 + t_f32)
    src = SafetensorsSource(path)
    shapes = {f"{k}.weight": [rows, cols] for k in QKV}
    with pytest.raises(WeightsError, match="only some are stored quantized"):
        load_linear(be, src, shapes, QKV, WQ.int8())
    with pytest.raises(WeightsError, match="mixed quantized storage"):
        load_linear(be, src, shapes, QKV[:2], WQ.int8())
    with pytest.raises(WeightsError, match="is stored 32x128, expected 64x128"):
        load_linear(be, src, {f"{QKV[0]}.weight": [64, 128]}, QKV[:1], WQ.int8())
    with pytest.raises(WeightsError, match="is not in the manifest"):
        load_linear(be, src, {}, QKV[:1], WQ.int8())

"""Host logic of the weight path (no device calls): the WeightQuant policy
(quant.rs:25-132), the Stored structs and the safetensors ingest /
writer (weights.rs:17-208, export.rs:4-274).

The WeightQuant known answers are the reference's own test values
(quant.rs:513-525); the rest are the reference's rules stated as cases.
"""

import numpy as np
import pytest

from lightx2v_hip.quant import (StoredFp8, StoredQ4, StoredQ8, WeightQuant, group_or_cols)
from lightx2v_hip.weights import (SafetensorsSource, WeightsError, bf16_to_f32, f16_bytes, f32_bytes,
                                  metadata, safetensors_bytes, write_safetensors)

WQ = WeightQuant


def test_reference_parse_kats():
    # quant.rs:513-525
    assert WQ.parse("int4-hqq-g32") == WQ.int4(32, True, False)
    assert WQ.parse("fp8") == WQ.fp8()
    assert WQ.parse("int4-hqq-g64-ffn").attn() == WQ.int8()


@pytest.mark.parametrize("s,want", [
    ("native", WQ.native()), ("bf16", WQ.native()), ("f16", WQ.native()),
    ("int8", WQ.int8()), ("q8", WQ.int8()), ("fp8-e4m3", WQ.fp8()),
    ("int4", WQ.int4(64, False, False)),            # default group 64
    ("int4-hqq", WQ.int4(64, True, False)),
    ("int4-ffn", WQ.int4(64, False, True)),
    ("int4-g16", WQ.int4(16, False, False)),
    ("int4-hqq-g128-ffn", WQ.int4(128, True, True)),
    ("int4-g+24", WQ.int4(24, False, False)),       # usize::from_str takes a leading '+'
])
def test_parse(s, want):
    assert WQ.parse(s) == want


@pytest.mark.parametrize("s,msg", [
    ("int16", "unknown weight format `int16`"),
    ("int4x", "bad weight format `int4x`"),
    ("foo", "unknown weight format `foo` (native | int8 | fp8 | int4[-hqq][-gN][-ffn])"),
    ("foo-ffn", "unknown weight format `foo`"),     # the message shows the string after -ffn is cut
    ("int4-g0", "int4 group must be a multiple of 8, got 0"),
    ("int4-g12", "int4 group must be a multiple of 8, got 12"),
    ("int4-gx", "bad group in `int4-gx`"),
    ("int4-g 8", "bad group in `int4-g 8`"),
    ("int4-g1_6", "bad group in `int4-g1_6`"),
    ("int4-g", "bad group in `int4-g`"),
    ("int4-ffn-hqq", "bad weight format `int4-ffn-hqq`"),
    ("int4-hqq-ffn-g8", "bad weight format `int4-hqq-ffn-g8`"),
    ("INT8", "unknown weight format `INT8`"),
])
def test_parse_errors(s, msg):
    with pytest.raises(ValueError) as e:
        WQ.parse(s)
    assert str(e.value).startswith(msg)


@pytest.mark.parametrize("q", [WQ.native(), WQ.int8(), WQ.fp8(), WQ.int4(8, False, False),
                               WQ.int4(64, True, False), WQ.int4(32, False, True), WQ.int4(256, True, True)])
def test_display_round_trips(q):
    assert WQ.parse(str(q)) == q


def test_display_strings():
    assert str(WQ.native()) == "native"
    assert str(WQ.int8()) == "int8"
    assert str(WQ.fp8()) == "fp8-e4m3"
    assert str(WQ.int4(64, True, True)) == "int4-hqq-g64-ffn"
    assert str(WQ.int4(32, False, False)) == "int4-g32"


def test_attn():
    assert WQ.int4(32, True, True).attn() == WQ.int8()
    for q in (WQ.native(), WQ.int8(), WQ.fp8(), WQ.int4(32, True, False)):
        assert q.attn() == q


FFN_ROLES = ["ffn.net.0.proj", "ffn.net.2"]
ATTN_ROLES = ["attn1.to_q", "attn1.to_k", "attn1.to_v", "attn1.to_out.0", "attn2.to_q", "attn2.to_k",
              "attn2.to_v", "attn2.to_out.0", "to_gate_compress"]


@pytest.mark.parametrize("q", [WQ.int8(), WQ.fp8(), WQ.int4(64, True, True), WQ.int4(32, False, False)])
def test_for_key(q):
    for layer in ("0", "29", "x"):  # the layer field is not parsed (quant.rs:58-62)
        for r in FFN_ROLES:
            assert q.for_key(f"blocks.{layer}.{r}") == q
        for r in ATTN_ROLES:
            assert q.for_key(f"blocks.{layer}.{r}") == q.attn()
        for r in ("norm2", "scale_shift_table", "attn1.norm_q", "ffn.net.0", "attn1.to_out", ""):
            assert q.for_key(f"blocks.{layer}.{r}") == WQ.native()
    for key in ("proj_out", "patch_embedding", "condition_embedder.text_embedder.linear_1", "blocks",
                "blocks.0", "block.0.ffn.net.2", "xblocks.0.ffn.net.2"):
        assert q.for_key(key) == WQ.native()


def test_group_fallback():
    assert group_or_cols(128, 1536) == 128
    assert group_or_cols(128, 1000) == 1000
    assert group_or_cols(64, 8960) == 64
    assert group_or_cols(48, 100) == 100


def test_q4_pack_and_unpack():
    rng = np.random.default_rng(0)
    for rows, cols in ((3, 8), (5, 7)):  # odd element count: the last byte's high nibble is padding
        n = rows * cols
        q = rng.integers(0, 16, n, dtype=np.uint8)
        ng = 1 if n % 8 else n // 8
        s = StoredQ4(q, np.ones(ng, np.float32), np.full(ng, 8, np.float32), rows, cols, n // ng)
        p = s.packed()
        assert p.size == (n + 1) // 2
        assert np.array_equal(p[0] & 15, q[0]) and np.array_equal(p[0] >> 4, q[1])  # element 2i low nibble
        back = StoredQ4.from_packed(p, s.scales, s.zeros, rows, cols)
        assert np.array_equal(back.q, q) and back.group == s.group


def test_stored_concat():
    a = StoredQ8(np.arange(8, dtype=np.int8), np.ones(2, np.float32), 2, 4, 4)
    b = StoredQ8(np.arange(8, 20, dtype=np.int8), np.full(3, 2, np.float32), 3, 4, 4)
    c = StoredQ8.concat([a, b])
    assert (c.rows, c.cols, c.group) == (5, 4, 4) and np.array_equal(c.q, np.arange(20))
    with pytest.raises(ValueError):
        StoredQ8.concat([a, StoredQ8(np.zeros(8, np.int8), np.ones(4, np.float32), 4, 2, 2)])
    f = StoredFp8.concat([StoredFp8(np.zeros(4, np.uint8), np.ones(2, np.float32), 2, 2, 2)] * 3)
    assert (f.rows, f.q.size, f.scales.size) == (6, 12, 6)


# ---- safetensors ------------------------------------------------------------------


def _bf16_bytes(v):
    b = np.asarray(v, np.float32).view(np.uint32)
    return ((b >> 16).astype("<u2")).tobytes()  # exactly representable values only


def test_safetensors_round_trip_and_dtypes(tmp_path):
    f32 = np.array([1.5, -2.25, 3e-3, 7.0], np.float32)
    f16v = np.array([0.5, -1.0, 65504.0], np.float32)
    bf = np.array([1.0, -0.5, 3.0, 2 ** -20], np.float32)
    tensors = [("a.weight", "F32", [2, 2], f32_bytes(f32)),
               ("b", "F16", [3], f16_bytes(f16v)),
               ("c", "BF16", [1, 4, 1], _bf16_bytes(bf)),
               ("d.weight.q8", "I8", [1, 3], np.array([-127, 0, 5], np.int8).tobytes()),
               ("e", "U8", [2], bytes([0x38, 0xFF]))]
    path = str(tmp_path / "t.safetensors")
    write_safetensors(path, tensors, {"k": "v"})
    raw = open(path, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    assert n % 8 == 0  # padded header
    src = SafetensorsSource(path)
    assert set(src.names()) == {"a.weight", "b", "c", "d.weight.q8", "e"}
    assert np.array_equal(src.get("a.weight", [2, 2]), f32)
    assert np.array_equal(src.get("a.weight", [1, 2, 2]), f32)  # size-1 dims ignored
    assert np.array_equal(src.get("b", [3]), f16v)
    assert np.array_equal(src.get("c", [4]), bf)
    dt, shape, data = src.raw("d.weight.q8")
    assert dt == "I8" and shape == [1, 3] and bytes(data) == np.array([-127, 0, 5], np.int8).tobytes()
    with pytest.raises(WeightsError, match="expected"):
        src.get("a.weight", [4, 2])
    with pytest.raises(WeightsError, match="missing tensor `zz`"):
        src.get("zz", [1])
    with pytest.raises(WeightsError, match="unsupported dtype I8"):
        src.get("d.weight.q8", [1, 3])
    assert src.has_linear("a") and src.has_linear("d") and not src.has_linear("b")
    assert safetensors_bytes(tensors, {"k": "v"}) == raw


def test_bf16_decode():
    assert np.array_equal(bf16_to_f32(np.array([0x3F80, 0xC000, 0x7F80], np.uint16)),
                          np.array([1.0, -2.0, np.inf], np.float32))


def _stored_file(tmp_path, tensors):
    path = str(tmp_path / "s.safetensors")
    write_safetensors(path, tensors)
    return SafetensorsSource(path)


def test_stored_q8_q4_fp8(tmp_path):
    rng = np.random.default_rng(1)
    q8 = rng.integers(-127, 128, (4, 64), dtype=np.int8)
    s8 = rng.random((4, 2), dtype=np.float32)
    codes = rng.integers(0, 16, 4 * 64, dtype=np.uint8)
    packed = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    s4 = rng.random((4, 4), dtype=np.float32).astype(np.float16).astype(np.float32)
    z4 = np.full((4, 4), 7.5, np.float32)
    fp = rng.integers(0, 256, (4, 64), dtype=np.uint8)
    sf = rng.random((4, 1), dtype=np.float32)
    src = _stored_file(tmp_path, [
        ("x.weight.q8", "I8", [4, 64], q8.tobytes()), ("x.weight.scale", "F32", [4, 2], f32_bytes(s8)),
        ("y.weight.q4", "U8", [4, 32], packed.tobytes()), ("y.weight.scale", "F16", [4, 4], f16_bytes(s4)),
        ("y.weight.zero", "F16", [4, 4], f16_bytes(z4)),
        ("z.weight.fp8", "U8", [4, 64], fp.tobytes()), ("z.weight.scale", "F32", [4, 1], f32_bytes(sf)),
        ("p.weight", "F32", [2, 2], f32_bytes(np.zeros(4)))])
    a = src.stored("x")
    assert isinstance(a, StoredQ8) and (a.rows, a.cols, a.group) == (4, 64, 32)
    assert np.array_equal(a.q, q8.ravel()) and np.array_equal(a.scales, s8.ravel())
    b = src.stored("y")
    assert isinstance(b, StoredQ4) and (b.rows, b.cols, b.group) == (4, 64, 16)
    assert np.array_equal(b.q, codes) and np.array_equal(b.scales, s4.ravel()) and np.array_equal(b.zeros, z4.ravel())
    c = src.stored("z")
    assert isinstance(c, StoredFp8) and (c.rows, c.cols, c.group) == (4, 64, 64)
    assert np.array_equal(c.q, fp.ravel()) and np.array_equal(c.scales, sf.ravel())
    assert src.stored("p") is None


@pytest.mark.parametrize("tensors,msg", [
    ([("x.weight.q8", "U8", [2, 8], bytes(16)), ("x.weight.scale", "F32", [2, 1], bytes(8))], "q8 is U8"),
    ([("x.weight.q8", "I8", [16], bytes(16)), ("x.weight.scale", "F32", [2, 1], bytes(8))], "q8 is I8 [16]"),
    ([("x.weight.q8", "I8", [2, 8], bytes(16)), ("x.weight.scale", "F32", [3, 1], bytes(12))], "scale [3, 1]"),
    ([("x.weight.q8", "I8", [2, 8], bytes(16)), ("x.weight.scale", "F32", [2, 3], bytes(24))], "scale [2, 3]"),
    ([("x.weight.q4", "U8", [2, 4], bytes(8)), ("x.weight.scale", "F16", [2, 1], bytes(4)),
      ("x.weight.zero", "F16", [2, 2], bytes(8))], "scale [2, 1] / zero [2, 2]"),
    ([("x.weight.fp8", "I8", [2, 8], bytes(16)), ("x.weight.scale", "F32", [2, 1], bytes(8))], "fp8 is I8"),
    ([("x.weight.fp8", "U8", [2, 8], bytes(16))], "missing tensor `x.weight.scale`"),
])
def test_stored_rejects(tmp_path, tensors, msg):
    src = _stored_file(tmp_path, tensors)
    with pytest.raises(WeightsError, match=msg.replace("[", r"\[").replace("]", r"\]")):
        src.stored("x")


def test_metadata():
    assert metadata(WQ.int4(64, True, False)) == {"lightx2v.format": "quant/1", "lightx2v.weights": "int4-hqq-g64"}
    assert metadata(WQ.native())["lightx2v.weights"] == "f16"

"""Backend::head_split (crates/lightx2v-core/src/backend.rs:255-273) on the
device against the oracle (crates/lightx2v-cpu/src/lib.rs:406-455
restated), at the DiT's call sites (crates/lightx2v-model/src/dit.rs:
477-489, 612-641, 705): q and k of the fused QKV output RMS-normed across
heads and RoPE-rotated, v plain; the cross-attention q normed; the text
K/V.

Bars: without the RMS norm every output is bit-identical to the oracle's
(the rotation's products and sums round as the reference's, no
contraction).  With it, the mean of squares is a lane reduction rather than
the reference's sequential fold: f32 output within rel-L2 2e-6 and max-abs
4e-6 * max|y| of the oracle (measured ~2e-7).  BF16 outputs round that
result once more (rel-L2 4e-3).
"""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import assert_close, u32

pytestmark = pytest.mark.gpu

HS_TIGHT = (2e-6, 4e-6)


def _buf(be, a, dtype):
    b = be.alloc(a.size, dtype)
    be.write(b, np.ascontiguousarray(a, np.float32).ravel())
    return b


def _tables(seed, rows, hd):
    ang = np.random.default_rng(seed).uniform(-np.pi, np.pi, (rows, hd // 2))
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _run(be, src, rows, stride, off, heads, hd, w, rope, eps, sdt, odt, pdt=H.DTYPE_F32):
    sb = _buf(be, src, sdt)
    wb = _buf(be, w, pdt) if w is not None else None
    rb = tuple(_buf(be, t, pdt) for t in rope) if rope is not None else None
    ob = be.alloc(heads * rows * hd, odt)
    be.head_split(sb, rows, stride, off, heads, hd, wb, rb, eps, ob)
    return be.download(ob).reshape(heads, rows, hd)


@pytest.mark.parametrize("sdt", [H.DTYPE_F32, H.DTYPE_BF16])
def test_dit_qkv_split(be, sdt):
    """The fused QKV output of the Wan chunk (4680 x 3*1536): q and k normed
    and rotated, v plain, one head_split call each."""
    rows, heads, hd, d = 4680, 12, 128, 1536
    rng = np.random.default_rng(1)
    src = rng.standard_normal((rows, 3 * d)).astype(np.float32) * np.float32(3.0)
    if sdt == H.DTYPE_BF16:
        src = O.bf16_round(src).reshape(rows, 3 * d)
    wq = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    rope = _tables(2, rows, hd)
    for off, w, rp in ((0, wq, rope), (d, wk, rope), (2 * d, None, None)):
        got = _run(be, src, rows, 3 * d, off, heads, hd, w, rp, 1e-6, sdt, H.DTYPE_F32)
        want = O.head_split(src, off, heads, hd, w, rp, 1e-6)
        if w is None:
            assert np.array_equal(u32(got), u32(want)), f"col_off {off}"
        else:
            assert_close(got, want, *HS_TIGHT, what=f"head_split col_off {off}")
        got16 = _run(be, src, rows, 3 * d, off, heads, hd, w, rp, 1e-6, sdt, H.DTYPE_BF16)
        if w is None:
            assert np.array_equal(u32(got16), u32(O.bf16_round(want).reshape(want.shape)))
        else:
            assert_close(got16, want, 4e-3, 8e-3, what="bf16 out")


def test_rope_only_bit_exact(be):
    """No norm, rotation only: bit-identical to the oracle."""
    rows, heads, hd = 300, 12, 128
    src = np.random.default_rng(3).standard_normal((rows, 2 * heads * hd)).astype(np.float32)
    rope = _tables(4, rows, hd)
    got = _run(be, src, rows, 2 * heads * hd, heads * hd, heads, hd, None, rope, 1e-6, H.DTYPE_F32, H.DTYPE_F32)
    assert np.array_equal(u32(got), u32(O.head_split(src, heads * hd, heads, hd, None, rope)))


@pytest.mark.parametrize("rows,d,off,heads,hd", [(4680, 1536, 0, 12, 128), (512, 3072, 0, 12, 128),
                                                 (512, 3072, 1536, 12, 128), (97, 2048, 0, 32, 64)])
def test_cross_attention_and_text_kv(be, rows, d, off, heads, hd):
    """Cross-attention q (rows x 1536, normed, no rope) and the text K/V
    (512 x 2*1536: k normed, v plain), plus a 64-wide head."""
    rng = np.random.default_rng(rows + off)
    src = rng.standard_normal((rows, d)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(heads * hd)).astype(np.float32) if off == 0 else None
    got = _run(be, src, rows, d, off, heads, hd, w, None, 1e-6, H.DTYPE_F32, H.DTYPE_F32)
    want = O.head_split(src, off, heads, hd, w, None, 1e-6)
    if w is None:
        assert np.array_equal(u32(got), u32(want))
    else:
        assert_close(got, want, *HS_TIGHT, what="head_split (no rope)")


def test_bf16_parameters(be):
    """rms_w and the rope tables as BF16 buffers: read as their bf16 values."""
    rows, heads, hd = 64, 4, 64
    rng = np.random.default_rng(5)
    src = rng.standard_normal((rows, heads * hd)).astype(np.float32)
    w = O.bf16_round((1 + 0.1 * rng.standard_normal(heads * hd)).astype(np.float32))
    rope = tuple(O.bf16_round(t).reshape(t.shape) for t in _tables(6, rows, hd))
    got = _run(be, src, rows, heads * hd, 0, heads, hd, w, rope, 1e-6, H.DTYPE_F32, H.DTYPE_F32, H.DTYPE_BF16)
    assert_close(got, O.head_split(src, 0, heads, hd, w, rope, 1e-6), *HS_TIGHT, what="bf16 parameters")


@pytest.mark.parametrize("rows,stride,off,heads,hd", [(33, 60, 0, 3, 20), (17, 61, 5, 2, 9), (40, 9000, 8, 60, 128)])
def test_generic_kernel(be, rows, stride, off, heads, hd):
    """Head sizes that are not multiples of 8 (an odd one leaves its last
    element unrotated, as the reference's loop over hd/2 pairs does),
    unaligned column offsets, and rows too wide for the register kernel."""
    rng = np.random.default_rng(rows)
    src = rng.standard_normal((rows, stride)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(heads * hd)).astype(np.float32)
    rope = _tables(rows + 1, rows, hd)
    got = _run(be, src, rows, stride, off, heads, hd, w, rope, 1e-5, H.DTYPE_F32, H.DTYPE_F32)
    assert_close(got, O.head_split(src, off, heads, hd, w, rope, 1e-5), *HS_TIGHT, what="generic head_split")
    got = _run(be, src, rows, stride, off, heads, hd, None, rope, 1e-5, H.DTYPE_F32, H.DTYPE_F32)
    assert np.array_equal(u32(got), u32(O.head_split(src, off, heads, hd, None, rope)))


def test_errors(be):
    rows, heads, hd = 8, 2, 16
    src = be.upload(np.zeros(rows * 64, np.float32))
    out = be.alloc(rows * heads * hd)
    with pytest.raises(H.HipError) as e:  # columns past the row
        be.head_split(src, rows, 64, 40, heads, hd, None, None, 1e-6, out)
    assert e.value.status == H.ERR_BAD_SHAPE
    with pytest.raises(H.HipError) as e:  # out too short
        be.head_split(src, rows, 64, 0, heads, hd, None, None, 1e-6, be.alloc(rows * heads * hd - 1))
    assert e.value.status == H.ERR_BAD_SHAPE
    with pytest.raises(H.HipError) as e:  # out aliases src
        be.head_split(src, rows, 64, 0, heads, hd, None, None, 1e-6, src)
    assert e.value.status == H.ERR_ALIAS
    with pytest.raises(H.HipError) as e:  # one rope table without the other
        lib = H.lib
        H._check(lib.lx2v_hip_head_split(be.ctx, src.h, rows, 64, 0, heads, hd, None, out.h, None,
                                          H.ctypes.c_float(1e-6), out.h))
    assert e.value.status == H.ERR_BAD_ARG

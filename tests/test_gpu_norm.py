"""layer_norm / residual_norm / gate_residual (backend.rs:214-252) on the
device against the oracle (crates/lightx2v-cpu/src/lib.rs:328-400), and the
fused producer: the norm writing the per-token / MX e4m3 input of the next
FP8 linear in the same pass.

Tolerances: the device sums mean and variance across lanes instead of the
reference's sequential f32 loop, which moves results by ~1e-7 relative;
F32 outputs are held to rel-L2 <= 2e-6 and max-abs <= 2e-5 * max|y|.
Element-wise residual updates in F32 are bit-exact (one multiply, one add).
Quantized outputs: >= 99.9% of e4m3 codes identical to the oracle's
quantization of the oracle's norm, the rest one code step away; the fused
norm + linear is bit-identical to norm -> F32 -> quantize_act -> linear.
"""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import assert_close, u32

pytestmark = pytest.mark.gpu
NK = H.NormKind
TOL = (2e-6, 2e-5)


def _data(seed, rows, dim):
    rng = O.Rng(seed)
    x = (rng.normal(rows * dim) * np.float32(2.0) + np.float32(0.5)).reshape(rows, dim).astype(np.float32)
    a = (rng.normal(rows * dim) * np.float32(0.7)).reshape(rows, dim).astype(np.float32)
    mods = (rng.normal(6 * dim) * np.float32(0.1)).reshape(6, dim).astype(np.float32)
    w = (1 + rng.normal(dim) * np.float32(0.1)).astype(np.float32)
    b = (rng.normal(dim) * np.float32(0.1)).astype(np.float32)
    return x, a, mods, w, b


def _up(be, v, dtype=H.DTYPE_F32):
    buf = be.alloc(v.size, dtype)
    be.write(buf, v)
    return buf


# 1536 / 3072 / 5120 / 8960: one, two, four waves per row; 100 and 16400: the any-width kernel
DIMS = [1536, 3072, 5120, 8960, 100, 16400]


@pytest.mark.parametrize("dim", DIMS)
@pytest.mark.parametrize("kind", [H.NORM_AFFINE, H.NORM_MOD])
def test_layer_norm_f32(be, dim, kind):
    rows = 37
    x, _, mods, w, b = _data(11 + dim, rows, dim)
    xb, mb, wb, bb = _up(be, x), _up(be, mods), _up(be, w), _up(be, b)
    out = be.alloc(rows * dim, H.DTYPE_F32)
    norm = NK.affine(wb, bb) if kind == H.NORM_AFFINE else NK.mod(1, 0)
    be.layer_norm(xb, rows, dim, norm, mb, 1e-6, out)
    want = O.layer_norm(x, kind, w, b, mods, scale=1, shift=0)
    assert_close(be.download(out).reshape(rows, dim), want, *TOL, what=f"layer_norm {dim}")


@pytest.mark.parametrize("dim", [1536, 100])
def test_layer_norm_bf16(be, dim):
    """bf16 activations, bf16 params (converted on the device), bf16 out."""
    rows = 29
    x, _, mods, w, b = _data(21 + dim, rows, dim)
    xr, mr = O.bf16_round(x), O.bf16_round(mods)
    xb, mb = _up(be, xr, H.DTYPE_BF16), _up(be, mr, H.DTYPE_BF16)
    out = be.alloc(rows * dim, H.DTYPE_BF16)
    be.layer_norm(xb, rows, dim, NK.mod(4, 3), mb, 1e-6, out)
    want = O.bf16_round(O.layer_norm(xr, 1, mods=mr, scale=4, shift=3))
    got = be.download(out).reshape(rows, dim)
    assert_close(got, want, 4e-3, 8e-3, what="bf16 layer_norm")  # one bf16 rounding of the output


@pytest.mark.parametrize("dim", [1536, 3072, 100])
@pytest.mark.parametrize("gate", [None, 2])
def test_residual_norm(be, dim, gate):
    rows = 41
    x, a, mods, w, b = _data(31 + dim, rows, dim)
    hb, ab, mb, wb, bb = _up(be, x), _up(be, a), _up(be, mods), _up(be, w), _up(be, b)
    out = be.alloc(rows * dim, H.DTYPE_F32)
    be.residual_norm(hb, ab, rows, dim, mb, gate, NK.affine(wb, bb), 1e-6, out)
    h_want, n_want = O.residual_norm(x, a, mods, gate, 0, w, b)
    assert np.array_equal(u32(be.download(hb).reshape(rows, dim)), u32(h_want))
    assert_close(be.download(out).reshape(rows, dim), n_want, *TOL, what="residual_norm")


def test_residual_norm_bf16_reads_unrounded_sum(be):
    """h is bf16: h is stored rounded, the norm reads the unrounded sum."""
    rows, dim = 23, 1536
    x, a, mods, _, _ = _data(41, rows, dim)
    xr, ar = O.bf16_round(x), O.bf16_round(a)
    hb, ab, mb = _up(be, xr, H.DTYPE_BF16), _up(be, ar, H.DTYPE_BF16), _up(be, mods)
    out = be.alloc(rows * dim, H.DTYPE_F32)
    be.residual_norm(hb, ab, rows, dim, mb, 5, NK.mod(1, 0), 1e-6, out)
    h_want, n_want = O.residual_norm(xr, ar, mods, 5, 1, scale=1, shift=0)
    assert np.array_equal(u32(be.download(hb).reshape(rows, dim)), u32(O.bf16_round(h_want)))
    assert_close(be.download(out).reshape(rows, dim), n_want, *TOL, what="bf16 residual_norm")


@pytest.mark.parametrize("dim,dtype", [(1536, H.DTYPE_F32), (1536, H.DTYPE_BF16), (100, H.DTYPE_F32), (99, H.DTYPE_BF16)])
def test_gate_residual(be, dim, dtype):
    rows = 19
    x, a, mods, _, _ = _data(51 + dim, rows, dim)
    if dtype == H.DTYPE_BF16:
        x, a = O.bf16_round(x), O.bf16_round(a)
    hb, ab, mb = _up(be, x, dtype), _up(be, a, dtype), _up(be, mods)
    be.gate_residual(hb, ab, rows, dim, mb, 4)
    want = O.gate_residual(x, a, mods, 4)
    if dtype == H.DTYPE_BF16:
        want = O.bf16_round(want)
    assert np.array_equal(u32(be.download(hb).reshape(rows, dim)), u32(want))


def _codes_close(got_q, got_s, want_q, want_s):
    same = got_q == want_q
    assert same.mean() >= 0.999, f"{(~same).sum()} of {same.size} codes differ"
    dq = np.abs(got_q.astype(np.int16) - want_q.astype(np.int16))
    # e4m3 codes of one sign are monotone in magnitude: a rounding flip is one code step
    assert np.all(dq[~same] == 1), np.unique(dq[~same])
    assert np.max(np.abs(got_s / want_s - 1.0)) <= 1e-5


@pytest.mark.parametrize("dim", [1536, 5120, 100])
def test_norm_to_e4m3(be, dim):
    rows = 33
    x, a, mods, w, b = _data(61 + dim, rows, dim)
    xb, mb = _up(be, x), _up(be, mods)
    xq = be.alloc_e4m3(rows, dim)
    be.layer_norm(xb, rows, dim, NK.mod(1, 0), mb, 1e-6, xq)
    q, s = be.download_e4m3(xq, rows, dim)
    wq, ws = O.act_quant_e4m3(O.layer_norm(x, 1, mods=mods, scale=1, shift=0))
    _codes_close(q, s, wq, ws)


@pytest.mark.parametrize("dim", [1536, 3072])
def test_residual_norm_to_mx(be, dim):
    rows = 40
    x, a, mods, w, b = _data(71 + dim, rows, dim)
    hb, ab, mb, wb, bb = _up(be, x), _up(be, a), _up(be, mods), _up(be, w), _up(be, b)
    xm = be.alloc_mx(rows, dim)
    be.residual_norm(hb, ab, rows, dim, mb, 2, NK.affine(wb, bb), 1e-6, xm)
    q, s = be.download_mx(xm, rows, dim)
    _, n_want = O.residual_norm(x, a, mods, 2, 0, w, b)
    wq, ws = O.act_quant_mx(n_want)
    same = q == wq
    assert same.mean() >= 0.999, f"{(~same).sum()} of {same.size} codes differ"
    assert np.mean(s == ws.reshape(s.shape)) >= 0.999


def test_fused_norm_quant_linear_equals_unfused(be):
    """residual_norm -> E4M3 -> linear is bit-identical to residual_norm ->
    F32 -> quantize_act -> linear: the fused pass quantizes the same values."""
    rows, dim, n = 300, 1536, 512
    x, a, mods, _, _ = _data(81, rows, dim)
    q, s = O.fp8_quantize((O.Rng(82).normal(n * dim) * np.float32(0.02)).reshape(n, dim), n, dim, dim, True)
    w = be.weight_fp8(q, s, n, dim, dim)
    mb = _up(be, mods)
    h1, h2, ab = _up(be, x), _up(be, x), _up(be, a)
    xq = be.alloc_e4m3(rows, dim)
    be.residual_norm(h1, ab, rows, dim, mb, 2, NK.mod(1, 0), 1e-6, xq)
    y1 = be.alloc(rows * n, H.DTYPE_F32)
    be.linear(xq, 0, rows, w, None, H.ACT_NONE, y1, 0)
    nf = be.alloc(rows * dim, H.DTYPE_F32)
    be.residual_norm(h2, ab, rows, dim, mb, 2, NK.mod(1, 0), 1e-6, nf)
    xq2 = be.alloc_e4m3(rows, dim)
    be.quantize_act(nf, 0, rows, xq2)
    y2 = be.alloc(rows * n, H.DTYPE_F32)
    be.linear(xq2, 0, rows, w, None, H.ACT_NONE, y2, 0)
    assert np.array_equal(u32(be.download(y1)), u32(be.download(y2)))
    assert np.array_equal(u32(be.download(h1)), u32(be.download(h2)))


def test_norm_errors(be):
    rows, dim = 4, 64
    x, a, mods, w, b = _data(91, rows, dim)
    xb, ab, mb = _up(be, x), _up(be, a), _up(be, mods)
    out = be.alloc(rows * dim, H.DTYPE_F32)
    with pytest.raises(H.HipError):  # a in another dtype
        be.residual_norm(xb, _up(be, a, H.DTYPE_BF16), rows, dim, mb, None, NK.mod(1, 0), 1e-6, out)
    with pytest.raises(H.HipError):  # mods row past the table
        be.layer_norm(xb, rows, dim, NK.mod(6, 0), mb, 1e-6, out)
    with pytest.raises(H.HipError):  # out aliases x
        be.layer_norm(xb, rows, dim, NK.mod(1, 0), mb, 1e-6, xb)
    with pytest.raises(H.HipError):  # E4M3 buffer of another width
        be.layer_norm(xb, rows, dim, NK.mod(1, 0), mb, 1e-6, be.alloc_e4m3(rows, 32))
    with pytest.raises(H.HipError):  # too many rows
        be.layer_norm(xb, rows + 1, dim, NK.mod(1, 0), mb, 1e-6, out)

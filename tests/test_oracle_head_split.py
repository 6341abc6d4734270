"""The oracle's head_split (oracle/lx2v_oracle.c orc_head_split, restating
crates/lightx2v-cpu/src/lib.rs:406-455), pinned by an independent numpy
restatement in f64 (complex multiplication for the rotation, a per-row
mean over all heads for the RMS) and by closed forms that a plausible
mistake breaks: a zero angle leaves the normalised values, a quarter turn
maps each pair (a, b) to (-b, a), a constant 0.5 row normalises to the
weight exactly, no norm and no rope is a pure transpose, and the RMS is
taken over all heads of a row (a per-head RMS fails the scaled-head case).
"""

import numpy as np
import pytest

import oracle as O


def np_head_split(src, col_off, heads, hd, w=None, rope=None, eps=1e-6):
    x = np.asarray(src, np.float64)[:, col_off:col_off + heads * hd]
    if w is not None:
        inv = 1.0 / np.sqrt(np.mean(x * x, axis=1) + eps)
        x = x * inv[:, None] * np.asarray(w, np.float64)[None, :]
    if rope is not None:
        c, s = (np.asarray(t, np.float64).reshape(x.shape[0], hd // 2) for t in rope)
        z = x.reshape(x.shape[0], heads, hd // 2, 2)
        zc = (z[..., 0] + 1j * z[..., 1]) * (c + 1j * s)[:, None, :]
        x = np.stack([zc.real, zc.imag], axis=-1).reshape(x.shape[0], heads * hd)
    return x.reshape(x.shape[0], heads, hd).transpose(1, 0, 2)


def _case(seed, rows, stride, heads, hd):
    rng = np.random.default_rng(seed)
    src = rng.standard_normal((rows, stride)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(heads * hd)).astype(np.float32)
    ang = rng.uniform(-np.pi, np.pi, (rows, hd // 2))
    return src, w, (np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32))


@pytest.mark.parametrize("rows,stride,off,heads,hd", [(7, 3 * 1536, 0, 12, 128), (5, 3 * 1536, 1536, 12, 128),
                                                     (9, 768, 256, 4, 64), (3, 48, 16, 2, 16)])
@pytest.mark.parametrize("norm,rope", [(True, True), (True, False), (False, True), (False, False)])
def test_against_numpy_f64(rows, stride, off, heads, hd, norm, rope):
    src, w, cs = _case(rows + heads, rows, stride, heads, hd)
    got = O.head_split(src, off, heads, hd, w if norm else None, cs if rope else None)
    want = np_head_split(src, off, heads, hd, w if norm else None, cs if rope else None)
    assert got.shape == (heads, rows, hd)
    err = np.max(np.abs(got - want)) / np.max(np.abs(want))
    assert err < 2e-6, err
    # and the oracle's own f64 twin
    g64 = O.head_split(src, off, heads, hd, w if norm else None, cs if rope else None, f64=True)
    assert np.max(np.abs(g64 - want)) / np.max(np.abs(want)) < 1e-12


def test_no_norm_no_rope_is_transpose():
    src, _, _ = _case(1, 6, 100, 3, 32)
    got = O.head_split(src, 4, 3, 32)
    want = src[:, 4:100].reshape(6, 3, 32).transpose(1, 0, 2)
    assert np.array_equal(got, want)


def test_zero_angle_and_quarter_turn():
    rows, heads, hd = 4, 3, 16
    src, w, _ = _case(2, rows, heads * hd, heads, hd)
    one, zero = np.ones((rows, hd // 2), np.float32), np.zeros((rows, hd // 2), np.float32)
    base = O.head_split(src, 0, heads, hd, w)
    assert np.array_equal(O.head_split(src, 0, heads, hd, w, (one, zero)), base)
    q = O.head_split(src, 0, heads, hd, w, (zero, one))
    assert np.array_equal(q[..., 0::2], -base[..., 1::2]) and np.array_equal(q[..., 1::2], base[..., 0::2])


def test_rope_row_indexing():
    """cos / sin are indexed by the row: a quarter turn on row 1 only."""
    rows, heads, hd = 3, 2, 8
    src, _, _ = _case(3, rows, heads * hd, heads, hd)
    c = np.ones((rows, hd // 2), np.float32)
    s = np.zeros((rows, hd // 2), np.float32)
    c[1], s[1] = 0.0, 1.0
    got = O.head_split(src, 0, heads, hd, None, (c, s))
    plain = O.head_split(src, 0, heads, hd)
    assert np.array_equal(got[:, [0, 2]], plain[:, [0, 2]])
    assert np.array_equal(got[:, 1, 0::2], -plain[:, 1, 1::2])


def test_constant_row_normalises_to_weight():
    """x = 0.5 everywhere, eps = 0: mean of squares 0.25 exactly, inv = 2,
    so the output is the weight, bit for bit."""
    heads, hd = 12, 128
    src = np.full((2, heads * hd), 0.5, np.float32)
    w = np.random.default_rng(4).standard_normal(heads * hd).astype(np.float32)
    got = O.head_split(src, 0, heads, hd, w, eps=0.0)
    assert np.array_equal(got.transpose(1, 0, 2).reshape(2, -1), np.stack([w, w]))


def test_rms_over_all_heads():
    """Heads at different scales: the normaliser is one per row."""
    heads, hd = 4, 32
    src, w, _ = _case(5, 3, heads * hd, heads, hd)
    src *= np.repeat(np.float32([1, 10, 100, 1000]), hd)[None, :]
    got = O.head_split(src, 0, heads, hd, np.ones(heads * hd, np.float32))
    x = src.astype(np.float64)
    per_row = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-6)
    assert np.allclose(got.transpose(1, 0, 2).reshape(3, -1), per_row, rtol=2e-6, atol=0)

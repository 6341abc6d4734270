"""Pins the oracle's restatement of the reference norms (crates/lightx2v-cpu/
src/lib.rs:328-400) without a device: against an independent float64
statement, closed forms and exact element-wise identities."""

import numpy as np
import pytest

import oracle as O


def _ln64(x, kind, w=None, b=None, mods=None, scale=0, shift=0, eps=1e-6):
    x = x.astype(np.float64)
    mean = x.mean(axis=1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
    n = (x - mean) / np.sqrt(var + eps)
    if kind == 0:
        return n * w.astype(np.float64) + b.astype(np.float64)
    return n * (1.0 + mods[scale].astype(np.float64)) + mods[shift].astype(np.float64)


def _data(seed, rows, dim):
    rng = O.Rng(seed)
    x = (rng.normal(rows * dim) * np.float32(2.0) + np.float32(0.5)).reshape(rows, dim)
    mods = (rng.normal(6 * dim) * np.float32(0.1)).reshape(6, dim)
    w = (1 + rng.normal(dim) * np.float32(0.1)).astype(np.float32)
    b = (rng.normal(dim) * np.float32(0.1)).astype(np.float32)
    return x.astype(np.float32), mods.astype(np.float32), w, b


@pytest.mark.parametrize("dim", [8, 100, 1536, 3072])
def test_layer_norm_vs_f64(dim):
    x, mods, w, b = _data(3 + dim, 17, dim)
    for kind in (0, 1):
        got = O.layer_norm(x, kind, w, b, mods, scale=1, shift=0)
        want = _ln64(x, kind, w, b, mods, scale=1, shift=0)
        assert np.max(np.abs(got - want)) <= 2e-5 * np.max(np.abs(want))


def test_layer_norm_closed_forms():
    dim = 64
    mods = np.zeros((6, dim), np.float32)
    mods[4] = np.linspace(-1, 1, dim, dtype=np.float32)   # shift
    mods[5] = np.linspace(0, 2, dim, dtype=np.float32)    # scale
    # constant rows: var 0, every normalized value 0, the output is exactly the shift / bias
    x = np.full((3, dim), 7.25, np.float32)
    assert np.array_equal(O.layer_norm(x, 1, mods=mods, scale=5, shift=4), np.broadcast_to(mods[4], (3, dim)))
    b = np.arange(dim, dtype=np.float32)
    assert np.array_equal(O.layer_norm(x, 0, np.ones(dim, np.float32), b), np.broadcast_to(b, (3, dim)))
    # rows of +-c: mean exactly 0, var exactly c^2, n = +-c / sqrt(c^2 + eps)
    c = np.float32(3.0)
    x = np.tile(np.array([c, -c], np.float32), (2, dim // 2))
    eps = np.float32(1e-6)
    n = c * (np.float32(1.0) / np.sqrt(c * c + eps))
    got = O.layer_norm(x, 1, mods=mods, scale=5, shift=4, eps=float(eps))
    want = (np.where(x > 0, n, -n) * (np.float32(1.0) + mods[5]) + mods[4]).astype(np.float32)
    assert np.array_equal(got, want)
    # Mod uses 1 + mods[scale]: with a zero scale row it is the plain LN
    z = np.zeros((6, dim), np.float32)
    assert np.array_equal(O.layer_norm(x, 1, mods=z, scale=2, shift=3, eps=float(eps)),
                          np.where(x > 0, n, -n).astype(np.float32))


def test_layer_norm_shift_and_scale_invariance():
    x, mods, w, b = _data(5, 9, 512)
    ref = O.layer_norm(x, 0, w, b)
    moved = O.layer_norm(x * np.float32(4.0) + np.float32(100.0), 0, w, b)
    assert np.max(np.abs(moved - ref)) <= 2e-4 * np.max(np.abs(ref))


def test_residual_norm_and_gate_residual_exact():
    x, mods, w, b = _data(7, 11, 96)
    a = (O.Rng(8).normal(11 * 96) * np.float32(0.5)).reshape(11, 96).astype(np.float32)
    h, normed = O.residual_norm(x, a, mods, 2, 1, scale=1, shift=0)
    assert np.array_equal(h, x + a * mods[2])                 # one multiply, one add, both rounded
    assert np.array_equal(normed, O.layer_norm(h, 1, mods=mods, scale=1, shift=0))
    h0, n0 = O.residual_norm(x, a, mods, None, 0, w, b)
    assert np.array_equal(h0, x + a)                          # no gate: a * 1.0
    assert np.array_equal(n0, O.layer_norm(h0, 0, w, b))
    assert np.array_equal(O.gate_residual(x, a, mods, 3), x + a * mods[3])

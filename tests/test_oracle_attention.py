"""Pins the oracle's restatement of the reference attention
(crates/lightx2v-cpu/src/lib.rs:155-203) without a device: against an
independent float64 softmax attention, closed forms and the mask rules."""

import numpy as np
import pytest

import oracle as O


def _attn64(q, k, v, mask=None):
    heads, sq, d = q.shape
    s = np.einsum("hqd,hkd->hqk", q.astype(np.float64), k.astype(np.float64)) / np.sqrt(d)
    if mask is not None:
        s = np.where(mask[None], s, -np.inf)
    s = s - s.max(axis=2, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=2, keepdims=True)
    o = np.einsum("hqk,hkd->hqd", p, v.astype(np.float64))
    return o.transpose(1, 0, 2).reshape(sq, heads * d)


def _qkv(seed, heads, sq, sk, d):
    rng = O.Rng(seed)
    q = rng.normal(heads * sq * d).reshape(heads, sq, d).astype(np.float32)
    k = rng.normal(heads * sk * d).reshape(heads, sk, d).astype(np.float32)
    v = rng.normal(heads * sk * d).reshape(heads, sk, d).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("heads,sq,sk,d", [(2, 5, 7, 16), (3, 33, 65, 64), (1, 8, 300, 128)])
def test_attention_vs_f64(heads, sq, sk, d):
    q, k, v = _qkv(heads * 100 + sk, heads, sq, sk, d)
    got = O.attention(q, k, v)
    assert np.max(np.abs(got - _attn64(q, k, v))) <= 1e-5
    mask = (np.arange(sk)[None, :] * sq <= (np.arange(sq)[:, None] + 1) * sk)  # every row keeps key 0
    got = O.attention(q, k, v, mask)
    assert np.max(np.abs(got - _attn64(q, k, v, mask))) <= 1e-5


def test_attention_closed_forms():
    heads, sq, sk, d = 2, 4, 6, 8
    q, k, v = _qkv(9, heads, sq, sk, d)
    # one key: the output is that key's value row for every query
    out = O.attention(q, k[:, :1], v[:, :1])
    assert np.array_equal(out, np.repeat(v[:, 0][None], sq, axis=0).reshape(sq, heads * d))
    # zero queries: uniform softmax, the output is the mean of v
    out = O.attention(np.zeros_like(q), k, v)
    assert np.allclose(out, np.repeat(v.mean(axis=1)[None], sq, axis=0).reshape(sq, heads * d), atol=1e-6)
    # a mask that keeps one key per query selects that key's value exactly
    mask = np.zeros((sq, sk), bool)
    keep = np.array([5, 0, 3, 3])
    mask[np.arange(sq), keep] = True
    out = O.attention(q, k, v, mask).reshape(sq, heads, d)
    for i in range(sq):
        assert np.array_equal(out[i], v[:, keep[i]])
    # heads are merged as [sq, heads * d] with head h at columns h*d .. h*d + d
    out = O.attention(q, k, v).reshape(sq, heads, d)
    assert np.allclose(out[:, 1], O.attention(q[1:], k[1:], v[1:]), atol=0)


def test_attention_threads_bit_identical():
    q, k, v = _qkv(3, 3, 17, 40, 32)
    assert np.array_equal(O.attention(q, k, v, nthreads=1), O.attention(q, k, v, nthreads=8))

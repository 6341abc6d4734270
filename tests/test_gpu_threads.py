"""Two contexts driven from two threads at once (the trait's threading
rule, crates/lightx2v-core/src/backend.rs: one context per thread at a
time; crates/lightx2v-wgpu/src/lib.rs:182-183 moves a backend into a worker
thread).  Each thread creates its context, allocates, uploads a weight,
grows and frees the context-owned staging (bf16 bias conversion, the
per-token activation workspace, the residual workspace) over and over,
and destroys its context, while the other does the same.  ctypes drops the
GIL for every foreign call, so the calls overlap in the library.

Each thread's outputs must equal what the same calls give on one thread.
"""

import threading

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O

pytestmark = pytest.mark.gpu


def _work(seed, iters, out, err):
    try:
        be = H.HipBackend(0)
        be.set_act_dtype(H.DTYPE_BF16)
        res = []
        for it in range(iters):
            m, k, n = 64 + 32 * (it % 3), 256, 128 + 64 * (it % 2)
            x = O.Rng(seed + it).normal(m * k)
            wf = O.Rng(seed + 100 + it).normal(n * k).reshape(n, k) * np.float32(0.02)
            q, s = O.fp8_quantize(wf, n, k, k, True)
            w = be.weight_fp8(q, s, n, k, k)
            xb = be.upload(x)
            bb = be.upload(O.Rng(seed + 200 + it).normal(n) * np.float32(0.01))  # bf16 bias: staged to f32
            yb = be.alloc(m * n)
            be.linear(xb, 0, m, w, bb, H.ACT_GELU_TANH, yb, 0)
            hb = be.upload(np.ones(m * n, np.float32))
            md = be.alloc(6 * n, H.DTYPE_F32)
            be.fill_normal(md, seed + it, 0.1)
            be.linear_residual(xb, 0, m, w, bb, 0, hb, 0, md, 5)
            res.append((be.download(yb), be.download(hb)))
            for b in (xb, bb, yb, hb, md):
                b.free()
            w.free()
        be.close()
        out[seed] = res
    except BaseException as e:  # noqa: BLE001 -- reported by the main thread
        err.append(e)


def test_two_contexts_two_threads():
    iters = 12
    solo, err = {}, []
    for seed in (1, 1000):
        _work(seed, iters, solo, err)
    assert not err, err
    par = {}
    ts = [threading.Thread(target=_work, args=(seed, iters, par, err)) for seed in (1, 1000)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in ts), "a thread did not finish"
    assert not err, err
    for seed in (1, 1000):
        for (ya, ha), (yb, hb) in zip(solo[seed], par[seed]):
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))
            assert np.array_equal(ha.view(np.uint32), hb.view(np.uint32))

"""Pre-quantized (E4M3) activation buffers and HIP-graph replay of the linear
path.  Neither has a reference counterpart (the reference keeps activations
f32, crates/lightx2v-core/src/backend.rs:9-11, and batches wgpu dispatches,
crates/lightx2v-wgpu/src/lib.rs:441-505); both must give exactly what the
plain Backend::linear path gives on the same inputs."""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import fp8_weight, normal, q8_weight, u32

pytestmark = pytest.mark.gpu


def _setup(be, M=300, K=1536, N=640, xdt=H.DTYPE_BF16):
    x = normal(71, M * K).reshape(M, K)
    _, q, s = fp8_weight(72, N, K, K)
    b = normal(73, N, 0.01)
    w = be.weight_fp8(q, s, N, K, K)
    bb = be.upload(b)
    be.set_act_dtype(xdt)
    try:
        xb = be.upload(x)
    finally:
        be.set_act_dtype(H.DTYPE_F32)
    return x, xb, w, bb


def test_e4m3_buffer_matches_internal_quantization(be):
    M, K, N = 300, 1536, 640
    x, xb, w, bb = _setup(be, M, K, N)
    xq = be.alloc_e4m3(M, K)
    assert xq.dtype == H.DTYPE_E4M3 and len(xq) == M * K
    be.quantize_act(xb, 0, M, xq)
    # the stored codes and scales are the oracle's per-token quantization
    qw, sw = O.act_quant_e4m3(O.bf16_round(x))
    dec = (O.e4m3_decode_ocp(qw.ravel()).reshape(M, K) * sw[:, None]).astype(np.float32)
    assert np.array_equal(u32(be.download(xq).reshape(M, K)), u32(dec))
    for act in (H.ACT_NONE, H.ACT_GELU_TANH):
        y1, y2 = be.alloc(M * N), be.alloc(M * N)
        be.linear(xb, 0, M, w, bb, act, y1, 0)
        be.linear(xq, 0, M, w, bb, act, y2, 0)
        assert np.array_equal(u32(be.download(y1)), u32(be.download(y2)))
    # row offsets on both sides
    xq2 = be.alloc_e4m3(100, K)
    be.quantize_act(xb, 150, 100, xq2)
    y3 = be.alloc(120 * N)
    be.linear(xq2, 10, 90, w, bb, H.ACT_NONE, y3, 30)
    y1 = be.alloc(M * N)
    be.linear(xb, 0, M, w, bb, H.ACT_NONE, y1, 0)
    assert np.array_equal(u32(be.download(y3).reshape(120, N)[30:]),
                          u32(be.download(y1).reshape(M, N)[160:250]))


def test_e4m3_buffer_errors(be):
    M, K, N = 64, 256, 128
    x, xb, w, bb = _setup(be, M, K, N)
    xq = be.alloc_e4m3(M, K)
    be.quantize_act(xb, 0, M, xq)
    _, q8, s8 = q8_weight(5, N, K, 32)
    w8 = be.weight_q8(q8, s8, N, K, 32)
    y = be.alloc(M * N)
    with pytest.raises(H.HipError) as e:
        be.linear(xq, 0, M, w8, bb, H.ACT_NONE, y, 0)
    assert e.value.status == H.ERR_UNSUPPORTED
    with pytest.raises(H.HipError) as e:
        be.write(xq, np.zeros(4, np.float32))
    assert e.value.status == H.ERR_BAD_ARG
    with pytest.raises(H.HipError) as e:
        be.quantize_act(xb, 0, M + 1, xq)
    assert e.value.status == H.ERR_BAD_SHAPE
    xq_bad = be.alloc_e4m3(M, K // 2)
    with pytest.raises(H.HipError) as e:
        be.linear(xq_bad, 0, M, w, bb, H.ACT_NONE, y, 0)
    assert e.value.status == H.ERR_BAD_SHAPE


def test_graph_replays_match_eager(be):
    """Capture quantize_act + three linears (one reading the pre-quantized
    buffer, one quantizing internally, one chained on the first's bf16
    output) and replay it three times with eager work and synchronisation
    in between; every replay equals the eager run bit for bit."""
    M, K, N = 300, 1536, 640
    x, xb, w, bb = _setup(be, M, K, N)
    _, q2, s2 = fp8_weight(74, K, N, N)
    w2 = be.weight_fp8(q2, s2, K, N, N)
    xq = be.alloc_e4m3(M, K)
    ya = be.alloc(M * N, H.DTYPE_BF16)
    yb = be.alloc(M * N)
    yc = be.alloc(M * K)

    def seq():
        be.quantize_act(xb, 0, M, xq)
        be.linear(xq, 0, M, w, bb, H.ACT_GELU_TANH, ya, 0)
        be.linear(xb, 0, M, w, bb, H.ACT_NONE, yb, 0)
        be.linear(ya, 0, M, w2, None, H.ACT_NONE, yc, 0)

    seq()  # eager; also sizes the workspace before capture
    want = [u32(be.download(b)).copy() for b in (ya, yb, yc)]
    be.graph_begin()
    seq()
    g = be.graph_end()
    for rep in range(3):
        for b in (ya, yb, yc):  # eager work between replays: clobber the outputs
            be.write(b, np.full(len(b), np.float32(rep + 1)))
        be.sync()
        g.launch()
        be.sync()
        got = [u32(be.download(b)) for b in (ya, yb, yc)]
        for gg, ww in zip(got, want):
            assert np.array_equal(gg, ww), f"replay {rep} differs"
    g.free()


def test_graph_capture_refuses_allocation(be):
    M, K, N = 64, 256, 128
    x, xb, w, bb = _setup(be, M, K, N)
    y = be.alloc(M * N)
    be.linear(xb, 0, M, w, bb, H.ACT_NONE, y, 0)
    be.graph_begin()
    with pytest.raises(H.HipError) as e:
        be.alloc(16)
    assert e.value.status == H.ERR_UNSUPPORTED
    with pytest.raises(H.HipError) as e:
        be.sync()
    assert e.value.status == H.ERR_UNSUPPORTED
    be.linear(xb, 0, M, w, bb, H.ACT_NONE, y, 0)
    g = be.graph_end()
    g.launch()
    be.sync()
    g.free()

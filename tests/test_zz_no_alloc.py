"""lx2v_hip_linear_noalloc (no counterpart in the reference; for callers that
cannot allocate) against lx2v_hip_linear through the C ABI: the same plan
and kernels run, so outputs are bit-identical.  Two calls in a row, the
second with a smaller input (the scratch keeps the first call's contents);
the paths that use scratch (per-token e4m3 activations, a bf16 bias's f32
copy, f32 activations' bf16 copy for the bf16 GEMM, split K's partial sums)
and the ones that need none; capture in a HIP graph on a fresh context,
where any workspace growth would fail, replayed against the eager result;
a call too large for the scratch refused with a message; two contexts on
one device, the second refused with LX2V_ERR_BUSY while the first one's
work on the scratch is in flight.
"""

import os

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import fp8_weight, normal, q8_weight, u32

pytestmark = pytest.mark.gpu


def _buf(be, a, dtype):
    b = be.alloc(a.size, dtype)
    be.write(b, np.ascontiguousarray(a, np.float32).ravel())
    return b


def _pair(be, x, w, bias, act, n, ydt):
    rows = x.len_rows
    y1 = be.alloc(rows * n, ydt)
    y2 = be.alloc(rows * n, ydt)
    be.linear(x.buf, 0, rows, w, bias, act, y1, 0)
    be.linear_noalloc(x.buf, 0, rows, w, bias, act, y2, 0)
    return be.download(y1), be.download(y2)


class _X:
    def __init__(self, be, a, dtype):
        self.buf = _buf(be, a, dtype)
        self.len_rows = a.shape[0]


@pytest.fixture(scope="module")
def be():
    if H.device_count() == 0:
        pytest.skip("no HIP device visible")
    b = H.HipBackend(0)
    yield b
    b.close()


def test_two_calls_second_smaller(be):
    # 1: the chunk's O projection, bf16 activations and bias (both staged), bf16 out
    M, K, N = 4680, 1536, 1536
    _, q, s = fp8_weight(1, N, K, K)
    w = be.weight_fp8(q, s, N, K, K)
    x = _X(be, normal(2, M * K).reshape(M, K), H.DTYPE_BF16)
    b16 = _buf(be, normal(3, N, 0.01), H.DTYPE_BF16)
    a, b = _pair(be, x, w, b16, H.ACT_NONE, N, H.DTYPE_BF16)
    assert np.array_equal(u32(a), u32(b))
    # 2: smaller, f32 activations, f32 bias, GELU, f32 out
    M, K, N = 300, 512, 640
    _, q, s = fp8_weight(4, N, K, K)
    w = be.weight_fp8(q, s, N, K, K)
    x = _X(be, normal(5, M * K).reshape(M, K), H.DTYPE_F32)
    a, b = _pair(be, x, w, be.upload(normal(6, N, 0.01)), H.ACT_GELU_TANH, N, H.DTYPE_F32)
    assert np.array_equal(u32(a), u32(b))


def test_other_paths(be):
    # group-128 FP8 weights
    M, K, N = 257, 1024, 512
    _, q, s = fp8_weight(7, N, K, 128)
    w = be.weight_fp8(q, s, N, K, 128)
    x = _X(be, normal(8, M * K).reshape(M, K), H.DTYPE_BF16)
    a, b = _pair(be, x, w, None, H.ACT_NONE, N, H.DTYPE_F32)
    assert np.array_equal(u32(a), u32(b))
    # Q8 with f32 activations: the bf16 GEMM's activation copy in scratch
    _, q8, s8 = q8_weight(9, N, K, 32)
    w8 = be.weight_q8(q8, s8, N, K, 32)
    x = _X(be, normal(10, M * K).reshape(M, K), H.DTYPE_F32)
    a, b = _pair(be, x, w8, None, H.ACT_GELU_TANH, N, H.DTYPE_F32)
    assert np.array_equal(u32(a), u32(b))
    # pre-quantized e4m3 activations: no scratch needed
    xq = be.alloc_e4m3(M, K)
    be.quantize_act(x.buf, 0, M, xq)
    y1, y2 = be.alloc(M * N), be.alloc(M * N)
    be.linear(xq, 0, M, w, None, H.ACT_NONE, y1, 0)
    be.linear_noalloc(xq, 0, M, w, None, H.ACT_NONE, y2, 0)
    assert np.array_equal(u32(be.download(y1)), u32(be.download(y2)))


def test_graph_capture_on_a_fresh_context():
    """A fresh context has no workspace: `linear` on bf16 activations would
    have to allocate one, which graph capture refuses; the no-alloc variant
    records, and every replay equals the eager `linear`."""
    fresh = H.HipBackend(0)
    try:
        M, K, N = 1000, 1536, 768
        _, q, s = fp8_weight(11, N, K, K)
        w = fresh.weight_fp8(q, s, N, K, K)
        x = _buf(fresh, normal(12, M * K).reshape(M, K), H.DTYPE_BF16)
        bias = _buf(fresh, normal(13, N, 0.01), H.DTYPE_BF16)
        y = fresh.alloc(M * N, H.DTYPE_BF16)
        fresh.graph_begin()
        with pytest.raises(H.HipError) as e:
            fresh.linear(x, 0, M, w, bias, H.ACT_NONE, y, 0)
        assert e.value.status == H.ERR_UNSUPPORTED
        fresh.linear_noalloc(x, 0, M, w, bias, H.ACT_NONE, y, 0)
        g = fresh.graph_end()
        want_y = fresh.alloc(M * N, H.DTYPE_BF16)
        fresh.linear(x, 0, M, w, bias, H.ACT_NONE, want_y, 0)
        want = u32(fresh.download(want_y)).copy()
        other = _buf(fresh, normal(14, 300 * K).reshape(300, K), H.DTYPE_BF16)
        for rep in range(3):
            # eager work between replays that reuses the scratch with other values
            fresh.linear_noalloc(other, 0, 300, w, None, H.ACT_GELU_TANH, fresh.alloc(300 * N), 0)
            fresh.write(y, np.full(M * N, np.float32(rep + 1)))
            fresh.sync()
            g.launch()
            fresh.sync()
            assert np.array_equal(u32(fresh.download(y)), want), f"replay {rep}"
        g.free()
    finally:
        fresh.close()


def _profiled_names(be, fn):
    be.profile_reset()
    be.profile_enable(True)
    try:
        fn()
        st = be.profile_stats()
    finally:
        be.profile_enable(False)
        be.profile_reset()
    return {k for k in st if k.startswith("gemm")}


def _one_pass(fn):
    old = os.environ.get("LIGHTX2V_HIP_FP8_SPLITK")
    os.environ["LIGHTX2V_HIP_FP8_SPLITK"] = "0"
    try:
        return fn()
    finally:
        if old is None:
            os.environ.pop("LIGHTX2V_HIP_FP8_SPLITK")
        else:
            os.environ["LIGHTX2V_HIP_FP8_SPLITK"] = old


@pytest.mark.parametrize("M,K,N", [(880, 14336, 3072), (300, 8192, 1536)])
def test_split_k_shapes(be, monkeypatch, M, K, N):
    """Split K in two (LIGHTX2V_HIP_FP8_SPLITK=2, read per call: at these
    shapes the planner itself prefers the 128 x 128 one-per-CU tile) at
    config 5's FFN down at M = 880, then a smaller shape (the scratch keeps
    the first call's partial sums): the no-alloc call plans the same split,
    its partial sums in the scratch, bit for bit; the one-pass kernel's sums
    differ, so the split did run."""
    monkeypatch.setenv("LIGHTX2V_HIP_FP8_SPLITK", "2")
    cfg = "c0k2"
    _, q, s = fp8_weight(21 + M, N, K, K, 0.015)
    w = be.weight_fp8(q, s, N, K, K)
    x = _X(be, normal(22 + M, M * K).reshape(M, K), H.DTYPE_BF16)
    bias = be.upload(normal(23 + M, N, 0.01))
    y = be.alloc(M * N, H.DTYPE_BF16)
    assert _profiled_names(be, lambda: be.linear(x.buf, 0, M, w, bias, H.ACT_NONE, y, 0)) == {f"gemm_fp8_e4m3.{cfg}"}
    a, b = _pair(be, x, w, bias, H.ACT_NONE, N, H.DTYPE_BF16)
    assert np.array_equal(u32(a), u32(b))
    a, b = _pair(be, x, w, bias, H.ACT_NONE, N, H.DTYPE_F32)
    assert np.array_equal(u32(a), u32(b))
    one = _one_pass(lambda: _pair(be, x, w, bias, H.ACT_NONE, N, H.DTYPE_F32))
    assert np.array_equal(u32(one[0]), u32(one[1]))
    assert not np.array_equal(u32(one[0]), u32(a)), "the split and one-pass f32 sums should differ somewhere"
    # pre-quantized activations with GELU and f32 output: partial sums only
    xq = be.alloc_e4m3(M, K)
    be.quantize_act(x.buf, 0, M, xq)
    y1, y2 = be.alloc(M * N), be.alloc(M * N)
    be.linear(xq, 0, M, w, bias, H.ACT_GELU_TANH, y1, 0)
    be.linear_noalloc(xq, 0, M, w, bias, H.ACT_GELU_TANH, y2, 0)
    assert np.array_equal(u32(be.download(y1)), u32(be.download(y2)))


def test_second_context_busy_while_first_in_flight(be):
    """The device's scratch is held by one context at a time: a second
    context's call while the first one's scratch work is still running fails
    with LX2V_ERR_BUSY (and enqueues nothing); once that work is done the
    second context takes the array over, and then the first is refused until
    the second's work is done."""
    M, K, N = 880, 14336, 3072
    _, q, s = fp8_weight(31, N, K, K, 0.015)
    other = H.HipBackend(0)
    try:
        wa, wb = be.weight_fp8(q, s, N, K, K), other.weight_fp8(q, s, N, K, K)
        xa = _buf(be, normal(32, M * K).reshape(M, K), H.DTYPE_BF16)
        xb = _buf(other, normal(32, M * K).reshape(M, K), H.DTYPE_BF16)
        ya, yb = be.alloc(M * N), other.alloc(M * N)
        be.sync()
        for _ in range(40):  # ~2 ms of queued scratch work on the first context
            be.linear_noalloc(xa, 0, M, wa, None, H.ACT_NONE, ya, 0)
        with pytest.raises(H.HipError) as e:
            other.linear_noalloc(xb, 0, M, wb, None, H.ACT_NONE, yb, 0)
        assert e.value.status == H.ERR_BUSY and "another context" in str(e.value)
        be.sync()
        for _ in range(40):
            other.linear_noalloc(xb, 0, M, wb, None, H.ACT_NONE, yb, 0)
        with pytest.raises(H.HipError) as e:
            be.linear_noalloc(xa, 0, M, wa, None, H.ACT_NONE, ya, 0)
        assert e.value.status == H.ERR_BUSY
        other.sync()
        be.linear_noalloc(xa, 0, M, wa, None, H.ACT_NONE, ya, 0)
        ref = be.alloc(M * N)
        be.linear(xa, 0, M, wa, None, H.ACT_NONE, ref, 0)
        assert np.array_equal(u32(be.download(ya)), u32(be.download(ref)))
        assert np.array_equal(u32(other.download(yb)), u32(be.download(ref)))
    finally:
        other.close()


def test_too_large_is_refused(be, monkeypatch):
    M, K, N = 6000, 8960, 256  # 6000 x 8960 e4m3 codes > 48 MiB
    _, q, s = fp8_weight(15, N, K, K)
    w = be.weight_fp8(q, s, N, K, K)
    x = be.alloc(M * K, H.DTYPE_BF16)
    y = be.alloc(M * N)
    with pytest.raises(H.HipError) as e:
        be.linear_noalloc(x, 0, M, w, None, H.ACT_NONE, y, 0)
    assert e.value.status == H.ERR_UNSUPPORTED and "scratch" in str(e.value)
    # 5000 rows: 42.7 MiB of codes fit; with K split two ways the partial
    # sums (9.8 MiB) do not fit beside them, and 4000 rows fit both
    be.linear_noalloc(x, 0, 5000, w, None, H.ACT_NONE, y, 0)
    monkeypatch.setenv("LIGHTX2V_HIP_FP8_SPLITK", "2")
    with pytest.raises(H.HipError) as e:
        be.linear_noalloc(x, 0, 5000, w, None, H.ACT_NONE, y, 0)
    assert e.value.status == H.ERR_UNSUPPORTED
    be.linear_noalloc(x, 0, 4000, w, None, H.ACT_NONE, y, 0)

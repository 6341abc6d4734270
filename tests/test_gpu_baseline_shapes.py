"""Backend::linear at the benchmark's full shapes.

Two kinds of check, both through the C ABI:
  * exact properties over the whole output: X rows that are (scaled) one-hot
    vectors pick one weight column, so Y = dequantize(W)[:, k] + b bit for
    bit when the scales are powers of two (every product and the single
    non-zero sum term are then exact).  This pins the packed layouts, nibble
    order, group indexing, tile edges and the epilogue over every output
    element of the 4680-token shapes;
  * parity of sampled rows of a seeded random problem against the oracle
    (same tolerances as test_gpu_linear.py).
Seeds: X 1001, W 1002, bias 1003, plus 10 x the config index.
"""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import FP8_TIGHT, W16_TIGHT, assert_close, normal, oracle_w16, oracle_w8a8, u32

pytestmark = pytest.mark.gpu

M = 4680  # 3 latent frames x 30 x 52 patches at 832x480


def _onehot(rows, k, value):
    x = np.zeros((rows, k), np.float32)
    x[np.arange(rows), np.arange(rows) % k] = value
    return x


def _pow2_scales(rng, shape):
    return np.exp2(rng.integers(-9, -4, shape)).astype(np.float32)


def _run(be, x, w, b, act=H.ACT_NONE, x_dtype=H.DTYPE_F32, y_dtype=H.DTYPE_F32):
    n = w.info()["rows"]
    be.set_act_dtype(x_dtype)
    try:
        xb = be.upload(x)
    finally:
        be.set_act_dtype(H.DTYPE_F32)
    bb = be.upload(b) if b is not None else None
    yb = be.alloc(x.shape[0] * n, y_dtype)
    be.linear(xb, 0, x.shape[0], w, bb, act, yb, 0)
    return be.download(yb).reshape(x.shape[0], n)


def _expect_onehot(wd, b, rows):
    k = wd.shape[1]
    cols = np.arange(rows) % k
    return (wd[:, cols].T + b[None, :]).astype(np.float32)


def test_cfg1_fp8_onehot_exact(be):
    N, K = 1536, 1536
    rng = np.random.default_rng(1)
    q = O.e4m3_encode_canon(normal(1012, N * K, 100.0)).reshape(N, K)
    s = _pow2_scales(rng, (N, 1))
    b = normal(1013, N, 0.01)
    w = be.weight_fp8(q, s, N, K, K)
    y = _run(be, _onehot(M, K, 448.0), w, b)
    want = _expect_onehot(O.fp8_dequantize(q, s, N, K, K) * np.float32(448.0), b, M)
    assert np.array_equal(u32(y), u32(want))


def test_cfg2_q8_g32_onehot_exact(be):
    N, K, g = 8960, 1536, 32
    rng = np.random.default_rng(2)
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = _pow2_scales(rng, (N, K // g))
    b = normal(1023, N, 0.01)
    w = be.weight_q8(q, s, N, K, g)
    y = _run(be, _onehot(M, K, 1.0), w, b, x_dtype=H.DTYPE_BF16)
    assert np.array_equal(u32(y), u32(_expect_onehot(O.q8_dequantize(q, s, N, K, g), b, M)))


def test_cfg3_q4_g32_onehot_exact(be):
    N, K, g = 1536, 8960, 32
    rng = np.random.default_rng(3)
    c = rng.integers(0, 16, (N, K)).astype(np.uint8)
    s = _pow2_scales(rng, (N, K // g))
    z = np.full((N, K // g), 8.0, np.float32)
    b = normal(1033, N, 0.01)
    w = be.weight_q4(O.q4_pack(c), s, z, N, K, g, packed=True)
    y = _run(be, _onehot(M, K, 1.0), w, b, x_dtype=H.DTYPE_BF16)
    assert np.array_equal(u32(y), u32(_expect_onehot(O.q4_dequantize(c, s, z, N, K, g), b, M)))


SAMPLE = np.sort(np.random.default_rng(0).choice(M, 96, replace=False))


def test_cfg1_fp8_sampled_rows(be):
    N, K = 1536, 1536
    x = normal(1011, M * K).reshape(M, K)
    wf = normal(1012, N * K, 0.02).reshape(N, K)
    q, s = O.fp8_quantize(wf, N, K, K, True)
    b = normal(1013, N, 0.01)
    w = be.weight_fp8(q, s, N, K, K)
    y = _run(be, x, w, b)
    assert np.all(np.isfinite(y))
    xs = x[SAMPLE]
    assert_close(y[SAMPLE], oracle_w8a8(xs, q, s, K, b, 0), *FP8_TIGHT, what="cfg1 vs oracle(e4m3 acts)")
    assert_close(y[SAMPLE], O.linear(xs, O.fp8_dequantize(q, s, N, K, K), b, 0, nthreads=8), 4e-2, 0.3,
                 what="cfg1 vs f32 oracle")


def test_cfg2_q8_gelu_sampled_rows(be):
    N, K, g = 8960, 1536, 32
    x = O.bf16_round(normal(1021, M * K).reshape(M, K))
    wf = normal(1022, N * K, 0.02).reshape(N, K)
    q, s = O.q8_quantize(wf, N, K, g)
    b = normal(1023, N, 0.01)
    w = be.weight_q8(q, s, N, K, g)
    y = _run(be, x, w, b, act=H.ACT_GELU_TANH, x_dtype=H.DTYPE_BF16, y_dtype=H.DTYPE_BF16)
    wd = O.q8_dequantize(q, s, N, K, g)
    want = oracle_w16(x[SAMPLE], wd, b, 1)
    assert_close(y[SAMPLE], want, 4e-3, 1e-2, what="cfg2 vs oracle(bf16 operands), bf16 out")
    assert_close(y[SAMPLE], O.linear(x[SAMPLE], wd, b, 1, nthreads=8), 6e-3, 0.05, what="cfg2 vs f32 oracle")


@pytest.mark.parametrize("heavy", [False, True])
def test_cfg3_q4_sampled_rows(be, heavy):
    N, K, g = 1536, 8960, 32
    x = O.bf16_round(O.gelu_tanh(normal(1031, M * K).reshape(M, K)))
    wf = normal(1032, N * K, 0.02).reshape(N, K)
    if heavy:
        wf[:, np.arange(K) % 100 == 37] *= np.float32(20.0)
    c, s, z = O.q4_quantize_sym(wf, N, K, g)
    b = normal(1033, N, 0.01)
    w = be.weight_q4(O.q4_pack(c), s, z, N, K, g, packed=True)
    y = _run(be, x, w, b, x_dtype=H.DTYPE_BF16)
    wd = O.q4_dequantize(c, s, z, N, K, g)
    assert_close(y[SAMPLE], oracle_w16(x[SAMPLE], wd, b, 0), *W16_TIGHT, what="cfg3 vs oracle(bf16 operands)")
    assert_close(y[SAMPLE], O.linear(x[SAMPLE], wd, b, 0, nthreads=8), 5e-3, 0.05, what="cfg3 vs f32 oracle")


@pytest.mark.parametrize("rows", [2640, 880])
@pytest.mark.parametrize("K,N", [(3072, 9216), (3072, 3072), (3072, 14336), (14336, 3072)])
def test_cfg5_wan22_5b_fp8(be, rows, K, N):
    """Wan2.2-TI2V-5B shapes, FP8 per-channel weights ~N(0, 0.015) with
    per-token dynamic e4m3 activations (bf16 in)."""
    x = O.bf16_round(normal(1051, rows * K).reshape(rows, K))
    wf = normal(1052 + N, N * K, 0.015).reshape(N, K)
    q, s = O.fp8_quantize(wf, N, K, K, True)
    b = normal(1053, N, 0.01)
    w = be.weight_fp8(q, s, N, K, K)
    y = _run(be, x, w, b, x_dtype=H.DTYPE_BF16)
    sample = SAMPLE[SAMPLE < rows][:48]
    assert_close(y[sample], oracle_w8a8(x[sample], q, s, K, b, 0), *FP8_TIGHT, what="cfg5 vs oracle(e4m3 acts)")

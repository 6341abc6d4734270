"""MX e4m3 activations: the FFN-up -> FFN-down hand-off format (no
reference counterpart -- the reference keeps activations f32,
crates/lightx2v-core/src/backend.rs:9-11).  The quantizer is checked bit
for bit against the oracle's (itself pinned against an independent numpy
restatement and closed-form properties in test_oracle.py); the GEMMs that
read MX activations against the oracle GEMM on the same dequantized
operands, to the fp8-MFMA tolerance; the GEMM epilogue that writes MX
output bit for bit against the standalone quantizer applied to the same
GEMM's f32 output."""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import FP8_TIGHT, assert_close, fp8_weight, normal, u32

pytestmark = pytest.mark.gpu


def _upload(be, x, dtype):
    be.set_act_dtype(dtype)
    try:
        return be.upload(x)
    finally:
        be.set_act_dtype(H.DTYPE_F32)


def _mx_data(seed, rows, cols):
    """Normal rows with per-block magnitudes spread over ~2^+-40, plus edge blocks."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x *= np.exp2(rng.integers(-40, 40, (rows, cols // 32))).repeat(32, axis=1).astype(np.float32)
    x[0, :32] = 0.0
    if rows > 1:
        x[1, :32] = 448.0
        x[1, 32 % cols:32 % cols + 1] = -448.0 * 1.5
    if rows > 2 and cols >= 64:
        x[2, 32:64] = np.float32(1.0625)  # RNE ties after scaling by 2^0
        x[2, 32] = 448.0
    return x


@pytest.mark.parametrize("rows,cols,x_row", [(1, 32, 0), (77, 96, 3), (300, 1536, 0), (64, 8960, 5)])
@pytest.mark.parametrize("xdt", [H.DTYPE_F32, H.DTYPE_BF16])
def test_quantize_mx_bit_exact(be, rows, cols, x_row, xdt):
    x = _mx_data(100 + rows, x_row + rows, cols)
    if xdt == H.DTYPE_BF16:
        x = O.bf16_round(x).reshape(x.shape)
    xb = _upload(be, x, xdt)
    xq = be.alloc_mx(rows + 2, cols)
    be.quantize_mx(xb, x_row, rows, xq)
    q, s = be.download_mx(xq, rows + 2, cols)
    qo, so = O.act_quant_mx(x[x_row:])
    assert np.array_equal(q[:rows], qo) and np.array_equal(s[:, :rows], so)
    # download decodes code * 2^k exactly
    d = be.download(xq).reshape(rows + 2, cols)[:rows]
    assert np.array_equal(u32(d), u32(O.dequant_mx(qo, so)))


# (M, K, N): the planner puts these on the 128x128 three-per-CU tile, the
# 256x128 one-per-CU tile and the 128x256 two-per-CU tile respectively.
MX_SHAPES = [(300, 1536, 640), (77, 256, 160), (3000, 512, 2048), (2100, 2048, 2048), (1000, 1536, 8960)]


@pytest.mark.parametrize("group", ["channel", 128])
@pytest.mark.parametrize("M,K,N", MX_SHAPES + [(4680, 8960, 1536)])  # + the chunk's FFN down
def test_linear_mx_input_vs_oracle(be, M, K, N, group):
    """MX e4m3 input, per-channel or group-128 weights (group 128: the
    256 x 128 grouped tile, the block-scaled MFMA into each group's partial
    sums): the oracle on the decoded input, FP8_TIGHT."""
    g = K if group == "channel" else 128
    x = normal(11 + M, M * K).reshape(M, K)
    _, q, s = fp8_weight(12 + N, N, K, g)
    b = normal(13, N, 0.01)
    w = be.weight_fp8(q, s, N, K, g)
    bb = be.upload(b)
    xb = _upload(be, x, H.DTYPE_F32)
    xq = be.alloc_mx(M + 16, K)
    be.quantize_mx(xb, 0, M, xq)
    # every row from offset 16 (or 0) through the GEMM; the oracle on a
    # sample of rows that includes the first and last tiles' rows
    r0 = 16 if M > 64 else 0
    rows = M - r0
    y = be.alloc((rows + 3) * N)
    be.linear(xq, r0, rows, w, bb, H.ACT_NONE, y, 3)
    got = be.download(y).reshape(rows + 3, N)[3:]
    pick = np.unique(np.concatenate([np.arange(min(rows, 40)), np.arange(max(0, rows - 40), rows),
                                     np.random.default_rng(M).choice(rows, min(rows, 64), replace=False)]))
    qx, sx = O.act_quant_mx(x)
    xd = O.dequant_mx(qx, sx)[r0:][pick]
    want = O.linear(xd, O.fp8_dequantize(q, s, N, K, g), b, 0, nthreads=8)
    assert_close(got[pick], want, *FP8_TIGHT, what=f"MX-input fp8 GEMM (group {g}) vs oracle")


@pytest.mark.parametrize("M,K,N", MX_SHAPES + [(4680, 1536, 8960)])
@pytest.mark.parametrize("act", [H.ACT_NONE, H.ACT_GELU_TANH])
@pytest.mark.parametrize("xmx", [False, True])
def test_linear_mx_output_is_quantized_f32_output(be, M, K, N, act, xmx):
    """y (MXE4M3) == quantize_mx(y (F32)) of the same contraction, every
    row, codes and scales bit for bit (y_row offsets on both sides)."""
    x = normal(21 + M, M * K).reshape(M, K)
    _, q, s = fp8_weight(22 + N, N, K, K)
    b = normal(23, N, 0.1)
    w = be.weight_fp8(q, s, N, K, K)
    bb = be.upload(b)
    xb = _upload(be, x, H.DTYPE_BF16)
    if xmx:
        xin = be.alloc_mx(M, K)
        be.quantize_mx(xb, 0, M, xin)
    else:
        xin = xb
    y32 = be.alloc((M + 2) * N)
    be.linear(xin, 0, M, w, bb, act, y32, 2)
    ymx = be.alloc_mx(M + 5, N)
    be.linear(xin, 0, M, w, bb, act, ymx, 5)
    ref = be.alloc_mx(M, N)
    be.quantize_mx(y32, 2, M, ref)
    q1, s1 = be.download_mx(ymx, M + 5, N)
    q2, s2 = be.download_mx(ref, M, N)
    assert np.array_equal(q1[5:], q2) and np.array_equal(s1[:, 5:], s2)


@pytest.mark.parametrize("M,K,N", [(300, 512, 640), (4680, 1536, 8960)])
def test_linear_mx_output_g128(be, M, K, N):
    """Group-128 FP8 weights writing MX output (the 256x128 grouped tile):
    codes and scales equal quantize_mx of the f32 output, bit for bit."""
    x = normal(24 + M, M * K).reshape(M, K)
    _, q, s = fp8_weight(25 + N, N, K, 128)
    b = normal(26, N, 0.1)
    w = be.weight_fp8(q, s, N, K, 128)
    bb = be.upload(b)
    xb = _upload(be, x, H.DTYPE_BF16)
    y32 = be.alloc(M * N)
    be.linear(xb, 0, M, w, bb, H.ACT_GELU_TANH, y32, 0)
    ymx = be.alloc_mx(M, N)
    be.linear(xb, 0, M, w, bb, H.ACT_GELU_TANH, ymx, 0)
    ref = be.alloc_mx(M, N)
    be.quantize_mx(y32, 0, M, ref)
    q1, s1 = be.download_mx(ymx, M, N)
    q2, s2 = be.download_mx(ref, M, N)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


def test_mx_ffn_chain(be):
    """FFN up (GELU, MX out) -> FFN down (MX in): the second GEMM equals the
    oracle on the first one's decoded output; the chain stays within the
    fp8 bound of the f32 oracle."""
    M, D, F = 520, 512, 1536
    x = normal(31, M * D).reshape(M, D)
    _, q1, s1 = fp8_weight(32, F, D, D)
    _, q2, s2 = fp8_weight(33, D, F, F)
    b1, b2 = normal(34, F, 0.01), normal(35, D, 0.01)
    w1, w2 = be.weight_fp8(q1, s1, F, D, D), be.weight_fp8(q2, s2, D, F, F)
    bb1, bb2 = be.upload(b1), be.upload(b2)
    xb = _upload(be, x, H.DTYPE_BF16)
    h = be.alloc_mx(M, F)
    y = be.alloc(M * D)
    be.linear(xb, 0, M, w1, bb1, H.ACT_GELU_TANH, h, 0)
    be.linear(h, 0, M, w2, bb2, H.ACT_NONE, y, 0)
    hd = be.download(h).reshape(M, F)
    got = be.download(y).reshape(M, D)
    w2d = O.fp8_dequantize(q2, s2, D, F, F)
    assert_close(got, O.linear(hd, w2d, b2, 0, nthreads=8), *FP8_TIGHT, what="FFN down on MX input")
    w1d = O.fp8_dequantize(q1, s1, F, D, D)
    hf = O.linear(O.bf16_round(x).reshape(M, D), w1d, b1, H.ACT_GELU_TANH, nthreads=8)
    assert_close(got, O.linear(hf, w2d, b2, 0, nthreads=8), 4e-2, 0.3, what="MX FFN chain vs f32 oracle")


def test_mx_graph_replays_match_eager(be):
    M, D, F = 300, 512, 1024
    x = normal(41, M * D).reshape(M, D)
    _, q1, s1 = fp8_weight(42, F, D, D)
    _, q2, s2 = fp8_weight(43, D, F, F)
    w1, w2 = be.weight_fp8(q1, s1, F, D, D), be.weight_fp8(q2, s2, D, F, F)
    xb = _upload(be, x, H.DTYPE_BF16)
    h = be.alloc_mx(M, F)
    y = be.alloc(M * D, H.DTYPE_BF16)

    def seq():
        be.linear(xb, 0, M, w1, None, H.ACT_GELU_TANH, h, 0)
        be.linear(h, 0, M, w2, None, H.ACT_NONE, y, 0)

    seq()
    want_h = be.download_mx(h, M, F)
    want_y = u32(be.download(y)).copy()
    be.graph_begin()
    seq()
    g = be.graph_end()
    for rep in range(3):
        # eager work between replays: other values into both outputs
        be.linear(xb, 0, M, w1, None, H.ACT_NONE, h, 0)
        be.write(y, np.full(M * D, np.float32(rep + 1)))
        be.sync()
        g.launch()
        be.sync()
        gh = be.download_mx(h, M, F)
        assert np.array_equal(gh[0], want_h[0]) and np.array_equal(gh[1], want_h[1]), f"replay {rep}"
        assert np.array_equal(u32(be.download(y)), want_y), f"replay {rep}"
    g.free()


def test_mx_errors(be):
    with pytest.raises(H.HipError) as e:
        be.alloc_mx(4, 48)
    assert e.value.status == H.ERR_BAD_SHAPE
    M, K, N = 64, 256, 128
    x = normal(51, M * K).reshape(M, K)
    _, q, s = fp8_weight(52, N, K, K)
    w = be.weight_fp8(q, s, N, K, K)
    xb = _upload(be, x, H.DTYPE_F32)
    xq = be.alloc_mx(M, K)
    be.quantize_mx(xb, 0, M, xq)
    y = be.alloc(M * N)
    with pytest.raises(H.HipError) as e:  # MX input row offset not a multiple of 16
        be.linear(xq, 8, 16, w, None, H.ACT_NONE, y, 0)
    assert e.value.status == H.ERR_UNSUPPORTED
    from helpers import q8_weight
    _, q8, s8 = q8_weight(53, N, K, 32)
    w8 = be.weight_q8(q8, s8, N, K, 32)
    with pytest.raises(H.HipError) as e:
        be.linear(xq, 0, M, w8, None, H.ACT_NONE, y, 0)
    assert e.value.status == H.ERR_UNSUPPORTED
    _, qg, sg = fp8_weight(55, N, K, 64)  # group 64: no MX output, no MX input
    wg = be.weight_fp8(qg, sg, N, K, 64)
    with pytest.raises(H.HipError) as e:
        be.linear(xb, 0, M, wg, None, H.ACT_NONE, be.alloc_mx(M, N), 0)
    assert e.value.status == H.ERR_UNSUPPORTED
    with pytest.raises(H.HipError) as e:
        be.linear(xq, 0, M, wg, None, H.ACT_NONE, y, 0)
    assert e.value.status == H.ERR_UNSUPPORTED
    with pytest.raises(H.HipError) as e:
        be.write(xq, np.zeros(4, np.float32))
    assert e.value.status == H.ERR_BAD_ARG
    e4 = be.alloc_e4m3(M, K)
    with pytest.raises(H.HipError) as e:
        be.quantize_mx(xb, 0, M, e4)
    assert e.value.status == H.ERR_BAD_ARG
    with pytest.raises(H.HipError) as e:
        be.linear(xq, 0, M, w, None, H.ACT_NONE, be.alloc_mx(M, 160), 0)  # y cols != N
    assert e.value.status == H.ERR_BAD_SHAPE

"""Native f32 weights (Backend::weight, WeightQuant::Native, quant.rs:28-30)
on the bf16 MFMA: the weight's bf16 copy made at upload times bf16
activations, f32 accumulation (k_gemm_bf16_dma), at the non-block linear
shapes of Wan2.1-1.3B -- patch_embed 64 -> 1536 (dit.rs:540-561), proj_out
1536 -> 64 (dit.rs:772-781), the text MLP 4096 -> 1536 (GELU) -> 1536 on
512 tokens (dit.rs:450-469) -- and ragged ones.

Checked against the oracle on the bf16-rounded operands (W16_TIGHT: the
products are exact in f32, only the summation order differs) and against
the plain f32 oracle with the stated native tolerance (two bf16 roundings
of relative 2^-9 per product: rel-L2 <= 4e-3 measured-bound, max-abs <=
2e-2 of the output's range).  LX2V_NATIVE_F32 restores the f32 operands
(the scalar kernel) within 1e-6 of the oracle.
"""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import W16_TIGHT, assert_close, normal, oracle_w16, rel_l2, u32

pytestmark = pytest.mark.gpu

NATIVE_TOL = (4e-3, 2e-2)

# (what, rows, K, N, act)
SHAPES = [
    ("patch_embed", 4680, 64, 1536, H.ACT_NONE),
    ("proj_out", 4680, 1536, 64, H.ACT_NONE),
    ("text_mlp1", 512, 4096, 1536, H.ACT_GELU_TANH),
    ("text_mlp2", 512, 1536, 1536, H.ACT_NONE),
    ("ragged", 77, 320, 130, H.ACT_GELU_TANH),
    ("one_row", 1, 128, 256, H.ACT_NONE),
]


def _linear(be, x, w, b, act, x_dtype, y_dtype, rows, n):
    be.set_act_dtype(x_dtype)
    try:
        xb = be.upload(x)
    finally:
        be.set_act_dtype(H.DTYPE_F32)
    yb = be.alloc(rows * n, y_dtype)
    be.linear(xb, 0, rows, w, be.upload(b), act, yb, 0)
    return be.download(yb).reshape(rows, n)


def _kernels(be, fn):
    be.profile_reset()
    be.profile_enable(True)
    try:
        fn()
        st = be.profile_stats()
    finally:
        be.profile_enable(False)
        be.profile_reset()
    return {k for k in st if k.startswith("gemm")}


@pytest.mark.parametrize("what,rows,K,N,act", SHAPES)
@pytest.mark.parametrize("x_dtype", [H.DTYPE_F32, H.DTYPE_BF16])
def test_native_bf16_mfma_vs_oracle(be, what, rows, K, N, act, x_dtype):
    x = normal(301 + K, rows * K).reshape(rows, K)
    if x_dtype == H.DTYPE_BF16:
        x = O.bf16_round(x)
    wf = normal(302 + N, N * K, 0.02).reshape(N, K)
    b = normal(303, N, 0.01)
    w = be.weight(wf, N, K)
    ks = _kernels(be, lambda: _linear(be, x, w, b, act, x_dtype, H.DTYPE_F32, rows, N))
    assert ks == {"gemm_bf16_native"}, ks
    y = _linear(be, x, w, b, act, x_dtype, H.DTYPE_F32, rows, N)
    assert np.all(np.isfinite(y))
    assert_close(y, oracle_w16(x, wf, b, act), *W16_TIGHT, what=f"{what} vs oracle(bf16 operands)")
    assert_close(y, O.linear(x, wf, b, act, nthreads=8), *NATIVE_TOL, what=f"{what} vs f32 oracle")
    y16 = _linear(be, x, w, b, act, x_dtype, H.DTYPE_BF16, rows, N)
    assert np.array_equal(u32(O.bf16_round(y)), u32(y16)), \
        "bf16 output = f32 output rounded"


def test_native_f32_mode_exact(be):
    rows, K, N = 200, 256, 192
    x = normal(311, rows * K).reshape(rows, K)
    wf = normal(312, N * K, 0.05).reshape(N, K)
    b = normal(313, N, 0.01)
    w = be.weight(wf, N, K)
    be.set_native_mode(H.NATIVE_F32)
    try:
        ks = _kernels(be, lambda: _linear(be, x, w, b, H.ACT_GELU_TANH, H.DTYPE_F32, H.DTYPE_F32, rows, N))
        y = _linear(be, x, w, b, H.ACT_GELU_TANH, H.DTYPE_F32, H.DTYPE_F32, rows, N)
    finally:
        be.set_native_mode(H.NATIVE_BF16)
    assert ks == {"gemm_generic"}, ks
    assert_close(y, O.linear(x, wf, b, 1, nthreads=8), 1e-6, 1e-5, what="native f32 mode")
    # and the default mode is measurably coarser, inside the native tolerance
    y_bf = _linear(be, x, w, b, H.ACT_GELU_TANH, H.DTYPE_F32, H.DTYPE_F32, rows, N)
    r = rel_l2(y_bf, y)
    assert 1e-5 < r <= NATIVE_TOL[0], r


def test_native_mode_rejects_unknown(be):
    with pytest.raises(H.HipError):
        be.set_native_mode(7)


def test_native_weight_noalloc_matches_linear(be):
    rows, K, N = 300, 192, 320
    x = normal(321, rows * K).reshape(rows, K)
    wf = normal(322, N * K, 0.02).reshape(N, K)
    b = normal(323, N, 0.01)
    w = be.weight(wf, N, K)
    xb, bb = be.upload(x), be.upload(b)
    y1, y2 = be.alloc(rows * N), be.alloc(rows * N)
    be.linear(xb, 0, rows, w, bb, H.ACT_NONE, y1, 0)
    be.linear_noalloc(xb, 0, rows, w, bb, H.ACT_NONE, y2, 0)
    assert np.array_equal(be.download(y1).view(np.uint32), be.download(y2).view(np.uint32))

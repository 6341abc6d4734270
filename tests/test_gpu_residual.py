"""linear + gate_residual fused (lx2v_hip_linear_residual): the add
h += act(x W^T + b) * mods[gate] riding in the FP8 GEMM's epilogue, as the
DiT runs it after the attention O, cross-attention O and FFN-down
projections (crates/lightx2v-model/src/dit.rs: `linear` into a temporary,
then `gate_residual`, backend.rs:243-252).

Bar: bit-identical to the unfused pair (linear into a temporary of h's
dtype, then gate_residual) on every path -- fused in the epilogue (FP8,
one scale per channel, K % 128 == 0; per-token or MX e4m3 input) and the
two-launch fallback elsewhere (Q8, grouped FP8, K % 128 != 0).  Against the
oracle (the reference's linear on the same e4m3 operands, then its
gate_residual in f32): FP8_TIGHT on the update h_new - h for f32 h.
"""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import FP8_TIGHT, assert_close, fp8_weight, normal, oracle_w8a8, q8_weight, u32

pytestmark = pytest.mark.gpu


def _up(be, a, dtype):
    b = be.alloc(a.size, dtype)
    be.write(b, np.ascontiguousarray(a, np.float32).ravel())
    return b


def _pair_and_fused(be, xb, x_row, rows, w, bias, act, h0, h_row, mods_b, gate, dtype, n):
    """(fused result, unfused result) as host arrays of h."""
    h1, h2 = _up(be, h0, dtype), _up(be, h0, dtype)
    be.linear_residual(xb, x_row, rows, w, bias, act, h1, h_row, mods_b, gate)
    tmp = be.alloc(rows * n, dtype)
    be.linear(xb, x_row, rows, w, bias, act, tmp, 0)
    view = be.alloc(rows * n, dtype)  # h rows [h_row, +rows) through a copy: gate_residual has no row offset
    be.copy(h2, h_row * n, view, 0, rows * n)
    be.gate_residual(view, tmp, rows, n, mods_b, gate)
    be.copy(view, 0, h2, h_row * n, rows * n)
    return be.download(h1), be.download(h2)


@pytest.mark.parametrize("dtype", [H.DTYPE_BF16, H.DTYPE_F32])
@pytest.mark.parametrize("m,k,n,act", [(4680, 1536, 1536, H.ACT_NONE), (300, 1536, 1536, H.ACT_GELU_TANH),
                                       (1000, 8960, 1536, H.ACT_NONE), (77, 256, 384, H.ACT_NONE)])
def test_fused_equals_pair(be, dtype, m, k, n, act):
    rng_seed = 10 + m + k
    x = normal(rng_seed, m * k).reshape(m, k)
    _, q, s = fp8_weight(rng_seed + 1, n, k, k)
    w = be.weight_fp8(q, s, n, k, k)
    bias = be.upload(normal(rng_seed + 2, n, 0.1))
    mods = normal(rng_seed + 3, 6 * n, 0.3)
    mods_b = be.upload(mods)
    h0 = normal(rng_seed + 4, m * n, 2.0)
    be.set_act_dtype(dtype)
    try:
        xb = _up(be, x, dtype)
        got, want = _pair_and_fused(be, xb, 0, m, w, bias, act, h0, 0, mods_b, 4, dtype, n)
    finally:
        be.set_act_dtype(H.DTYPE_F32)
    assert np.array_equal(u32(got), u32(want)), f"{(u32(got) != u32(want)).sum()} of {got.size} differ"


def test_fused_row_offsets_and_mx_input(be):
    """x_row / h_row offsets; FFN-down's MX e4m3 input (written by FFN-up's
    epilogue in the bench) through the fused epilogue."""
    m, k, n = 640, 1024, 512
    x = normal(41, m * k).reshape(m, k)
    _, q, s = fp8_weight(42, n, k, k)
    w = be.weight_fp8(q, s, n, k, k)
    mods_b = be.upload(normal(43, 6 * n, 0.3))
    h0 = normal(44, (m + 32) * n, 2.0)
    be.set_act_dtype(H.DTYPE_BF16)
    try:
        xb = _up(be, x, H.DTYPE_BF16)
        got, want = _pair_and_fused(be, xb, 16, 400, w, None, H.ACT_NONE, h0, 32, mods_b, 2, H.DTYPE_BF16, n)
        assert np.array_equal(u32(got), u32(want))
        xm = be.alloc_mx(m, k)
        be.quantize_mx(xb, 0, m, xm)
        got, want = _pair_and_fused(be, xm, 16, 400, w, None, H.ACT_NONE, h0, 32, mods_b, 5, H.DTYPE_BF16, n)
        assert np.array_equal(u32(got), u32(want))
    finally:
        be.set_act_dtype(H.DTYPE_F32)
    # rows outside [h_row, h_row + 400) are untouched
    assert np.array_equal(u32(got[:32 * n]), u32(O.bf16_round(h0[:32 * n])))


def test_fallback_paths_equal_pair(be):
    """Q8, grouped FP8 and K % 128 != 0 run the pair as two launches."""
    m, n = 200, 256
    mods_b = be.upload(normal(51, 6 * n, 0.3))
    for kind, k in (("q8", 512), ("fp8_grouped", 512), ("fp8_k", 272)):
        x = normal(52 + k, m * k).reshape(m, k)
        if kind == "q8":
            _, q, s = q8_weight(53, n, k, 32)
            w = be.weight_q8(q, s, n, k, 32)
        else:
            group = 128 if kind == "fp8_grouped" else k
            _, q, s = fp8_weight(54, n, k, group)
            w = be.weight_fp8(q, s, n, k, group)
        h0 = normal(55, m * n, 2.0)
        be.set_act_dtype(H.DTYPE_BF16)
        try:
            xb = _up(be, x, H.DTYPE_BF16)
            got, want = _pair_and_fused(be, xb, 0, m, w, None, H.ACT_NONE, h0, 0, mods_b, 1, H.DTYPE_BF16, n)
        finally:
            be.set_act_dtype(H.DTYPE_F32)
        assert np.array_equal(u32(got), u32(want)), kind


def test_against_oracle(be):
    """f32 h: the update equals the oracle's linear on the same e4m3 operands
    times the gate row (the reference's gate_residual is h + a * g in f32)."""
    m, k, n = 300, 1536, 768
    x = normal(61, m * k).reshape(m, k)
    _, q, s = fp8_weight(62, n, k, k)
    w = be.weight_fp8(q, s, n, k, k)
    bias = normal(63, n, 0.1)
    mods = normal(64, 6 * n, 0.3).reshape(6, n)
    h0 = normal(65, m * n, 2.0).reshape(m, n)
    xb, hb = _up(be, x, H.DTYPE_F32), _up(be, h0, H.DTYPE_F32)
    be.linear_residual(xb, 0, m, w, be.upload(bias), H.ACT_GELU_TANH, hb, 0, be.upload(mods.ravel()), 3)
    got = be.download(hb).reshape(m, n)
    y = oracle_w8a8(x, q, s, k, bias, H.ACT_GELU_TANH)
    want = O.gate_residual(h0, y, mods, 3)
    assert_close(got - h0, want - h0, *FP8_TIGHT, what="linear_residual update")


def test_errors(be):
    m, k, n = 8, 256, 128
    _, q, s = fp8_weight(71, n, k, k)
    w = be.weight_fp8(q, s, n, k, k)
    xb = be.upload(normal(72, m * k))
    mods_b = be.upload(normal(73, 6 * n))
    with pytest.raises(H.HipError):  # h too short
        be.linear_residual(xb, 0, m, w, None, H.ACT_NONE, be.alloc(m * n - 1), 0, mods_b, 0)
    with pytest.raises(H.HipError):  # gate row past the table
        be.linear_residual(xb, 0, m, w, None, H.ACT_NONE, be.alloc(m * n), 0, mods_b, 6)
    with pytest.raises(H.HipError):  # E4M3 h
        be.linear_residual(xb, 0, m, w, None, H.ACT_NONE, be.alloc_e4m3(m, n), 0, mods_b, 0)

"""The benchmark chunk's GEMMs at their own shapes (config 4: the Wan2.1-1.3B
block-linear set for one 3-frame chunk, crates/lightx2v-model/src/dit.rs:
602-759), called the way bench.py calls them: bf16 activation buffers,
FP8 per-channel weights, the planner's kernel configuration for each shape.

Per call site: every output row computed; a sample of rows (first and last
tiles included) against the oracle on the same e4m3 operands (FP8_TIGHT,
f32 output); the bf16 output equal to the f32 output rounded, bit for bit;
and the kernel configuration that ran, read from the profile report, equal
to the one the bench's chunk uses.  The FFN pair runs as in the bench: FFN
up with GELU writes MX e4m3 (checked bit for bit against the standalone MX
quantizer of its f32 output), FFN down reads it (against the oracle on the
decoded MX input), and the chain against the plain f32 oracle (4e-2).

The same shapes with group-128 weights (the reference's FP8 default) run
the grouped tiles, each asserted by name.  The bench's other timed launches
run here too: the 30 layers' cross-attention K/V projections as one call
over their concatenated weights (512 x 1536 -> 92160), and config 5's
Wan2.2-5B shapes with the bf16 output the bench writes.
"""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import FP8_TIGHT, assert_bits_equal, assert_close, normal, oracle_w8a8, u32

pytestmark = pytest.mark.gpu

DIM, FFN, TEXT, M = 1536, 8960, 512, 4680

# (name, rows, K, N, act, the configuration the planner picks on 256 CUs
# with per-channel / group-128 weights, bf16 output)
SITES = [
    ("qkv", M, DIM, 3 * DIM, H.ACT_NONE, "c7", "c6.g128"),
    ("o", M, DIM, DIM, H.ACT_NONE, "c1", "c1.g128"),
    ("kv2", TEXT, DIM, 2 * DIM, H.ACT_NONE, "c10", "c10.g128"),
    ("ffn1", M, DIM, FFN, H.ACT_GELU_TANH, "c9", "c7.g128"),
    ("ffn2", M, FFN, DIM, H.ACT_NONE, "c1", "c1.g128"),
]


def _pick(rows, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([np.arange(32), np.arange(rows - 32, rows),
                                     rng.choice(rows, 64, replace=False)]))


def _bf16_buf(be, x):
    be.set_act_dtype(H.DTYPE_BF16)
    try:
        return be.upload(x)
    finally:
        be.set_act_dtype(H.DTYPE_F32)


def _profiled(be, fn):
    be.profile_reset()
    be.profile_enable(True)
    try:
        fn()
        st = be.profile_stats()
    finally:
        be.profile_enable(False)
        be.profile_reset()
    return {k for k in st if k.startswith("gemm")}


@pytest.mark.parametrize("name,rows,K,N,act,cfg,cfg_g128", SITES)
@pytest.mark.parametrize("group", ["channel", 128])
def test_call_site(be, name, rows, K, N, act, cfg, cfg_g128, group):
    g = K if group == "channel" else 128
    x = O.bf16_round(normal(1001 + N, rows * K).reshape(rows, K))
    wf = normal(1002 + N, N * K, 0.02).reshape(N, K)
    q, s = O.fp8_quantize(wf, N, K, g, True)
    b = normal(1003 + N, N, 0.01)
    w = be.weight_fp8(q, s, N, K, g)
    xb, bb = _bf16_buf(be, x), be.upload(b)
    y16 = be.alloc(rows * N, H.DTYPE_BF16)
    y32 = be.alloc(rows * N, H.DTYPE_F32)
    ks = _profiled(be, lambda: be.linear(xb, 0, rows, w, bb, act, y16, 0))
    assert ks == {f"gemm_fp8_e4m3.{cfg if group == 'channel' else cfg_g128}"}, ks
    be.linear(xb, 0, rows, w, bb, act, y32, 0)
    got32 = be.download(y32).reshape(rows, N)
    got16 = be.download(y16).reshape(rows, N)
    assert np.all(np.isfinite(got32))
    assert_bits_equal(got16, O.bf16_round(got32), "bf16 output = f32 output rounded")
    p = _pick(rows, N)
    assert_close(got32[p], oracle_w8a8(x[p], q, s, g, b, act), *FP8_TIGHT, what=f"{name} g{g} vs oracle")


@pytest.mark.parametrize("group", ["channel", 128])
def test_ffn_pair_mx_handoff(be, group):
    """FFN up 4680x1536->8960 (GELU, MX output) -> FFN down 4680x8960->1536
    (MX input), as the bench chains them; both weights per-channel or both
    group 128."""
    g1 = DIM if group == "channel" else 128
    g2 = FFN if group == "channel" else 128
    x = O.bf16_round(normal(1101, M * DIM).reshape(M, DIM))
    w1f = normal(1102, FFN * DIM, 0.02).reshape(FFN, DIM)
    w2f = normal(1103, DIM * FFN, 0.02).reshape(DIM, FFN)
    q1, s1 = O.fp8_quantize(w1f, FFN, DIM, g1, True)
    q2, s2 = O.fp8_quantize(w2f, DIM, FFN, g2, True)
    b1, b2 = normal(1104, FFN, 0.01), normal(1105, DIM, 0.01)
    w1, w2 = be.weight_fp8(q1, s1, FFN, DIM, g1), be.weight_fp8(q2, s2, DIM, FFN, g2)
    xb, bb1, bb2 = _bf16_buf(be, x), be.upload(b1), be.upload(b2)
    h = be.alloc_mx(M, FFN)
    y = be.alloc(M * DIM, H.DTYPE_F32)
    ks = _profiled(be, lambda: (be.linear(xb, 0, M, w1, bb1, H.ACT_GELU_TANH, h, 0),
                                be.linear(h, 0, M, w2, bb2, H.ACT_NONE, y, 0)))
    if group == "channel":
        assert ks == {"gemm_fp8_e4m3.c9.mxout", "gemm_fp8_e4m3.c1.mxin"}, ks
    else:
        assert ks == {"gemm_fp8_e4m3.c7.g128.mxout", "gemm_fp8_e4m3.c1.g128.mxin"}, ks
    # FFN up: MX output == MX quantizer of the same GEMM's f32 output, whole tensor
    h32 = be.alloc(M * FFN, H.DTYPE_F32)
    be.linear(xb, 0, M, w1, bb1, H.ACT_GELU_TANH, h32, 0)
    ref = be.alloc_mx(M, FFN)
    be.quantize_mx(h32, 0, M, ref)
    qa, sa = be.download_mx(h, M, FFN)
    qb, sb = be.download_mx(ref, M, FFN)
    assert np.array_equal(qa, qb) and np.array_equal(sa, sb)
    p = _pick(M, 7)
    hf32 = be.download(h32).reshape(M, FFN)
    assert_close(hf32[p], oracle_w8a8(x[p], q1, s1, g1, b1, 1), *FP8_TIGHT, what="FFN up vs oracle")
    del hf32
    # FFN down on the decoded MX input
    hd = be.download(h).reshape(M, FFN)[p]
    got = be.download(y).reshape(M, DIM)[p]
    w2d = O.fp8_dequantize(q2, s2, DIM, FFN, g2)
    assert_close(got, O.linear(hd, w2d, b2, 0, nthreads=8), *FP8_TIGHT, what="FFN down on MX input vs oracle")
    # the chain against the plain f32 oracle
    w1d = O.fp8_dequantize(q1, s1, FFN, DIM, g1)
    hf = O.linear(x[p], w1d, b1, 1, nthreads=8)
    assert_close(got, O.linear(hf, w2d, b2, 0, nthreads=8), 4e-2, 0.3, what="FFN chain vs f32 oracle")


@pytest.mark.parametrize("group,cfg", [("channel", "c9"), (128, "c6.g128")])
def test_cross_kv_30_layers_one_call(be, group, cfg):
    """The bench's per-step cross-attention K/V call: the 30 layers' K/V
    weights concatenated by rows ([30 x 2 x 1536, 1536], scales and bias
    concatenated the same way, as the bench builds them), one linear over
    the 512 text tokens, 512 x 1536 -> 92160: on the persistent 256 x 256
    tile with per-channel weights, on the persistent 256 x 128 one with
    group-128 weights.  bf16 output == f32 output rounded over the whole
    tensor; sampled rows against the oracle over every column."""
    rows, K, N = TEXT, DIM, 30 * 2 * DIM
    g = K if group == "channel" else group
    x = O.bf16_round(normal(1201, rows * K).reshape(rows, K))
    wf = normal(1202, N * K, 0.02).reshape(N, K)
    q, s = O.fp8_quantize(wf, N, K, g, True)
    del wf
    b = normal(1203, N, 0.01)
    w = be.weight_fp8(q, s, N, K, g)
    xb, bb = _bf16_buf(be, x), be.upload(b)
    y16 = be.alloc(rows * N, H.DTYPE_BF16)
    y32 = be.alloc(rows * N, H.DTYPE_F32)
    assert _profiled(be, lambda: be.linear(xb, 0, rows, w, bb, H.ACT_NONE, y16, 0)) == {f"gemm_fp8_e4m3.{cfg}"}
    be.linear(xb, 0, rows, w, bb, H.ACT_NONE, y32, 0)
    got32 = be.download(y32).reshape(rows, N)
    assert_bits_equal(be.download(y16), O.bf16_round(got32).ravel(), "bf16 output = f32 output rounded")
    p = np.array([0, 1, 2, 31, 32, 255, 256, 300, 480, 510, 511])
    assert_close(got32[p], oracle_w8a8(x[p], q, s, g, b, 0), *FP8_TIGHT, what="30-layer K/V call vs oracle")
    # each layer's slice is that layer's own K/V linear
    for l in (0, 17, 29):
        sl = slice(l * 2 * DIM, (l + 1) * 2 * DIM)
        assert_close(got32[p][:, sl], oracle_w8a8(x[p], q[sl], s[sl], g, b[sl], 0), *FP8_TIGHT, what=f"layer {l}")


# Config 5 (Wan2.2-TI2V-5B, per-token e4m3 activations) with the bf16 output
# the bench writes: (rows, K, N, the configuration the planner picks).
CFG5 = [(2640, 3072, 9216, "c1"), (2640, 3072, 3072, "c1"), (2640, 3072, 14336, "c9"), (2640, 14336, 3072, "c1"),
        (880, 3072, 9216, "c1"), (880, 3072, 3072, "c10"), (880, 3072, 14336, "c9"), (880, 14336, 3072, "c10")]


@pytest.mark.parametrize("rows,K,N,cfg", CFG5)
def test_cfg5_bf16_output(be, rows, K, N, cfg):
    x = O.bf16_round(normal(1051, rows * K).reshape(rows, K))
    wf = normal(1052 + N, N * K, 0.015).reshape(N, K)
    q, s = O.fp8_quantize(wf, N, K, K, True)
    b = normal(1053, N, 0.01)
    w = be.weight_fp8(q, s, N, K, K)
    xb, bb = _bf16_buf(be, x), be.upload(b)
    y16 = be.alloc(rows * N, H.DTYPE_BF16)
    y32 = be.alloc(rows * N, H.DTYPE_F32)
    assert _profiled(be, lambda: be.linear(xb, 0, rows, w, bb, H.ACT_NONE, y16, 0)) == {f"gemm_fp8_e4m3.{cfg}"}
    be.linear(xb, 0, rows, w, bb, H.ACT_NONE, y32, 0)
    got32 = be.download(y32).reshape(rows, N)
    got16 = be.download(y16).reshape(rows, N)
    assert_bits_equal(got16, O.bf16_round(got32), "bf16 output = f32 output rounded")
    p = _pick(rows, N)[:48]
    assert_close(got16[p], oracle_w8a8(x[p], q, s, K, b, 0), 4e-3, 1e-2, what="cfg5 bf16 out vs oracle(e4m3 acts)")
    assert_close(got32[p], oracle_w8a8(x[p], q, s, K, b, 0), *FP8_TIGHT, what="cfg5 f32 out vs oracle(e4m3 acts)")


@pytest.mark.parametrize("group", ["channel", 128])
@pytest.mark.parametrize("name,seed", [("o", 1301), ("o2", 1302)])
def test_o_on_mx_input(be, name, seed, group):
    """The headline chunk's O and cross-attn O: 4680 x 1536 -> 1536 on the MX
    e4m3 input attention's epilogue writes (here the standalone MX quantizer
    of bf16 N(0,1) values), bf16 output, as the bench runs them, per-channel
    or group-128 weights: the kernel configuration asserted; sampled rows
    against the oracle on the decoded MX input (FP8_TIGHT, f32 output) and
    against the plain f32 oracle on the bf16 values (4e-2)."""
    g = DIM if group == "channel" else 128
    x = O.bf16_round(normal(seed, M * DIM).reshape(M, DIM))
    wf = normal(seed + 1, DIM * DIM, 0.02).reshape(DIM, DIM)
    q, s = O.fp8_quantize(wf, DIM, DIM, g, True)
    b = normal(seed + 2, DIM, 0.01)
    w = be.weight_fp8(q, s, DIM, DIM, g)
    xb, bb = _bf16_buf(be, x), be.upload(b)
    xm = be.alloc_mx(M, DIM)
    be.quantize_mx(xb, 0, M, xm)
    y16 = be.alloc(M * DIM, H.DTYPE_BF16)
    y32 = be.alloc(M * DIM, H.DTYPE_F32)
    want = "gemm_fp8_e4m3.c1.mxin" if group == "channel" else "gemm_fp8_e4m3.c1.g128.mxin"
    assert _profiled(be, lambda: be.linear(xm, 0, M, w, bb, H.ACT_NONE, y16, 0)) == {want}
    be.linear(xm, 0, M, w, bb, H.ACT_NONE, y32, 0)
    got32 = be.download(y32).reshape(M, DIM)
    assert np.array_equal(u32(be.download(y16).reshape(M, DIM)), u32(O.bf16_round(got32)))
    p = _pick(M, seed)
    xd = be.download(xm).reshape(M, DIM)[p]  # the decoded MX input
    # the device decoder against the oracle's own MX quantizer of the same values
    qo, so = O.act_quant_mx(x[p])
    assert np.array_equal(u32(xd), u32(O.dequant_mx(qo, so)))
    wd = O.fp8_dequantize(q, s, DIM, DIM, g)
    assert_close(got32[p], O.linear(xd, wd, b, 0, nthreads=8), *FP8_TIGHT, what=f"{name} on MX input vs oracle")
    assert_close(got32[p], O.linear(x[p], wd, b, 0, nthreads=8), 4e-2, 0.3, what=f"{name} vs f32 oracle")

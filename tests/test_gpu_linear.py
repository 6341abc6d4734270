"""Backend::linear (crates/lightx2v-core/src/backend.rs:198-212) on the gfx950
kernels against the CPU oracle (crates/lightx2v-cpu/src/lib.rs:296-326).

Tolerances (rel-L2 over the output, max-abs as a fraction of max|y|):
  * against the oracle applied to the same rounded operands the device
    contracts (per-token e4m3 activations for FP8; bf16 activations and
    bf16-rounded dequantized weights for the bf16-MFMA path):
    W16_TIGHT / FP8_TIGHT from helpers.py (only the accumulation differs;
    the fp8 matrix cores' 64-product dot carries a measured 1.5e-5 rel-L2);
  * against the plain f32 oracle on the unrounded activations: FP8 (e4m3
    activations, 3 mantissa bits) rel-L2 <= 4e-2 (measured ~2.6e-2);
    bf16 paths rel-L2 <= 5e-3 (measured ~2.3e-3);
  * bf16 outputs add one bf16 rounding: rel-L2 <= 4e-3 against the oracle.
"""

import json
import os

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import (FP8_TIGHT, W16_TIGHT, assert_close, fp8_weight, normal, oracle_w16, oracle_w8a8,
                     q4_sym_weight, q8_weight, u32)

pytestmark = pytest.mark.gpu
GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "quant_kats.json")))



def run_linear(be, x, w, bias, act, y_dtype=H.DTYPE_F32, x_dtype=H.DTYPE_F32, x_row=0, y_row=0,
               rows=None):
    M, K = x.shape
    n = w.info()["rows"]
    rows = M - x_row if rows is None else rows
    bb = be.upload(bias) if bias is not None else None  # f32, as the oracle's
    be.set_act_dtype(x_dtype)
    try:
        xb = be.upload(x)
    finally:
        be.set_act_dtype(H.DTYPE_F32)
    yb = be.alloc((y_row + rows) * n, y_dtype)
    be.linear(xb, x_row, rows, w, bb, act, yb, y_row)
    return be.download(yb).reshape(y_row + rows, n)[y_row:]


def test_check_linear_f32_weight(be):
    """check.rs:74-103's hand case, tol 1e-6 (wgpu measured 0.0)."""
    g = GOLD["check_linear"]
    w = be.weight(np.array(g["w"], np.float32), g["n"], g["k"])
    y = run_linear(be, np.array(g["x"], np.float32).reshape(g["rows"], g["k"]), w,
                   np.array(g["b"], np.float32), H.ACT_NONE)
    assert np.max(np.abs(y.ravel() - np.array(g["want"]))) <= g["tolerance"]


# ---- FP8 per-output-channel: per-token e4m3 activations, fp8 MFMA ----------------------

FP8_SHAPES = [(64, 256, 192), (77, 272, 130), (300, 1536, 1536), (1, 128, 64), (257, 384, 513),
              (520, 1024, 640)]


@pytest.mark.parametrize("M,K,N", FP8_SHAPES)
def test_fp8_channel_vs_oracle(be, M, K, N):
    x = normal(1001 + M, M * K).reshape(M, K)
    _, q, s = fp8_weight(1002 + N, N, K, K)
    b = normal(1003, N, 0.01)
    w = be.weight_fp8(q, s, N, K, K)
    y = run_linear(be, x, w, b, H.ACT_NONE)
    assert_close(y, oracle_w8a8(x, q, s, K, b, 0), *FP8_TIGHT, what="fp8 vs oracle(same e4m3 acts)")
    wd = O.fp8_dequantize(q, s, N, K, K)
    assert_close(y, O.linear(x, wd, b, 0, nthreads=8), 4e-2, 0.3, what="fp8 vs f32 oracle")


@pytest.mark.parametrize("act", [H.ACT_NONE, H.ACT_GELU_TANH])
@pytest.mark.parametrize("ydt", [H.DTYPE_F32, H.DTYPE_BF16])
@pytest.mark.parametrize("xdt", [H.DTYPE_F32, H.DTYPE_BF16])
def test_fp8_epilogue_dtypes_offsets(be, act, ydt, xdt):
    M, K, N = 200, 512, 384
    x = normal(5, M * K).reshape(M, K)
    xs = x if xdt == H.DTYPE_F32 else O.bf16_round(x)
    _, q, s = fp8_weight(6, N, K, K)
    b = normal(7, N, 0.01)
    w = be.weight_fp8(q, s, N, K, K)
    y = run_linear(be, x, w, b, act, y_dtype=ydt, x_dtype=xdt, x_row=13, y_row=7, rows=150)
    want = oracle_w8a8(xs[13:163], q, s, K, b, act)
    if ydt == H.DTYPE_F32:
        assert_close(y, want, *FP8_TIGHT, what="fp8 epilogue")
    else:
        assert_close(y, want, 4e-3, 8e-3, what="fp8 epilogue bf16 out")


@pytest.mark.parametrize("M,K,N", [(77, 256, 130), (300, 1536, 1000), (513, 512, 2056), (1, 128, 8),
                                   (260, 384, 1540)])
def test_fp8_bf16_out_is_rounded_f32_out(be, M, K, N):
    """The bf16 output is the f32 output of the same contraction rounded to
    nearest-even bf16, bit for bit, ragged N included (N % 8 != 0 takes the
    per-element stores); the f32 output is checked against the oracle."""
    x = normal(2001 + M, M * K).reshape(M, K)
    _, q, s = fp8_weight(2002 + N, N, K, K)
    b = normal(2003, N, 0.01)
    w = be.weight_fp8(q, s, N, K, K)
    for act in (H.ACT_NONE, H.ACT_GELU_TANH):
        y32 = run_linear(be, x, w, b, act)
        y16 = run_linear(be, x, w, b, act, y_dtype=H.DTYPE_BF16)
        assert np.array_equal(u32(y16), u32(O.bf16_round(y32))), f"act {act}"
        assert_close(y32, oracle_w8a8(x, q, s, K, b, act), *FP8_TIGHT, what="fp8 f32 out")


@pytest.mark.parametrize("M,K,N,act,ydt", [(300, 1536, 1536, H.ACT_NONE, H.DTYPE_F32),
                                            (880, 3072, 1024, H.ACT_GELU_TANH, H.DTYPE_BF16),
                                            (129, 2048, 384, H.ACT_NONE, H.DTYPE_F32),
                                            (600, 1024, 512, H.ACT_GELU_TANH, H.DTYPE_MXE4M3)])
def test_fp8_split_k_vs_one_pass(be, monkeypatch, M, K, N, act, ydt):
    """Split K (Fp8Plan::splits: the 256 x 128 tiles' K range over S
    workgroups, partial sums reduced with the scales, bias and activation
    by a second pass), forced to 2 and 4 pieces, against the oracle to
    FP8_TIGHT and against the one-pass kernel (only the f32 summation order
    differs); MX output equals quantize_mx of the split path's own f32
    output."""
    x = normal(3001 + M, M * K).reshape(M, K)
    _, q, s = fp8_weight(3002 + N, N, K, K)
    b = normal(3003, N, 0.01)
    w = be.weight_fp8(q, s, N, K, K)
    want = oracle_w8a8(x, q, s, K, b, act)
    monkeypatch.setenv("LIGHTX2V_HIP_FP8_SPLITK", "0")
    one = run_linear(be, x, w, b, act)
    for pieces in ("2", "4"):
        monkeypatch.setenv("LIGHTX2V_HIP_FP8_SPLITK", pieces)
        y32 = run_linear(be, x, w, b, act)
        assert_close(y32, want, *FP8_TIGHT, what=f"split {pieces} vs oracle")
        assert_close(y32, one, 1e-6, 1e-5, what=f"split {pieces} vs one pass")
        if ydt == H.DTYPE_BF16:
            y16 = run_linear(be, x, w, b, act, y_dtype=H.DTYPE_BF16)
            assert np.array_equal(u32(y16), u32(O.bf16_round(y32)))
        elif ydt == H.DTYPE_MXE4M3:
            xb = be.alloc(M * K)
            be.write(xb, x)
            yf, ym, ref = be.alloc(M * N), be.alloc_mx(M, N), be.alloc_mx(M, N)
            be.linear(xb, 0, M, w, be.upload(b), act, yf, 0)
            be.linear(xb, 0, M, w, be.upload(b), act, ym, 0)
            be.quantize_mx(yf, 0, M, ref)
            c1, s1 = be.download_mx(ym, M, N)
            c2, s2 = be.download_mx(ref, M, N)
            assert np.array_equal(c1, c2) and np.array_equal(s1, s2)


def test_fp8_split_k_row_offsets(be, monkeypatch):
    """Split K with x_row / y_row offsets and a row count short of the
    buffers (the reduction's token scales, output rows and MX scale rows all
    start at the offsets): equal to the one-pass kernel up to f32 summation
    order, and to the oracle to FP8_TIGHT."""
    M, K, N = 400, 8192, 384
    x = normal(3101, M * K).reshape(M, K)
    _, q, s = fp8_weight(3102, N, K, K)
    b = normal(3103, N, 0.01)
    w = be.weight_fp8(q, s, N, K, K)
    monkeypatch.setenv("LIGHTX2V_HIP_FP8_SPLITK", "0")
    one = run_linear(be, x, w, b, H.ACT_GELU_TANH, x_row=37, y_row=11, rows=300)
    monkeypatch.setenv("LIGHTX2V_HIP_FP8_SPLITK", "3")
    two = run_linear(be, x, w, b, H.ACT_GELU_TANH, x_row=37, y_row=11, rows=300)
    assert_close(two, one, 1e-6, 1e-5, what="split vs one pass, offsets")
    assert_close(two, oracle_w8a8(x[37:337], q, s, K, b, H.ACT_GELU_TANH), *FP8_TIGHT, what="split, offsets")


@pytest.mark.parametrize("cfg,act,ydt", [(6, H.ACT_GELU_TANH, H.DTYPE_BF16), (6, H.ACT_NONE, H.DTYPE_F32),
                                         (6, H.ACT_GELU_TANH, H.DTYPE_MXE4M3), (7, H.ACT_GELU_TANH, H.DTYPE_BF16),
                                         (7, H.ACT_NONE, H.DTYPE_BF16), (7, H.ACT_GELU_TANH, H.DTYPE_MXE4M3),
                                         (8, H.ACT_GELU_TANH, H.DTYPE_BF16), (8, H.ACT_NONE, H.DTYPE_BF16),
                                         (8, H.ACT_GELU_TANH, H.DTYPE_MXE4M3), (8, H.ACT_NONE, H.DTYPE_MXE4M3),
                                         (9, H.ACT_GELU_TANH, H.DTYPE_BF16), (9, H.ACT_NONE, H.DTYPE_BF16),
                                         (9, H.ACT_GELU_TANH, H.DTYPE_MXE4M3), (9, H.ACT_NONE, H.DTYPE_MXE4M3),
                                         (10, H.ACT_GELU_TANH, H.DTYPE_BF16), (10, H.ACT_NONE, H.DTYPE_F32),
                                         (1, H.ACT_GELU_TANH, H.DTYPE_BF16), (1, H.ACT_NONE, H.DTYPE_F32),
                                         (1, H.ACT_GELU_TANH, H.DTYPE_MXE4M3)])
def test_fp8_forced_persistent_vs_config0(be, monkeypatch, cfg, act, ydt):
    """The persistent tiles (and the one-per-CU 128 x 128 and 128 x 256 tiles, 10 and 1) forced
    (LIGHTX2V_HIP_FP8_CFG, read per call) against the one-shot configuration
    0, bit for bit over the whole output:
    1937 rows (ragged: 7 x 256 + 145) x 9216 channels is 576 tiles of 256 x
    128 or 288 of 256 x 256 (configurations 8, 9), so every workgroup of the
    grid walks two or more; GELU or none; bf16, f32 (configuration 6; 7 to
    9 store bf16 or MX only) and MX e4m3 output.  All share the K order of
    every sum, so only a fault in the walk or the epilogue could differ."""
    M, K, N = 1937, 1536, 9216
    x = normal(3201, M * K).reshape(M, K)
    _, q, s = fp8_weight(3202, N, K, K)
    w = be.weight_fp8(q, s, N, K, K)
    xb, bb = be.upload(x), be.upload(normal(3203, N, 0.01))
    mx = ydt == H.DTYPE_MXE4M3
    sfx = ".mxout" if mx else ""

    def run(c):
        monkeypatch.setenv("LIGHTX2V_HIP_FP8_CFG", str(c))
        y = be.alloc_mx(M, N) if mx else be.alloc(M * N, ydt)
        if not mx:  # an element left unwritten stays NaN (a reused allocation cannot mask it)
            be.write(y, np.full(M * N, np.nan, np.float32))
        _, names = _kernels(be, lambda: be.linear(xb, 0, M, w, bb, act, y, 0))
        assert {k for k in names if k.startswith("gemm")} == {f"gemm_fp8_e4m3.c{c}{sfx}"}, names
        return be.download_mx(y, M, N) if mx else (u32(be.download(y)),)

    want, got = run(0), run(cfg)
    assert all(np.array_equal(a, b) for a, b in zip(want, got))
    if not mx:
        p = np.arange(0, M, 97)
        y = got[0].view(np.float32).reshape(M, N)[p]
        tol = FP8_TIGHT if ydt == H.DTYPE_F32 else (4e-3, 1e-2)
        assert_close(y, oracle_w8a8(x[p], q, s, K, normal(3203, N, 0.01), act), *tol, what=f"c{cfg} vs oracle")


@pytest.mark.parametrize("cfg,act,ydt", [(1, H.ACT_GELU_TANH, H.DTYPE_BF16), (1, H.ACT_NONE, H.DTYPE_F32),
                                         (1, H.ACT_GELU_TANH, H.DTYPE_MXE4M3),
                                         (7, H.ACT_GELU_TANH, H.DTYPE_BF16), (7, H.ACT_NONE, H.DTYPE_BF16),
                                         (7, H.ACT_GELU_TANH, H.DTYPE_MXE4M3), (7, H.ACT_NONE, H.DTYPE_MXE4M3),
                                         (6, H.ACT_GELU_TANH, H.DTYPE_BF16), (6, H.ACT_NONE, H.DTYPE_F32),
                                         (6, H.ACT_GELU_TANH, H.DTYPE_MXE4M3), (10, H.ACT_GELU_TANH, H.DTYPE_BF16),
                                         (10, H.ACT_NONE, H.DTYPE_F32)])
def test_fp8_grouped_forced_vs_config0(be, monkeypatch, cfg, act, ydt):
    """Group-128 weights (one scale per 128 columns of K per channel) on the
    grouped configurations forced, against configuration 0, bit for bit over
    the whole output.  Every configuration rescales a block's sums by the
    group's s_{g-1} / s_g right before the group's first MFMA on the block
    and applies the last group's scale in the epilogue, so the sums are the
    same f32 operations (the overlapped-epilogue tile, 7, included: it
    walks two or more tiles per workgroup here).  1937 rows (ragged) x 9216
    channels x K 1536; GELU or none; bf16, f32 or MX e4m3 output; sampled
    rows against the oracle."""
    M, K, N = 1937, 1536, 9216
    x = normal(3211, M * K).reshape(M, K)
    _, q, s = fp8_weight(3212, N, K, 128)
    w = be.weight_fp8(q, s, N, K, 128)
    xb, bb = be.upload(x), be.upload(normal(3213, N, 0.01))
    mx = ydt == H.DTYPE_MXE4M3
    sfx = ".g128.mxout" if mx else ".g128"

    def run(c):
        monkeypatch.setenv("LIGHTX2V_HIP_FP8_CFG", str(c))
        y = be.alloc_mx(M, N) if mx else be.alloc(M * N, ydt)
        if not mx:  # an element left unwritten stays NaN (a reused allocation cannot mask it)
            be.write(y, np.full(M * N, np.nan, np.float32))
        _, names = _kernels(be, lambda: be.linear(xb, 0, M, w, bb, act, y, 0))
        assert {k for k in names if k.startswith("gemm")} == {f"gemm_fp8_e4m3.c{c}{sfx}"}, names
        return be.download_mx(y, M, N) if mx else (u32(be.download(y)),)

    want, got = run(0), run(cfg)
    assert all(np.array_equal(a, b) for a, b in zip(want, got))
    if not mx:
        p = np.arange(0, M, 97)
        y = got[0].view(np.float32).reshape(M, N)[p]
        tol = FP8_TIGHT if ydt == H.DTYPE_F32 else (4e-3, 1e-2)
        assert_close(y, oracle_w8a8(x[p], q, s, 128, normal(3213, N, 0.01), act), *tol, what=f"c{cfg}.g128 vs oracle")


@pytest.mark.parametrize("cfg,ydt", [(1, H.DTYPE_BF16), (1, H.DTYPE_F32), (10, H.DTYPE_BF16), (10, H.DTYPE_F32)])
def test_fp8_grouped_ragged_n_vs_config0(be, monkeypatch, cfg, ydt):
    """Group-128 weights with both edges ragged: 613 rows x 1000 channels
    (1000 = 3 x 256 + 232 = 7 x 128 + 104, so every tile shape ends on a
    partial column tile, whose staged epilogue takes the per-element store
    path) x K 1024 (8 groups), GELU.  The transposed blocks of the one-shot
    tiles (bf16 / f32 output) store the partial tiles' columns in range and
    only those: configurations 1 and 10 against 0, bit for bit over the
    whole output (NaN-filled first), and sampled rows against the oracle."""
    M, K, N = 613, 1024, 1000
    x = normal(3311, M * K).reshape(M, K)
    _, q, s = fp8_weight(3312, N, K, 128)
    w = be.weight_fp8(q, s, N, K, 128)
    b = normal(3313, N, 0.01)
    xb, bb = be.upload(x), be.upload(b)

    def run(c):
        monkeypatch.setenv("LIGHTX2V_HIP_FP8_CFG", str(c))
        y = be.alloc(M * N, ydt)
        be.write(y, np.full(M * N, np.nan, np.float32))
        _, names = _kernels(be, lambda: be.linear(xb, 0, M, w, bb, H.ACT_GELU_TANH, y, 0))
        assert {k for k in names if k.startswith("gemm")} == {f"gemm_fp8_e4m3.c{c}.g128"}, names
        return u32(be.download(y))

    want, got = run(0), run(cfg)
    assert np.array_equal(want, got)
    y = got.view(np.float32).reshape(M, N)
    assert not np.isnan(y).any(), "an output element was left unwritten"
    p = np.arange(0, M, 41)
    tol = FP8_TIGHT if ydt == H.DTYPE_F32 else (4e-3, 1e-2)
    assert_close(y[p], oracle_w8a8(x[p], q, s, 128, b, H.ACT_GELU_TANH), *tol, what=f"c{cfg}.g128 vs oracle")


@pytest.mark.parametrize("group", ["channel", 128])
@pytest.mark.parametrize("act,ydt", [(H.ACT_NONE, H.DTYPE_BF16), (H.ACT_GELU_TANH, H.DTYPE_F32),
                                     (H.ACT_GELU_TANH, H.DTYPE_MXE4M3)])
def test_fp8_mx_input_forced_vs_config0(be, monkeypatch, group, act, ydt):
    """MX e4m3 activations (a power-of-two scale per 32 columns of K, applied
    by the scaled MFMA) on the one-per-CU 128 x 256 tile (configuration 1)
    forced against the 256 x 128 tile (0), bit for bit over the whole
    output, per-channel or group-128 weights, bf16, f32 or MX e4m3 output:
    1937 rows (ragged for both tiles) x 2304 channels x K 1536, an MX input
    read from row 16 of its buffer; sampled rows against the oracle on the
    decoded input."""
    M, K, N, r0 = 1937, 1536, 2304, 16
    g = K if group == "channel" else 128
    x = normal(3221, (M + r0) * K).reshape(M + r0, K)
    _, q, s = fp8_weight(3222, N, K, g)
    b = normal(3223, N, 0.01)
    w = be.weight_fp8(q, s, N, K, g)
    xb, bb = be.upload(x), be.upload(b)
    xm = be.alloc_mx(M + r0, K)
    be.quantize_mx(xb, 0, M + r0, xm)
    mx = ydt == H.DTYPE_MXE4M3
    sfx = (".g128" if group == 128 else "") + ".mxin" + (".mxout" if mx else "")

    def run(c):
        monkeypatch.setenv("LIGHTX2V_HIP_FP8_CFG", str(c))
        y = be.alloc_mx(M, N) if mx else be.alloc(M * N, ydt)
        if not mx:  # an element left unwritten stays NaN (a reused allocation cannot mask it)
            be.write(y, np.full(M * N, np.nan, np.float32))
        _, names = _kernels(be, lambda: be.linear(xm, r0, M, w, bb, act, y, 0))
        assert {k for k in names if k.startswith("gemm")} == {f"gemm_fp8_e4m3.c{c}{sfx}"}, names
        return be.download_mx(y, M, N) if mx else (u32(be.download(y)),)

    want, got = run(0), run(1)
    assert all(np.array_equal(a, b) for a, b in zip(want, got))
    if ydt == H.DTYPE_F32:
        p = np.arange(0, M, 97)
        qx, sx = O.act_quant_mx(x)
        xd = O.dequant_mx(qx, sx)[r0:][p]
        yv = got[0].view(np.float32).reshape(M, N)[p]
        assert_close(yv, O.linear(xd, O.fp8_dequantize(q, s, N, K, g), b, act, nthreads=8), *FP8_TIGHT,
                     what=f"c1 MX input (group {g}) vs oracle")


def test_fp8_no_bias(be):
    M, K, N = 96, 640, 320
    x = normal(8, M * K).reshape(M, K)
    _, q, s = fp8_weight(9, N, K, K)
    w = be.weight_fp8(q, s, N, K, K)
    y = run_linear(be, x, w, None, H.ACT_NONE)
    assert_close(y, oracle_w8a8(x, q, s, K, None, 0), *FP8_TIGHT, what="fp8 no bias")


def test_fp8_reference_quantizer_codes(be):
    """Weights from the reference's own encoder (quant.rs:376-406, exponent-0
    and NaN codes included): exponent-0 codes are stored as zero, so the
    result equals the oracle with those weights zeroed; NaN codes give NaN
    columns in both."""
    M, K, N = 64, 512, 256
    x = normal(10, M * K).reshape(M, K)
    wf = normal(11, N * K, 0.02).reshape(N, K)
    q, s = O.fp8_quantize(wf, N, K, K, False)
    w = be.weight_fp8(q, s, N, K, K)
    n_e0 = int(np.sum(((q & 0x78) == 0) & ((q & 7) != 0)))
    assert w.info()["canonicalized"] == n_e0
    qc = np.where(((q & 0x78) == 0) & ((q & 7) != 0), q & 0x80, q).astype(np.uint8)
    y = run_linear(be, x, w, None, H.ACT_NONE)
    want = oracle_w8a8(x, qc, s, K, None, 0)
    nan_cols = np.any((q & 0x7F) == 0x7F, axis=1)
    assert np.array_equal(np.isnan(y).any(0), nan_cols)
    ok = ~nan_cols
    assert_close(y[:, ok], want[:, ok], *FP8_TIGHT, what="fp8 reference-encoder codes")


def _kernels(be, fn):
    """The profile names of the kernels fn() launches."""
    be.profile_reset()
    be.profile_enable(True)
    try:
        out = fn()
        st = be.profile_stats()
    finally:
        be.profile_enable(False)
        be.profile_reset()
    return out, set(st)


# (M, K, N): the 256x128 and 128x256 grouped tiles, ragged M / N, one-row,
# and the Wan chunk's O shape
G128_SHAPES = [(130, 512, 200), (77, 256, 132), (300, 1536, 1536), (1, 128, 64), (513, 512, 2056),
               (260, 1024, 1540)]


@pytest.mark.parametrize("M,K,N", G128_SHAPES)
def test_fp8_g128_mfma_vs_oracle(be, M, K, N):
    """Group-128 FP8 (the reference default, FP8_GROUP, quant.rs:21, 425-429)
    on the fp8 MFMA: each 128-column stage's partial sum is scaled by its
    group's scale.  Against the oracle on the same e4m3 activations, with a
    heavy-tailed column block so the groups' scales differ by 20x."""
    x = normal(15 + M, M * K).reshape(M, K)
    wf = normal(16 + N, N * K, 0.02).reshape(N, K)
    wf[:, 128:256 if K > 128 else 128] *= np.float32(20.0)
    q, s = O.fp8_quantize(wf, N, K, 128, True)
    b = normal(17, N, 0.01)
    w = be.weight_fp8(q, s, N, K, 128)
    y, ks = _kernels(be, lambda: run_linear(be, x, w, b, H.ACT_GELU_TANH))
    if K > 128:  # (at K = 128 one group per channel: the per-channel tiles)
        assert any(k.startswith("gemm_fp8_e4m3.c") and k.endswith(".g128") for k in ks), ks
    assert "gemm_generic" not in ks
    assert_close(y, oracle_w8a8(x, q, s, 128, b, 1), *FP8_TIGHT, what="fp8 g128 MFMA vs oracle")
    # bf16 output: the f32 output rounded, bit for bit
    y16 = run_linear(be, x, w, b, H.ACT_GELU_TANH, y_dtype=H.DTYPE_BF16)
    assert np.array_equal(u32(y16), u32(O.bf16_round(y)))


def test_fp8_g128_reference_contract(be):
    """The reference's own FP8 weights (its encoder, group 128, exponent-0
    codes included) against the unmodified contract: the oracle's linear
    with weight(&q.dequantize()) (backend.rs:179-188) on the same e4m3
    activations.  Canonicalizing the exponent-0 codes moves each such
    weight by <= 7 * 2^-12 * s, inside the fp8 tolerance."""
    M, K, N = 192, 1536, 512
    x = normal(18, M * K).reshape(M, K)
    wf = normal(19, N * K, 0.02).reshape(N, K)
    q, s = O.fp8_quantize(wf, N, K, 128, False)
    w = be.weight_fp8(q, s, N, K, 128)
    assert w.info()["canonicalized"] > 0
    y = run_linear(be, x, w, None, H.ACT_NONE)
    nan_cols = np.any((q & 0x7F) == 0x7F, axis=1)
    assert np.array_equal(np.isnan(y).any(0), nan_cols)
    want = oracle_w8a8(x, q, s, 128, None, 0)
    ok = ~nan_cols
    assert_close(y[:, ok], want[:, ok], *FP8_TIGHT, what="fp8 g128, reference codes, unmodified contract")


@pytest.mark.parametrize("group", [64, 256])
def test_fp8_other_groups_bf16_mfma(be, group):
    """FP8 groups other than 128 and cols: the bf16 GEMM (weight dequantized
    to bf16 in its loader, bf16 activations) rather than the scalar kernel."""
    M, K, N = 150, 1024, 320
    x = normal(20 + group, M * K).reshape(M, K)
    _, q, s = fp8_weight(21 + group, N, K, group)
    w = be.weight_fp8(q, s, N, K, group)
    y, ks = _kernels(be, lambda: run_linear(be, x, w, None, H.ACT_NONE))
    assert any(k.startswith("gemm_w16_fp8") for k in ks) and "gemm_generic" not in ks, ks
    wd = O.fp8_dequantize(q, s, N, K, group)
    assert_close(y, oracle_w16(x, wd, None, 0), *W16_TIGHT, what=f"fp8 g{group} on the bf16 MFMA")


@pytest.mark.parametrize("case", ["zero_group", "wide_range"])
def test_fp8_g128_ratio_fallback(be, case):
    """Group-128 FP8 weights whose scales the fp8 MFMA kernels' per-group
    rescaling cannot carry (a channel with an all-zero group, scale 0; or
    two groups of a channel more than 2^60 apart) take the bf16 MFMA kernel;
    its result against the oracle on the dequantized weight (W16_TIGHT)."""
    M, K, N = 150, 1024, 320
    x = normal(31, M * K).reshape(M, K)
    _, q, s = fp8_weight(32, N, K, 128)
    q, s = q.copy(), s.copy().reshape(N, K // 128)
    if case == "zero_group":
        q.reshape(N, K)[7, 256:384] = 0
        s[7, 2] = 0.0
    else:
        s[11, 5] *= 2.0 ** 70
    s = s.ravel()
    w = be.weight_fp8(q, s, N, K, 128)
    y, ks = _kernels(be, lambda: run_linear(be, x, w, None, H.ACT_NONE))
    assert any(k.startswith("gemm_w16_fp8") for k in ks) and not any(k.startswith("gemm_fp8_e4m3") for k in ks), ks
    wd = O.fp8_dequantize(q, s, N, K, 128)
    assert_close(y, oracle_w16(x, wd, None, 0), *W16_TIGHT, what=f"fp8 g128 ({case}) on the bf16 MFMA")


def test_fp8_grouped_paths(be):
    """Group-128 FP8 (the reference default, quant.rs:21): e4m3 activations
    and the bf16-activation mode."""
    M, K, N = 130, 512, 200
    x = normal(12, M * K).reshape(M, K)
    _, q, s = fp8_weight(13, N, K, 128)
    b = normal(14, N, 0.01)
    w = be.weight_fp8(q, s, N, K, 128)
    y = run_linear(be, x, w, b, H.ACT_NONE)
    assert_close(y, oracle_w8a8(x, q, s, 128, b, 0), *FP8_TIGHT, what="fp8 g128 e4m3 acts")
    be.set_fp8_act(H.FP8_ACT_BF16)
    try:
        y2 = run_linear(be, x, w, b, H.ACT_NONE)
    finally:
        be.set_fp8_act(H.FP8_ACT_E4M3)
    wd = O.fp8_dequantize(q, s, N, K, 128)
    assert_close(y2, oracle_w16(x, wd, b, 0), *W16_TIGHT, what="fp8 g128 bf16 acts")
    assert_close(y2, O.linear(x, wd, b, 0), 5e-3, 0.05, what="fp8 g128 bf16 acts vs f32 oracle")


# ---- Q8 / Q4: bf16 MFMA with in-loader dequantization ----------------------------------

@pytest.mark.parametrize("M,K,N,group", [(64, 256, 192, 32), (77, 288, 130, 32), (300, 1536, 1000, 128),
                                         (129, 512, 256, 512), (256, 1536, 896, 32), (96, 256, 320, 16),
                                         (130, 384, 200, 48)])
@pytest.mark.parametrize("xdt", [H.DTYPE_F32, H.DTYPE_BF16])
def test_q8_vs_oracle(be, M, K, N, group, xdt):
    x = normal(20 + M, M * K).reshape(M, K)
    _, q, s = q8_weight(21 + N, N, K, group)
    b = normal(22, N, 0.01)
    w = be.weight_q8(q, s, N, K, group)
    y = run_linear(be, x, w, b, H.ACT_GELU_TANH, x_dtype=xdt)
    wd = O.q8_dequantize(q, s, N, K, group)
    assert_close(y, oracle_w16(x, wd, b, 1), *W16_TIGHT, what="q8 vs oracle(bf16 operands)")
    assert_close(y, O.linear(x, wd, b, 1, nthreads=8), 5e-3, 0.05, what="q8 vs f32 oracle")


@pytest.mark.parametrize("M,K,N,group,hqq", [(64, 256, 192, 32, None), (77, 320, 130, 32, None),
                                             (300, 1536, 512, 64, True), (200, 512, 384, 64, False),
                                             (129, 896, 256, 128, None), (70, 384, 136, 16, False),
                                             (260, 384, 264, 48, None)])
@pytest.mark.parametrize("xdt", [H.DTYPE_F32, H.DTYPE_BF16])
def test_q4_vs_oracle(be, M, K, N, group, hqq, xdt):
    x = normal(30 + M, M * K).reshape(M, K)
    if hqq is None:
        _, c, s, z = q4_sym_weight(31 + N, N, K, group)
    else:
        wf = normal(31 + N, N * K, 0.02).reshape(N, K)
        c, s, z = O.q4_quantize(wf, N, K, group, hqq)
    b = normal(32, N, 0.01)
    w = be.weight_q4(O.q4_pack(c), s, z, N, K, group, packed=True)
    y = run_linear(be, x, w, b, H.ACT_NONE, x_dtype=xdt)
    wd = O.q4_dequantize(c, s, z, N, K, group)
    assert_close(y, oracle_w16(x, wd, b, 0), *W16_TIGHT, what="q4 vs oracle(bf16 operands)")
    assert_close(y, O.linear(x, wd, b, 0, nthreads=8), 5e-3, 0.05, what="q4 vs f32 oracle")


@pytest.mark.parametrize("fmt", ["q8_g32", "q8_g128", "q4_sym_g32", "q4_hqq_g64", "fp8_g64"])
def test_w16_configs_bit_equal(be, monkeypatch, fmt):
    """The bf16-MFMA tiles forced (LIGHTX2V_HIP_W16_CFG, read per call):
    256 x 128 and 128 x 256 with 64-element K stages and 256 x 256 with
    32-element ones contract the same 16-element MFMA slices in the same K
    order, so their outputs agree bit for bit over the whole tensor (outputs
    prefilled with NaN); ragged M and N (517 rows, 896 channels: 3.5 tiles of
    256), GELU, bf16 and f32 output; the 256 x 256 tile's sampled rows
    against the oracle on the bf16 operands."""
    M, K, N = 517, 1536, 896
    x = normal(60, M * K).reshape(M, K)
    b = normal(61, N, 0.01)
    kind, g = fmt.split("_g")[0], int(fmt.split("_g")[1])
    if kind == "q8":
        _, q, s = q8_weight(62, N, K, g)
        w, wd = be.weight_q8(q, s, N, K, g), O.q8_dequantize(q, s, N, K, g)
    elif kind == "fp8":
        _, q, s = fp8_weight(62, N, K, g)
        w, wd = be.weight_fp8(q, s, N, K, g), O.fp8_dequantize(q, s, N, K, g)
    else:
        if kind == "q4_sym":
            _, c, s, z = q4_sym_weight(62, N, K, g)
        else:
            c, s, z = O.q4_quantize(normal(62, N * K, 0.02).reshape(N, K), N, K, g, True)
        w, wd = be.weight_q4(O.q4_pack(c), s, z, N, K, g, packed=True), O.q4_dequantize(c, s, z, N, K, g)
    be.set_act_dtype(H.DTYPE_BF16)
    try:
        xb = be.upload(x)
    finally:
        be.set_act_dtype(H.DTYPE_F32)
    bb = be.upload(b)
    if kind == "fp8":
        be.set_fp8_act(H.FP8_ACT_BF16)  # FP8 group 64: the bf16 MFMA path
    try:
        for ydt in (H.DTYPE_BF16, H.DTYPE_F32):
            outs = []
            for c_ in (0, 1, 2):
                monkeypatch.setenv("LIGHTX2V_HIP_W16_CFG", str(c_))
                y = be.alloc(M * N, ydt)
                be.write(y, np.full(M * N, np.nan, np.float32))
                _, ks = _kernels(be, lambda: be.linear(xb, 0, M, w, bb, H.ACT_GELU_TANH, y, 0))
                assert any(k.startswith("gemm_w16_") and k.endswith(f".c{c_}") for k in ks), ks
                outs.append(be.download(y).reshape(M, N))
            assert not np.isnan(outs[2]).any()
            for c_ in (1, 2):
                assert np.array_equal(u32(outs[c_]), u32(outs[0])), f"{fmt} config {c_} vs 0, dtype {ydt}"
        p = np.arange(0, M, 23)
        assert_close(outs[2][p], oracle_w16(O.bf16_round(x[p]), wd, b, 1), *W16_TIGHT, what=f"{fmt} 256x256 vs oracle")
    finally:
        be.set_fp8_act(H.FP8_ACT_E4M3)


@pytest.mark.parametrize("M,K,N", [(300, 1536, 512), (1000, 8960, 1536)])
def test_q4_zero8_path_equals_affine_path(be, M, K, N):
    """Symmetric Q4 (every zero 8) dequantizes as fma(c, s, -8 s) without
    loading zeros; the same dequantized weights through the affine path
    (one group re-expressed as codes c - 1 with zero 7, which decode to the
    same values) give the same output, bit for bit."""
    x = normal(40 + M, M * K).reshape(M, K)
    _, c, s, z = q4_sym_weight(41 + N, N, K, 32)
    assert (z == 8.0).all()
    g = int(np.flatnonzero((c.reshape(-1, 32) >= 1).all(axis=1))[0])  # a group with no code 0
    c2, z2 = c.reshape(-1, 32).copy(), z.reshape(-1).copy()
    c2[g] -= 1
    z2[g] = 7.0
    c2 = c2.reshape(c.shape)
    assert np.array_equal(O.q4_dequantize(c2, s, z2.reshape(z.shape), N, K, 32), O.q4_dequantize(c, s, z, N, K, 32))
    b = normal(42, N, 0.01)
    w_sym = be.weight_q4(O.q4_pack(c), s, z, N, K, 32, packed=True)
    w_aff = be.weight_q4(O.q4_pack(c2), s, z2.reshape(z.shape), N, K, 32, packed=True)
    y1 = run_linear(be, x, w_sym, b, H.ACT_NONE, x_dtype=H.DTYPE_BF16)
    y2 = run_linear(be, x, w_aff, b, H.ACT_NONE, x_dtype=H.DTYPE_BF16)
    assert np.array_equal(u32(y1), u32(y2))


# ---- shapes the MFMA kernels do not tile: the generic kernel ----------------------------

@pytest.mark.parametrize("fmt", ["f32", "q8", "q4", "fp8"])
def test_odd_shapes_generic(be, fmt):
    M, K, N = 9, 100, 7
    x = normal(40, M * K).reshape(M, K)
    b = normal(41, N, 0.01)
    if fmt == "f32":
        wf = normal(42, N * K, 0.1).reshape(N, K)
        w = be.weight(wf, N, K)
        y = run_linear(be, x, w, b, H.ACT_GELU_TANH)
        assert_close(y, O.linear(x, wf, b, 1), 1e-6, 1e-5, what="f32 weight generic")
    elif fmt == "q8":
        _, q, s = q8_weight(42, N, K, 20)
        w = be.weight_q8(q, s, N, K, 20)
        y = run_linear(be, x, w, b, H.ACT_NONE)
        assert_close(y, O.linear(x, O.q8_dequantize(q, s, N, K, 20), b, 0), 1e-6, 1e-5, what="q8 generic")
    elif fmt == "q4":
        wf = normal(42, N * K, 0.02).reshape(N, K)
        c, s, z = O.q4_quantize(wf, N, K, 50, True)
        w = be.weight_q4(c, s, z, N, K, 50)
        y = run_linear(be, x, w, b, H.ACT_NONE)
        assert_close(y, O.linear(x, O.q4_dequantize(c, s, z, N, K, 50), b, 0), 1e-6, 1e-5, what="q4 generic")
    else:
        _, q, s = fp8_weight(42, N, K, K)
        w = be.weight_fp8(q, s, N, K, K)
        y = run_linear(be, x, w, b, H.ACT_NONE)
        assert_close(y, oracle_w8a8(x, q, s, K, b, 0), 1e-5, 1e-4, what="fp8 generic")


# ---- boundary errors ----------------------------------------------------------------------

def test_alias_and_shape_errors(be):
    K, N = 64, 64
    _, q, s = fp8_weight(50, N, K, K)
    w = be.weight_fp8(q, s, N, K, K)
    x = be.upload(normal(51, 4 * K))
    with pytest.raises(H.HipError) as e:
        be.linear(x, 0, 2, w, None, H.ACT_NONE, x, 1)  # y rows [1,3) overlap x rows [0,2)
    assert e.value.status == H.ERR_ALIAS
    be.linear(x, 0, 2, w, None, H.ACT_NONE, x, 2)  # disjoint rows of one buffer: allowed
    with pytest.raises(H.HipError) as e:
        be.linear(x, 0, 4, w, None, H.ACT_NONE, x, 0)
    assert e.value.status == H.ERR_ALIAS
    y = be.alloc(4 * N)
    with pytest.raises(H.HipError) as e:
        be.linear(x, 1, 4, w, None, H.ACT_NONE, y, 0)
    assert e.value.status == H.ERR_BAD_SHAPE
    be.linear(x, 0, 0, w, None, H.ACT_NONE, y, 0)  # zero rows: no-op


def test_profile_report_names_kernels(be):
    M, K, N = 64, 256, 128
    _, q, s = fp8_weight(60, N, K, K)
    w = be.weight_fp8(q, s, N, K, K)
    be.profile_reset()
    be.profile_enable(True)
    try:
        run_linear(be, normal(61, M * K).reshape(M, K), w, None, H.ACT_NONE)
        rep = be.profile_report()
        st = be.profile_stats()
    finally:
        be.profile_enable(False)
    assert rep and "act_quant_e4m3" in rep
    gemm = [k for k in st if k.startswith("gemm_fp8_e4m3.")]  # named by configuration
    assert len(gemm) == 1 and st[gemm[0]][0] == 1 and st[gemm[0]][1] > 0


def test_cpp_check_harness(be):
    """The C++ consumer of the boundary (`lightx2v check --backend hip`):
    exact quantized-linear checks and bit-exact dequant through the C ABI."""
    import subprocess

    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lightx2v-rs_amd", "bin",
                       "lx2v_hip_check")
    if not os.path.exists(exe):
        pytest.fail("lightx2v-rs_amd/bin/lx2v_hip_check is not built")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "5 checks, 5 passed, 0 failed" in r.stdout

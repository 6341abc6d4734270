"""Input builders and comparison metrics shared by the GPU parity tests.

Tolerance pairs are (rel-L2 over the output, max-abs as a fraction of
max|want|).  Both "tight" pairs compare against the oracle applied to the
very operands the device contracts, so only the accumulation differs:

  * W16_TIGHT, the bf16 MFMA path (v_mfma_f32_32x32x16_bf16) against the
    oracle on bf16-rounded activations and bf16-rounded dequantized weights:
    measured <= 1.2e-6 rel-L2 (the f32 sequential oracle itself is within
    1e-6 of an f64 sum of the same operands);
  * FP8_TIGHT, the fp8 MFMA path (v_mfma_f32_32x32x64_f8f6f4) against the
    oracle on the same per-token e4m3 activations and e4m3 weight codes:
    measured 1.4-1.5e-5 rel-L2 against an f64 sum of those operands for K
    from 512 to 8960 (flat in K, so it comes from inside each 64-product
    MFMA dot rather than from the accumulator chain), max-abs <= 1.7e-4 *
    max|y|.  The bound leaves ~3x headroom on both.
"""

W16_TIGHT = (1e-5, 1e-4)
FP8_TIGHT = (5e-5, 5e-4)

import numpy as np

import oracle as O


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bits_equal(got, want, what=""):
    """Bit equality of two f32 arrays; on failure, how many elements differ
    and where (row, column of a 2-D array), with their values."""
    g, w = u32(got), u32(want)
    assert g.shape == w.shape, (what, g.shape, w.shape)
    bad = np.argwhere(g != w)
    if len(bad):
        at = [tuple(int(v) for v in b) for b in bad[:8]]
        gv = np.asarray(got, np.float32)[tuple(bad[:8].T)]
        wv = np.asarray(want, np.float32)[tuple(bad[:8].T)]
        raise AssertionError(f"{what}: {len(bad)} of {g.size} differ; first at {at}: got {gv} want {wv}")


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))


def max_abs(got, want):
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))))


def assert_close(got, want, rel_tol, abs_frac, what=""):
    """rel-L2 <= rel_tol and max-abs <= abs_frac * max|want|."""
    r = rel_l2(got, want)
    m = max_abs(got, want)
    scale = float(np.max(np.abs(want))) or 1.0
    assert r <= rel_tol and m <= abs_frac * scale, (
        f"{what}: rel_l2={r:.3e} (tol {rel_tol:.1e}) max_abs={m:.3e} (tol {abs_frac * scale:.3e})")
    return r, m


def normal(seed, n, std=1.0):
    return O.Rng(seed).normal(n) * np.float32(std)


def fp8_weight(seed, n, k, group, std=0.02):
    w = normal(seed, n * k, std).reshape(n, k)
    q, s = O.fp8_quantize(w, n, k, group, True)
    return w, q, s


def q8_weight(seed, n, k, group, std=0.02):
    w = normal(seed, n * k, std).reshape(n, k)
    q, s = O.q8_quantize(w, n, k, group)
    return w, q, s


def q4_sym_weight(seed, n, k, group, std=0.02, heavy=False):
    w = normal(seed, n * k, std).reshape(n, k)
    if heavy:  # 1% of K-columns scaled by 20x (columns k % 100 == 37)
        w[:, np.arange(k) % 100 == 37] *= np.float32(20.0)
    c, s, z = O.q4_quantize_sym(w, n, k, group)
    return w, c, s, z


def oracle_w8a8(x, q_w, s_w, group, bias, act):
    """The oracle applied to the same per-token e4m3 activations the device
    computes: X' = e4m3(q_x) * s_x, W' = Fp8E4M3::dequantize."""
    n, k = q_w.shape
    qx, sx = O.act_quant_e4m3(x)
    xd = (O.e4m3_decode_ocp(qx.ravel()).reshape(qx.shape) * sx[:, None]).astype(np.float32)
    wd = O.fp8_dequantize(q_w, s_w, n, k, group)
    return O.linear(xd, wd, bias, act, nthreads=8)


def oracle_w16(x, wd, bias, act):
    """The oracle on the bf16-rounded activations and bf16-rounded
    dequantized weight the bf16 MFMA contracts."""
    return O.linear(O.bf16_round(x), O.bf16_round(wd), bias, act, nthreads=8)

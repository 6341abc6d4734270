"""attention / causal_attention (backend.rs:273-305) on the device against the
oracle's restatement of the reference (crates/lightx2v-cpu/src/lib.rs:155-203).

Tolerances: head_dim 64 / 128 run on the bf16 MFMA (q, k, v and the softmax
weights P rounded to bf16, f32 accumulation and softmax): against the oracle
on the same bf16-rounded q, k, v, rel-L2 <= 5e-3 and max-abs <= 1e-2 *
max|y| (measured 1.3e-3 .. 1.7e-3 and <= 2.1e-3 * max|y|; P's bf16 rounding
is the remaining term), and against the reference's f32 attention on the
unrounded inputs F32REF_TOL below.  Other head sizes run the per-query f32 kernel:
rel-L2 <= 1e-5 (only the summation order and exp2 differ).  Masks: fully
masked tiles are skipped, mixed tiles read mask bytes; a query with no
allowed key is NaN in both, sk = 0 gives zeros in both.
"""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from helpers import assert_close, u32

pytestmark = pytest.mark.gpu
MFMA_TOL = (5e-3, 1e-2)
ROWS_TOL = (1e-5, 1e-4)


def _qkv(seed, heads, sq, sk, d):
    rng = O.Rng(seed)
    q = rng.normal(heads * sq * d).reshape(heads, sq, d).astype(np.float32)
    k = rng.normal(heads * sk * d).reshape(heads, sk, d).astype(np.float32)
    v = rng.normal(heads * sk * d).reshape(heads, sk, d).astype(np.float32)
    return q, k, v


def _up(be, a, dtype):
    b = be.alloc(a.size, dtype)
    be.write(b, a)
    return b


def _run(be, q, k, v, mask=None, dtype=H.DTYPE_F32, odtype=H.DTYPE_F32, resident=False):
    heads, sq, d = q.shape
    sk = k.shape[1]
    qb, kb, vb = _up(be, q, dtype), _up(be, k, dtype), _up(be, v, dtype)
    out = be.alloc(sq * heads * d, odtype)
    if mask is None:
        be.attention(qb, kb, vb, heads, sq, sk, d, out)
    elif resident:
        m = be.mask_upload(mask, sq, sk)
        be.causal_attention(qb, kb, vb, heads, sq, sk, d, m, out)
        m.free()
    else:
        be.causal_attention(qb, kb, vb, heads, sq, sk, d, mask, out)
    return be.download(out).reshape(sq, heads * d)


def _want(q, k, v, mask=None, bf16=True):
    if bf16:
        q, k, v = O.bf16_round(q), O.bf16_round(k), O.bf16_round(v)
    return O.attention(q, k, v, mask)


def _frame_causal(sq, sk, frame):
    """MemRoPE-style block mask: query frame i sees key frames <= i (keys and
    queries indexed in frames of `frame` tokens, the chunk's queries last)."""
    qf = (np.arange(sq) + (sk - sq)) // frame
    kf = np.arange(sk) // frame
    return kf[None, :] <= qf[:, None]


@pytest.mark.parametrize("heads,sq,sk,d", [(2, 128, 64, 128), (3, 77, 130, 128), (1, 300, 1000, 64),
                                           (4, 256, 512, 128), (2, 1, 1, 128), (1, 129, 65, 64)])
@pytest.mark.parametrize("dtype", [H.DTYPE_F32, H.DTYPE_BF16])
def test_attention_mfma(be, heads, sq, sk, d, dtype):
    q, k, v = _qkv(1000 + sq + sk, heads, sq, sk, d)
    got = _run(be, q, k, v, dtype=dtype)
    assert_close(got, _want(q, k, v), *MFMA_TOL, what=f"attention {heads}x{sq}x{sk}x{d}")


# The MFMA path against the reference's own f32 attention on the unrounded
# f32 inputs (cpu/src/lib.rs:171-203): the deviation the bf16 operands and
# bf16 P add.  Measured on gfx950 (printed by this test): rel-L2 2.95e-3 ..
# 3.46e-3 and max-abs <= 4.9e-3 * max|y| at these shapes, about twice the
# deviation from the oracle on bf16-rounded q / k / v (rel-L2 1.3e-3 ..
# 1.7e-3, max-abs <= 2.1e-3 * max|y|): P's rounding and the inputs'
# contribute alike.
F32REF_TOL = (5e-3, 1e-2)


@pytest.mark.parametrize("heads,sq,sk,d", [(2, 128, 64, 128), (1, 300, 1000, 64), (4, 256, 512, 128),
                                           (2, 512, 2048, 128)])
def test_attention_mfma_vs_f32_reference(be, heads, sq, sk, d):
    q, k, v = _qkv(7000 + sq + sk, heads, sq, sk, d)
    got = _run(be, q, k, v, dtype=H.DTYPE_F32)
    r32, m32 = assert_close(got, _want(q, k, v, bf16=False), *F32REF_TOL, what=f"vs f32 reference {sq}x{sk}x{d}")
    r16, m16 = assert_close(got, _want(q, k, v), *MFMA_TOL, what=f"vs bf16-operand oracle {sq}x{sk}x{d}")
    scale = float(np.max(np.abs(got)))
    print(f"attention {heads}x{sq}x{sk}x{d}: vs f32 reference rel-L2 {r32:.3e} max-abs {m32 / scale:.3e}*max; "
          f"vs bf16-operand oracle rel-L2 {r16:.3e} max-abs {m16 / scale:.3e}*max")


@pytest.mark.parametrize("heads,sq,sk,d", [(2, 40, 33, 80), (1, 5, 7, 16), (3, 17, 100, 256)])
def test_attention_other_head_dims(be, heads, sq, sk, d):
    q, k, v = _qkv(2000 + d, heads, sq, sk, d)
    got = _run(be, q, k, v)
    assert_close(got, _want(q, k, v, bf16=False), *ROWS_TOL, what=f"attention d={d}")


@pytest.mark.parametrize("d", [64, 128, 48])
@pytest.mark.parametrize("kind", ["frames", "random", "keep_first"])
def test_causal_attention(be, d, kind):
    heads, sq, sk = 2, 200, 600
    q, k, v = _qkv(3000 + d, heads, sq, sk, d)
    if kind == "frames":
        mask = _frame_causal(sq, sk, 100)
    elif kind == "random":
        mask = np.random.default_rng(5).random((sq, sk)) < 0.3
        mask[:, 0] = True
    else:  # one allowed key per query past the first
        mask = np.zeros((sq, sk), bool)
        mask[:, 0] = True
        mask[np.arange(sq), (np.arange(sq) * 7) % sk] = True
    got = _run(be, q, k, v, mask)
    tol = MFMA_TOL if d in (64, 128) else ROWS_TOL
    assert_close(got, _want(q, k, v, mask, bf16=d in (64, 128)), *tol, what=f"causal {kind} d={d}")
    # the resident mask gives the same result, bit for bit
    assert np.array_equal(u32(_run(be, q, k, v, mask, resident=True)), u32(got))


def test_fully_masked_rows_and_no_keys(be):
    heads, sq, sk, d = 1, 130, 70, 128
    q, k, v = _qkv(4000, heads, sq, sk, d)
    mask = np.ones((sq, sk), bool)
    mask[5] = False
    mask[129] = False
    got = _run(be, q, k, v, mask)
    want = _want(q, k, v, mask)
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.isnan(got[5]).all() and np.isnan(got[129]).all()
    ok = ~np.isnan(want).any(axis=1)
    assert_close(got[ok], want[ok], *MFMA_TOL, what="partly masked")
    # sk = 0: the reference's empty sums are 0
    qb = _up(be, q, H.DTYPE_F32)
    kb, vb = be.alloc(1, H.DTYPE_F32), be.alloc(1, H.DTYPE_F32)
    out = be.alloc(sq * d, H.DTYPE_F32)
    be.write(out, np.full(sq * d, 7.0, np.float32))
    be.attention(qb, kb, vb, heads, sq, 0, d, out)
    assert np.array_equal(be.download(out), np.zeros(sq * d, np.float32))


def test_attention_bf16_out(be):
    heads, sq, sk, d = 2, 96, 160, 128
    q, k, v = _qkv(5000, heads, sq, sk, d)
    y32 = _run(be, q, k, v, dtype=H.DTYPE_BF16)
    y16 = _run(be, q, k, v, dtype=H.DTYPE_BF16, odtype=H.DTYPE_BF16)
    assert np.array_equal(u32(y16), u32(O.bf16_round(y32)))


def test_attention_wan_shape_sampled(be):
    """12 heads x 128 (Wan2.1-1.3B), a 3-frame chunk of 1560-token frames
    after one cached frame, frame-causal mask; 96 sampled query rows."""
    heads, d, frame = 12, 128, 1560
    sq, sk = 3 * frame, 4 * frame
    q, k, v = _qkv(6000, heads, sq, sk, d)
    mask = _frame_causal(sq, sk, frame)
    got = _run(be, q, k, v, mask, dtype=H.DTYPE_BF16)
    rows = np.linspace(0, sq - 1, 96).astype(int)
    want = O.attention(O.bf16_round(q[:, rows]), O.bf16_round(k), O.bf16_round(v), mask[rows])
    assert_close(got[rows], want, *MFMA_TOL, what="wan shape")


@pytest.mark.parametrize("heads,sq,sk,d,frame", [(2, 300, 257, 128, 0), (3, 200, 320, 64, 0), (2, 520, 780, 128, 260),
                                                (12, 1560, 3120, 128, 1560)])
def test_attention_mx_out_is_quantized_f32_out(be, heads, sq, sk, d, frame):
    """out (MXE4M3) == quantize_mx(out (F32)) of the same attention: the
    epilogue quantizes the values the F32 output holds, so codes and scales
    agree bit for bit; a fully masked row (NaN, as the reference) keeps NaN
    codes."""
    q, k, v = _qkv(8000 + sq, heads, sq, sk, d)
    mask = _frame_causal(sq, sk, frame) if frame else None
    if mask is not None:
        mask[7] = False  # no allowed key: NaN
    qb, kb, vb = _up(be, q, H.DTYPE_BF16), _up(be, k, H.DTYPE_BF16), _up(be, v, H.DTYPE_BF16)
    m = be.mask_upload(mask, sq, sk) if mask is not None else None

    def attend(out):
        if m is None:
            be.attention(qb, kb, vb, heads, sq, sk, d, out)
        else:
            be.causal_attention(qb, kb, vb, heads, sq, sk, d, m, out)

    of = be.alloc(sq * heads * d, H.DTYPE_F32)
    attend(of)
    om = be.alloc_mx(sq + 3, heads * d)
    attend(om)
    ref = be.alloc_mx(sq, heads * d)
    be.quantize_mx(of, 0, sq, ref)
    q1, s1 = be.download_mx(om, sq + 3, heads * d)
    q2, s2 = be.download_mx(ref, sq, heads * d)
    ok = np.ones(sq, bool)
    if m is not None:
        m.free()
        assert np.isnan(be.download(of).reshape(sq, heads * d)[7]).all()
        # NaN stays NaN (quantize_mx clamps it to -448): e4m3 NaN is s.1111.111
        assert ((q1[7] & 0x7F) == 0x7F).all()
        ok[7] = False
    assert np.array_equal(q1[:sq][ok], q2[ok]) and np.array_equal(s1[:, :sq][:, ok], s2[:, ok])


@pytest.mark.parametrize("heads,sq,sk,d,frame,pieces", [(2, 520, 780, 128, 260, 2), (3, 300, 900, 64, 300, 3),
                                                       (4, 700, 1400, 128, 0, 4), (12, 1560, 3120, 128, 1560, 2),
                                                       (2, 256, 4096, 128, 1024, 8), (1, 100, 70, 64, 0, 16)])
def test_attention_split_equals_one_pass(be, monkeypatch, heads, sq, sk, d, frame, pieces):
    """The split mode (S pieces per (head, query tile) over parts of its
    allowed key tiles, merged in a second pass) beside the one-pass kernel,
    both against the oracle on sampled rows: each piece rounds P to bf16
    relative to its own running max, so the two differ at the level of that
    rounding (measured rel-L2 ~1.5e-3 between them), and the split is held to
    MFMA_TOL and to no more than 1.25x the one-pass error.  NaN rows (no
    allowed key) in the same places; MX output equal to quantize_mx of its
    own F32 output.  S = 16 over 2 key tiles leaves most pieces empty."""
    q, k, v = _qkv(8200 + sq, heads, sq, sk, d)
    mask = _frame_causal(sq, sk, frame) if frame else None
    if mask is not None:
        mask[3] = False
        mask[sq - 1, : sk // 2] = False  # the last query: keys of the second half only
    qb, kb, vb = _up(be, q, H.DTYPE_BF16), _up(be, k, H.DTYPE_BF16), _up(be, v, H.DTYPE_BF16)
    m = be.mask_upload(mask, sq, sk) if mask is not None else None

    def attend(out, split):
        monkeypatch.setenv("LIGHTX2V_HIP_ATTN_SPLIT", split)
        if m is None:
            be.attention(qb, kb, vb, heads, sq, sk, d, out)
        else:
            be.causal_attention(qb, kb, vb, heads, sq, sk, d, m, out)
        be.sync()

    one, two = be.alloc(sq * heads * d, H.DTYPE_F32), be.alloc(sq * heads * d, H.DTYPE_F32)
    attend(one, "0")
    attend(two, str(pieces))
    a, b = be.download(one).reshape(sq, heads * d), be.download(two).reshape(sq, heads * d)
    nan = np.isnan(a).any(axis=1)
    assert np.array_equal(nan, np.isnan(b).any(axis=1)) and (nan[3] if mask is not None else not nan.any())
    rows = np.unique(np.r_[np.linspace(0, sq - 1, 48).astype(int), sq - 1])
    rows = rows[~nan[rows]]
    want = O.attention(O.bf16_round(q[:, rows]), O.bf16_round(k), O.bf16_round(v),
                       mask[rows] if mask is not None else None)
    r1, _ = assert_close(a[rows], want, *MFMA_TOL, what="one pass")
    r2, _ = assert_close(b[rows], want, *MFMA_TOL, what="split")
    assert r2 <= 1.25 * r1 + 1e-4, (r2, r1)
    om = be.alloc_mx(sq, heads * d)
    attend(om, str(pieces))
    ref = be.alloc_mx(sq, heads * d)
    be.quantize_mx(two, 0, sq, ref)
    q1, s1 = be.download_mx(om, sq, heads * d)
    q2, s2 = be.download_mx(ref, sq, heads * d)
    assert np.array_equal(q1[~nan], q2[~nan]) and np.array_equal(s1[:, ~nan], s2[:, ~nan])
    if m is not None:
        m.free()


def test_attention_mx_out_feeds_o_linear(be):
    """attention -> MXE4M3 -> FP8 linear against attention -> BF16 -> FP8
    linear (per-token e4m3 inside the linear), both against the f32 chain
    of the oracle: the MX hand-off is no less accurate."""
    heads, sq, sk, d, n = 4, 300, 400, 128, 256
    q, k, v = _qkv(8100, heads, sq, sk, d)
    qb, kb, vb = _up(be, q, H.DTYPE_BF16), _up(be, k, H.DTYPE_BF16), _up(be, v, H.DTYPE_BF16)
    wq, ws = O.fp8_quantize((O.Rng(8101).normal(n * heads * d) * np.float32(0.02)).reshape(n, heads * d), n,
                            heads * d, heads * d, True)
    w = be.weight_fp8(wq, ws, n, heads * d, heads * d)
    a16 = be.alloc(sq * heads * d, H.DTYPE_BF16)
    be.attention(qb, kb, vb, heads, sq, sk, d, a16)
    amx = be.alloc_mx(sq, heads * d)
    be.attention(qb, kb, vb, heads, sq, sk, d, amx)
    y16, ymx = be.alloc(sq * n), be.alloc(sq * n)
    be.linear(a16, 0, sq, w, None, H.ACT_NONE, y16, 0)
    be.linear(amx, 0, sq, w, None, H.ACT_NONE, ymx, 0)
    a = _want(q, k, v).reshape(sq, heads * d)
    want = a @ O.fp8_dequantize(wq, ws, n, heads * d, heads * d).reshape(n, heads * d).T
    err16 = np.linalg.norm(be.download(y16).reshape(sq, n) - want) / np.linalg.norm(want)
    errmx = np.linalg.norm(be.download(ymx).reshape(sq, n) - want) / np.linalg.norm(want)
    assert errmx <= max(1.1 * err16, 1e-2), (errmx, err16)


def test_attention_errors(be):
    heads, sq, sk, d = 1, 8, 8, 64
    q, k, v = _qkv(7000, heads, sq, sk, d)
    qb, kb, vb = _up(be, q, H.DTYPE_F32), _up(be, k, H.DTYPE_F32), _up(be, v, H.DTYPE_BF16)
    out = be.alloc(sq * d, H.DTYPE_F32)
    with pytest.raises(H.HipError):  # v in another dtype
        be.attention(qb, kb, vb, heads, sq, sk, d, out)
    vb = _up(be, v, H.DTYPE_F32)
    with pytest.raises(H.HipError):  # k too short for sk
        be.attention(qb, kb, vb, heads, sq, sk + 1, d, out)
    with pytest.raises(H.HipError):  # out aliases q
        be.attention(qb, kb, vb, heads, sq, sk, d, qb)
    with pytest.raises(H.HipError):  # head_dim past 256
        be.attention(qb, kb, vb, 1, 1, 1, 300, out)
    with pytest.raises(H.HipError):  # MX output of another width
        be.attention(qb, kb, vb, heads, sq, sk, d, be.alloc_mx(sq, 2 * d))
    with pytest.raises(H.HipError):  # MX output with a head_dim off the MFMA path
        be.attention(qb, kb, vb, 2, sq, sk // 2, 32, be.alloc_mx(sq, 64))
    with pytest.raises(H.HipError):  # per-token E4M3 output
        be.attention(qb, kb, vb, heads, sq, sk, d, be.alloc_e4m3(sq, d))
    m = be.mask_upload(np.ones((sq, sk), bool), sq, sk)
    with pytest.raises(H.HipError):  # resident mask of another shape
        be.causal_attention(qb, kb, vb, heads, sq - 1, sk, d, m, out)

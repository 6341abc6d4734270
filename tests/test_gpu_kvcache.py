"""The KV cache / MemRoPE ops (backend.rs:333-392) on the device against the
oracle's restatement of the reference CPU backend (oracle/kvcache.py,
crates/lightx2v-cpu/src/lib.rs:607-806).

Bar: bit-exact.  Row bookkeeping (length, temporal indices, slot kinds) is
compared after every call; K / V after every update.  F32 caches match the
oracle exactly (copies, and the EMA as two products and a sum in f32).  BF16
caches hold bf16 inputs exactly; an update folds in f32 and rounds each
changed row to bf16 once, so the oracle's rows are rounded after every
update to compare.
"""

import numpy as np
import pytest

import lightx2v_hip as H
import oracle as O
from oracle import kvcache as KC
from helpers import u32

pytestmark = pytest.mark.gpu
CFG = H.MemRopeConfig()
OCFG = KC.MemRopeConfig()


def _up(be, a, dtype):
    b = be.alloc(a.size, dtype)
    be.write(b, a.ravel())
    return b


def _new(be, heads, hd, cap, dtype):
    old = be.act_dtype
    be.set_act_dtype(dtype)
    try:
        return be.kv_cache_new(heads, hd, cap)
    finally:
        be.set_act_dtype(old)


def _round(a, dtype):
    return O.bf16_round(a) if dtype == H.DTYPE_BF16 else a


def _check_rows(c, oc):
    assert len(c) == oc.rows()
    assert c.temporal() == oc.temporal
    assert c.kinds() == oc.kinds


def _check_kv(be, c, oc, dtype):
    kb, vb = c.kv()
    k, v = oc.kv()
    n = k.size
    got_k, got_v = be.download(kb)[:n], be.download(vb)[:n]
    assert np.array_equal(u32(got_k), u32(_round(k, dtype).ravel()))
    assert np.array_equal(u32(got_v), u32(_round(v, dtype).ravel()))
    kb.free()
    vb.free()


def _bf16_oracle_rows(oc, dtype):
    if dtype == H.DTYPE_BF16:
        oc.k, oc.v = O.bf16_round(oc.k), O.bf16_round(oc.v)


@pytest.mark.parametrize("dtype", [H.DTYPE_F32, H.DTYPE_BF16])
@pytest.mark.parametrize("heads,hd,ft", [(3, 128, 7), (2, 64, 5), (2, 6, 3)])
def test_dit_pattern(be, dtype, heads, hd, ft):
    """dit.rs:640-642: a 3-frame chunk, put + update on each of 4 DMD steps;
    7 chunks take the cache through seeding, graduation and eviction."""
    rows = 3 * ft
    c = _new(be, heads, hd, OCFG.cache_frames * ft, dtype)
    oc = KC.KvCache(heads, hd, OCFG.cache_frames * ft)
    rng = np.random.default_rng(100 + hd)
    for chunk in range(7):
        temporal = [chunk * 3 + i // ft for i in range(rows)]
        for step in range(4):
            k = _round(rng.standard_normal((heads, rows, hd)).astype(np.float32), dtype)
            v = _round(rng.standard_normal((heads, rows, hd)).astype(np.float32), dtype)
            kb, vb = _up(be, k, dtype), _up(be, v, dtype)
            c.put(kb, vb, rows, temporal)
            oc.put(k, v, rows, temporal)
            _check_rows(c, oc)
            c.memrope_update(CFG, ft)
            oc.memrope_update(OCFG, ft)
            _bf16_oracle_rows(oc, dtype)
            _check_rows(c, oc)
            _check_kv(be, c, oc, dtype)
    c.free()


def test_conformance_40_frames(be):
    """conformance.rs:141-178 on the device: append + update of 40 two-token
    frames; bounded, sinks pinned, newest present, 11 distinct indices."""
    heads, hd, ft = 2, 4, 2
    c = _new(be, heads, hd, OCFG.cache_frames * ft, H.DTYPE_F32)
    oc = KC.KvCache(heads, hd, OCFG.cache_frames * ft)
    rng = np.random.default_rng(21)
    for frame in range(40):
        k = rng.standard_normal((heads, ft, hd)).astype(np.float32)
        v = rng.standard_normal((heads, ft, hd)).astype(np.float32)
        c.append(_up(be, k, H.DTYPE_F32), _up(be, v, H.DTYPE_F32), ft, [frame] * ft)
        oc.append(k, v, ft, [frame] * ft)
        c.memrope_update(CFG, ft)
        oc.memrope_update(OCFG, ft)
        assert len(c) <= OCFG.cache_frames * ft
    t = c.temporal()
    assert t[:6] == [0, 0, 1, 1, 2, 2] and t[-1] == 39 and len(t) // ft == 12 and len(set(t)) == 11
    _check_rows(c, oc)
    _check_kv(be, c, oc, H.DTYPE_F32)


def test_grows_past_capacity_and_reads_other_dtype(be):
    heads, hd = 2, 32
    c = _new(be, heads, hd, 3, H.DTYPE_BF16)
    oc = KC.KvCache(heads, hd, 3)
    rng = np.random.default_rng(3)
    for i in range(6):
        rows = 5 + i
        k = O.bf16_round(rng.standard_normal((heads, rows, hd)).astype(np.float32))
        v = O.bf16_round(rng.standard_normal((heads, rows, hd)).astype(np.float32))
        # F32 inputs into a BF16 cache: converted (exactly, they are bf16 values)
        c.append(_up(be, k, H.DTYPE_F32), _up(be, v, H.DTYPE_F32), rows, list(range(100 * i, 100 * i + rows)))
        oc.append(k, v, rows, list(range(100 * i, 100 * i + rows)))
    _check_rows(c, oc)
    _check_kv(be, c, oc, H.DTYPE_BF16)
    n = heads * len(c) * hd
    kf, vf = be.alloc(n, H.DTYPE_F32), be.alloc(n, H.DTYPE_F32)
    c.read(kf, vf)
    k, v = oc.kv()
    assert np.array_equal(be.download(kf), k.ravel()) and np.array_equal(be.download(vf), v.ravel())


@pytest.mark.parametrize("split", [None, "4"])
@pytest.mark.parametrize("hd", [128, 64, 48])
def test_attention_reads_the_cache_in_place(be, monkeypatch, hd, split):
    """kv_cache_attention == causal_attention on kv_cache_kv's copy, bit for
    bit, with the DiT's mask (key temporal <= query temporal, dit.rs:643-653);
    also with attention's split mode forced to 4 pieces (the cache's head
    stride is its capacity, the copy's is sk)."""
    if split:
        monkeypatch.setenv("LIGHTX2V_HIP_ATTN_SPLIT", split)
    heads, ft = 2, 40
    dtype = H.DTYPE_BF16
    c = _new(be, heads, hd, 5 * ft, dtype)  # small capacity: the head stride moves as it grows
    rng = np.random.default_rng(hd)
    for chunk in range(5):
        rows = 3 * ft
        temporal = [chunk * 3 + i // ft for i in range(rows)]
        k = O.bf16_round(rng.standard_normal((heads, rows, hd)).astype(np.float32))
        v = O.bf16_round(rng.standard_normal((heads, rows, hd)).astype(np.float32))
        c.put(_up(be, k, dtype), _up(be, v, dtype), rows, temporal)
        c.memrope_update(CFG, ft)
    sq, sk = 3 * ft, len(c)
    tq = np.array([12 + i // ft for i in range(sq)])
    mask = np.array(c.temporal())[None, :] <= tq[:, None]
    q = O.bf16_round(rng.standard_normal((heads, sq, hd)).astype(np.float32))
    qb = _up(be, q, dtype)
    m = be.mask_upload(mask, sq, sk)
    o1, o2 = be.alloc(sq * heads * hd, H.DTYPE_F32), be.alloc(sq * heads * hd, H.DTYPE_F32)
    c.attention(qb, sq, m, o1)
    kb, vb = c.kv()
    be.causal_attention(qb, kb, vb, heads, sq, sk, hd, m, o2)
    assert np.array_equal(u32(be.download(o1)), u32(be.download(o2)))
    # the same mask built on the device from the temporal indices
    mt = be.mask_temporal(tq, c.temporal())
    o3 = be.alloc(sq * heads * hd, H.DTYPE_F32)
    c.attention(qb, sq, mt, o3)
    assert np.array_equal(u32(be.download(o3)), u32(be.download(o2)))
    mt.free()
    # dense (no mask) as well
    c.attention(qb, sq, None, o1)
    be.attention(qb, kb, vb, heads, sq, sk, hd, o2)
    assert np.array_equal(u32(be.download(o1)), u32(be.download(o2)))
    m.free()


@pytest.mark.parametrize("hd", [128, 48])
def test_mask_temporal_matches_host_mask(be, hd):
    """Random (unsorted, repeated) temporal indices, ragged sizes: the device-built
    mask gives the same attention as the host-built one, bit for bit."""
    rng = np.random.default_rng(hd + 1)
    heads, sq, sk = 2, 300, 777
    tq = rng.integers(0, 40, sq)
    tk = rng.integers(0, 40, sk)
    tk[5] = 0  # every query has an allowed key
    mask = tk[None, :] <= tq[:, None]
    q = O.bf16_round(rng.standard_normal((heads, sq, hd)).astype(np.float32))
    k = O.bf16_round(rng.standard_normal((heads, sk, hd)).astype(np.float32))
    v = O.bf16_round(rng.standard_normal((heads, sk, hd)).astype(np.float32))
    qb, kb, vb = (_up(be, a, H.DTYPE_BF16) for a in (q, k, v))
    o1, o2 = be.alloc(sq * heads * hd, H.DTYPE_F32), be.alloc(sq * heads * hd, H.DTYPE_F32)
    m1, m2 = be.mask_upload(mask, sq, sk), be.mask_temporal(tq, tk)
    be.causal_attention(qb, kb, vb, heads, sq, sk, hd, m1, o1)
    be.causal_attention(qb, kb, vb, heads, sq, sk, hd, m2, o2)
    assert np.array_equal(u32(be.download(o1)), u32(be.download(o2)))
    m1.free()
    m2.free()


def test_wan_shape(be):
    """12 heads x 128, 1560-token frames (Wan2.1-1.3B at 480x832), BF16:
    five chunks with a re-run step each, against the oracle bit for bit."""
    heads, hd, ft = 12, 128, 1560
    rows = 3 * ft
    c = _new(be, heads, hd, OCFG.cache_frames * ft, H.DTYPE_BF16)
    oc = KC.KvCache(heads, hd, OCFG.cache_frames * ft)
    rng = np.random.default_rng(9)
    for chunk in range(5):
        temporal = [chunk * 3 + i // ft for i in range(rows)]
        for step in range(2):
            k = O.bf16_round(rng.standard_normal((heads, rows, hd)).astype(np.float32))
            v = O.bf16_round(rng.standard_normal((heads, rows, hd)).astype(np.float32))
            c.put(_up(be, k, H.DTYPE_BF16), _up(be, v, H.DTYPE_BF16), rows, temporal)
            oc.put(k, v, rows, temporal)
            c.memrope_update(CFG, ft)
            oc.memrope_update(OCFG, ft)
            _bf16_oracle_rows(oc, H.DTYPE_BF16)
        _check_rows(c, oc)
    _check_kv(be, c, oc, H.DTYPE_BF16)
    assert len(c) == 12 * ft


def test_kv_cache_errors(be):
    heads, hd = 2, 16
    c = _new(be, heads, hd, 8, H.DTYPE_F32)
    k = be.alloc(heads * 4 * hd, H.DTYPE_F32)
    with pytest.raises(H.HipError):  # k too short for 5 rows
        c.append(k, k, 5, list(range(5)))
    with pytest.raises(H.HipError):  # temporal length
        c.put(k, k, 4, [0, 1])
    with pytest.raises(H.HipError):  # E4M3 input
        c.append(be.alloc_e4m3(4, heads * hd), k, 4, list(range(4)))
    c.append(k, k, 4, list(range(4)))
    q = be.alloc(heads * 3 * hd, H.DTYPE_F32)
    out = be.alloc(3 * heads * hd, H.DTYPE_F32)
    with pytest.raises(H.HipError):  # heads differ from the cache's
        H._check(H.lib.lx2v_hip_kv_cache_attention(be.ctx, q.h, c.h, heads + 1, 3, hd, None, out.h))
    m = be.mask_upload(np.ones((3, 5), bool), 3, 5)
    with pytest.raises(H.HipError):  # mask for 5 keys, the cache holds 4
        c.attention(q, 3, m, out)
    with pytest.raises(H.HipError):  # frame_tokens 0
        c.memrope_update(CFG, 0)
    small = be.alloc(heads * 3 * hd, H.DTYPE_F32)
    with pytest.raises(H.HipError):  # read into buffers shorter than the cache
        c.read(small, small)
    c.free()

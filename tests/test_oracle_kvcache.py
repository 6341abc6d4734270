"""The oracle's KV cache (oracle/kvcache.py) pinned against the reference's own
tests and against what the mathematics fixes.

Reference tests restated here (their assertions, on the same inputs):
* crates/lightx2v-model/tests/conformance.rs:141-178
  (cpu_kv_cache_memrope_bounds_and_keeps_sinks: 40 frames of 2 tokens);
* crates/lightx2v-core/src/memrope.rs:248-258 (ema_update_math) and
  :260-306 (sinks pinned, one long and one short slot, temporal order);
* crates/lightx2v-wgpu/src/lib.rs:1640-1670 (7 chunks x 4 DMD steps of
  put + update: step 0 appends, re-runs overwrite in place).
Closed forms: a slot folded with frames f_1..f_n holds
sum_i alpha (1 - alpha)^(n - i) f_i (+ (1 - alpha)^n of its start), which a
reversed fold order or a swapped alpha fails.
"""

import numpy as np

from oracle import kvcache as KC


def _rng_kv(rng, heads, rows, hd):
    return (rng.standard_normal((heads, rows, hd)).astype(np.float32),
            rng.standard_normal((heads, rows, hd)).astype(np.float32))


def test_ema_update_kat():
    ema = np.array([1.0, 2.0, 3.0], np.float32)
    frame = np.array([11.0, 12.0, 13.0], np.float32)
    out = KC.ema_update(ema, frame, 0.1)
    assert abs(out[0] - 2.0) < 1e-6 and abs(out[1] - 3.0) < 1e-6
    assert np.array_equal(KC.ema_update(ema, frame, 1.0), frame)
    assert np.array_equal(KC.ema_update(ema, frame, 0.0), ema)
    # no fused multiply-add: the two products round apart
    a = np.float32(0.1)
    want = (np.float32(1) - a) * np.float32(1.0) + a * np.float32(11.0)
    assert out[0] == want


def test_conformance_bounds_and_keeps_sinks():
    cfg = KC.MemRopeConfig()
    heads, hd, ft = 2, 4, 2
    c = KC.KvCache(heads, hd, cfg.cache_frames * ft)
    rng = np.random.default_rng(21)
    for frame in range(40):
        k, v = _rng_kv(rng, heads, ft, hd)
        c.append(k, v, ft, [frame] * ft)
        c.memrope_update(cfg, ft)
        assert c.rows() <= cfg.cache_frames * ft, frame
    t = c.temporal
    assert t[:ft * 3] == [0, 0, 1, 1, 2, 2]
    assert t[-1] == 39
    assert len(t) // ft == 12
    distinct = set(t)
    assert len(distinct) == 11 and 0 in distinct and 39 in distinct
    k, v = c.kv()
    assert k.shape == (heads, c.rows(), hd) and v.shape == k.shape


def test_layout_slots_and_order():
    cfg = KC.MemRopeConfig()
    ft = 3
    c = KC.KvCache(1, 2, 36)
    for t in range(40):
        c.append(np.full((1, ft, 2), t, np.float32), np.full((1, ft, 2), -t, np.float32), ft, [t] * ft)
        c.memrope_update(cfg, ft)
        assert c.rows() // ft <= 12
    fk = [c.kinds[f * ft] for f in range(c.rows() // ft)]
    assert fk == [KC.SINK] * 3 + [KC.LONG_EMA, KC.SHORT_EMA] + [KC.RECENT] * 4 + [KC.NEW] * 3
    sinks = [c.temporal[f * ft] for f in range(3)]
    assert sinks == [0, 1, 2]
    idx = [c.temporal[f * ft] for f, kd in enumerate(fk) if kd not in (KC.LONG_EMA, KC.SHORT_EMA)]
    assert all(a < b for a, b in zip(idx, idx[1:])), idx
    # every frame's rows share its temporal index and kind
    for f in range(len(fk)):
        assert len(set(c.temporal[f * ft:(f + 1) * ft])) == 1 and len(set(c.kinds[f * ft:(f + 1) * ft])) == 1


def test_ema_slots_closed_form():
    """Constant frames t: the slots hold the exponentially weighted sums of the
    evicted frames 3, 4, ... (the first non-sink frames, in order)."""
    cfg = KC.MemRopeConfig()
    ft = 1
    c = KC.KvCache(1, 1, 12)
    n = 30
    for t in range(n):
        c.append(np.full((1, 1, 1), float(t), np.float32), np.full((1, 1, 1), 2.0 * t, np.float32), 1, [t])
        c.memrope_update(cfg, ft)
    evicted = [t for t in range(3, n) if t not in c.temporal[5:]]
    for kind, alpha in ((KC.LONG_EMA, cfg.ema_alpha_long), (KC.SHORT_EMA, cfg.ema_alpha_short)):
        r = c.kinds.index(kind)
        m = len(evicted)
        want = sum(alpha * (1 - alpha) ** (m - 1 - i) * f for i, f in enumerate(evicted))
        assert abs(float(c.k[r, 0]) - want) <= 1e-5 * max(1.0, abs(want)), (kind, c.k[r, 0], want)
        assert abs(float(c.v[r, 0]) - 2 * want) <= 2e-5 * max(1.0, abs(want))
        rev = sum(alpha * (1 - alpha) ** i * f for i, f in enumerate(evicted))
        assert abs(rev - want) > 1e-3  # the order is pinned


def test_put_overwrites_reruns_in_place():
    """The DiT's pattern: a chunk of 3 frames, put + update on each of 4 DMD
    steps; step 0 appends, steps 1-3 overwrite the same rows."""
    cfg = KC.MemRopeConfig()
    heads, hd, ft = 2, 4, 5
    rows = 3 * ft
    c = KC.KvCache(heads, hd, cfg.cache_frames * ft)
    rng = np.random.default_rng(7)
    for chunk in range(7):
        temporal = [chunk * 3 + i // ft for i in range(rows)]
        for step in range(4):
            before = c.rows()
            k, v = _rng_kv(rng, heads, rows, hd)
            c.put(k, v, rows, temporal)
            if step > 0:
                assert c.rows() == before
                pos = next(i for i, (t, kd) in enumerate(zip(c.temporal, c.kinds))
                           if t == temporal[0] and kd not in (KC.LONG_EMA, KC.SHORT_EMA))
                kk, _ = c.kv()
                assert np.array_equal(kk[:, pos:pos + rows], k)
            c.memrope_update(cfg, ft)
            assert c.rows() <= cfg.cache_frames * ft
    assert c.temporal[-1] == 20


def test_put_skips_ema_slots():
    """EMA slots carry the first non-sink frame's temporal index; put of that
    index must not land on them (lib.rs:652-661)."""
    cfg = KC.MemRopeConfig()
    ft = 1
    c = KC.KvCache(1, 1, 12)
    for t in range(5):
        c.append(np.full((1, 1, 1), float(t + 1), np.float32), np.zeros((1, 1, 1), np.float32), 1, [t])
        c.memrope_update(cfg, ft)
    assert c.kinds[3] == KC.LONG_EMA and c.kinds[4] == KC.SHORT_EMA and c.temporal[3] == 3
    c.put(np.full((1, 1, 1), 99.0, np.float32), np.zeros((1, 1, 1), np.float32), 1, [3])
    r = [i for i, (t, kd) in enumerate(zip(c.temporal, c.kinds)) if t == 3 and kd == KC.RECENT or
         (t == 3 and kd == KC.NEW)]
    assert c.k[r[0], 0] == 99.0 and c.k[3, 0] == 0.0 and c.k[4, 0] == 0.0

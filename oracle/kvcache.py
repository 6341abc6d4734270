"""Restatement of the reference CPU backend's per-layer KV cache (TEST INFRASTRUCTURE).

Only ``tests/`` may use this module, as the checker of the device cache.

Follows crates/lightx2v-cpu/src/lib.rs:126-146 (the ``KvCache`` struct: K/V
rows ``[rows, heads*head_dim]`` f32, a temporal index and a slot kind per
row) and its ``Backend`` methods at lib.rs:607-806:

* ``append``          lib.rs:620-645
* ``put``             lib.rs:647-678
* ``kv``              lib.rs:689-705  (re-emitted as ``[heads, rows, d]``)
* ``memrope_update``  lib.rs:707-806, with ``ema_update`` from
  crates/lightx2v-core/src/memrope.rs:57-63 and ``MemRopeConfig``'s
  defaults / ``new_frames() == 3`` from crates/lightx2v-core/src/config.rs:265-300.

Arithmetic: the EMA is ``(1 - alpha) * e + alpha * f`` in f32 with no fused
multiply-add (Rust evaluates the two products and the sum separately);
numpy float32 scalars and arrays do the same, so results are bit-exact.
Everything else is row bookkeeping and copies.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

# SlotKind (crates/lightx2v-core/src/memrope.rs:31-37), in declaration order.
SINK, LONG_EMA, SHORT_EMA, RECENT, NEW = range(5)


@dataclass
class MemRopeConfig:
    """config.rs:265-300 (the fields the cache reads)."""

    cache_frames: int = 12
    sink_frames: int = 3
    ema_alpha_long: float = 0.01
    ema_alpha_short: float = 0.1

    def new_frames(self) -> int:  # config.rs:298-300
        return 3


def ema_update(ema: np.ndarray, frame: np.ndarray, alpha: float) -> np.ndarray:
    """memrope.rs:57-63: (1 - alpha) * e + alpha * f, f32, no FMA."""
    a = np.float32(alpha)
    return ((np.float32(1.0) - a) * ema.astype(np.float32) + a * frame.astype(np.float32)).astype(np.float32)


class KvCache:
    def __init__(self, heads: int, head_dim: int, capacity_tokens: int):
        self.heads, self.head_dim, self.capacity_tokens = heads, head_dim, capacity_tokens
        self.k = np.zeros((0, heads * head_dim), np.float32)
        self.v = np.zeros((0, heads * head_dim), np.float32)
        self.temporal: list[int] = []
        self.kinds: list[int] = []

    def rows(self) -> int:
        return len(self.temporal)

    def _rows_of(self, x: np.ndarray, rows: int) -> np.ndarray:
        """[heads, rows, d] -> [rows, heads*d] (lib.rs:632-638's copy order)."""
        return np.ascontiguousarray(np.asarray(x, np.float32).reshape(self.heads, rows, self.head_dim)
                                    .transpose(1, 0, 2).reshape(rows, self.heads * self.head_dim))

    def append(self, k, v, rows: int, temporal) -> None:
        """lib.rs:620-645: rows appended as New."""
        assert len(temporal) == rows
        self.k = np.concatenate([self.k, self._rows_of(k, rows)])
        self.v = np.concatenate([self.v, self._rows_of(v, rows)])
        self.temporal += [int(t) for t in temporal]
        self.kinds += [NEW] * rows

    def put(self, k, v, rows: int, temporal) -> None:
        """lib.rs:647-678: overwrite in place when the first non-EMA row with
        temporal[0] starts a run equal to `temporal`, else append."""
        assert len(temporal) == rows
        pos = next((i for i, (t, kd) in enumerate(zip(self.temporal, self.kinds))
                    if t == temporal[0] and kd not in (LONG_EMA, SHORT_EMA)), None)
        if pos is not None and all(pos + i < self.rows() and self.temporal[pos + i] == temporal[i]
                                   for i in range(rows)):
            self.k[pos:pos + rows] = self._rows_of(k, rows)
            self.v[pos:pos + rows] = self._rows_of(v, rows)
            return
        self.append(k, v, rows, temporal)

    def kv(self):
        """lib.rs:689-705: K and V as [heads, rows, d]."""
        r = self.rows()
        f = lambda x: np.ascontiguousarray(x.reshape(r, self.heads, self.head_dim).transpose(1, 0, 2))
        return f(self.k), f(self.v)

    def memrope_update(self, cfg: MemRopeConfig, frame_tokens: int) -> None:
        """lib.rs:707-806."""
        ft = frame_tokens
        n_frames = self.rows() // ft
        if n_frames == 0:
            return
        frame_kind = [self.kinds[f * ft] for f in range(n_frames)]
        # seed the two zero EMA frames after the sinks (lib.rs:728-752)
        if LONG_EMA not in frame_kind and n_frames > cfg.sink_frames:
            at = cfg.sink_frames * ft
            t = self.temporal[min(at, max(self.rows() - 1, 0))]
            zero = np.zeros((ft, self.k.shape[1]), np.float32)
            for kind in (SHORT_EMA, LONG_EMA):
                self.k = np.concatenate([self.k[:at], zero, self.k[at:]])
                self.v = np.concatenate([self.v[:at], zero, self.v[at:]])
                self.temporal[at:at] = [t] * ft
                self.kinds[at:at] = [kind] * ft
            frame_kind = [self.kinds[f * ft] for f in range(self.rows() // ft)]
        # graduate New frames past the window to Recent (lib.rs:754-768)
        new_frames = [i for i, kd in enumerate(frame_kind) if kd == NEW]
        if len(new_frames) > cfg.new_frames():
            for f in new_frames[:len(new_frames) - cfg.new_frames()]:
                self.kinds[f * ft:(f + 1) * ft] = [RECENT] * ft
        # fold and evict while over capacity (lib.rs:769-799)
        while self.rows() // ft > cfg.cache_frames:
            kinds_now = [self.kinds[f * ft] for f in range(self.rows() // ft)]
            evict = next((i for i, kd in enumerate(kinds_now) if kd == RECENT), None)
            if evict is None:
                evict = next((i for i, kd in enumerate(kinds_now) if kd == NEW), None)
            if evict is None:
                break
            f = evict
            ev_k, ev_v = self.k[f * ft:(f + 1) * ft].copy(), self.v[f * ft:(f + 1) * ft].copy()
            for slot_kind, alpha in ((LONG_EMA, cfg.ema_alpha_long), (SHORT_EMA, cfg.ema_alpha_short)):
                sf = next((i for i, kd in enumerate(kinds_now) if kd == slot_kind), None)
                if sf is not None:
                    sl = slice(sf * ft, (sf + 1) * ft)
                    self.k[sl] = ema_update(self.k[sl], ev_k, alpha)
                    self.v[sl] = ema_update(self.v[sl], ev_v, alpha)
            keep = np.r_[0:f * ft, (f + 1) * ft:self.rows()]
            self.k, self.v = self.k[keep], self.v[keep]
            del self.temporal[f * ft:(f + 1) * ft]
            del self.kinds[f * ft:(f + 1) * ft]
        # the first sink_frames frames are sinks (lib.rs:800-805)
        for f in range(min(cfg.sink_frames, self.rows() // ft)):
            self.kinds[f * ft:(f + 1) * ft] = [SINK] * ft

"""Which DiT block linears get which quantized format, and the quantized
forms a checkpoint stores them in.

Host-side mirror of ``crates/lightx2v-core/src/quant.rs``:

* ``WeightQuant`` -- the format enum (quant.rs:26-43) with ``attn``
  (:46-53), ``for_key`` (:55-72), ``str`` (the ``Display`` impl, :74-92) and
  ``parse`` (the ``FromStr`` impl, :94-132), same strings, same defaults and
  the same error messages;
* ``StoredQ8`` / ``StoredQ4`` / ``StoredFp8`` -- the ``Stored`` variants
  (:134-140), i.e. the ``Q8`` / ``Q4`` / ``Fp8E4M3`` structs as read from a
  file, with ``concat`` (:189-200, :339-351) and the reference's group
  fallback (:155-159, :227-231, :424-428).

Quantizing happens on the device (``HipBackend.quantize_q8`` /
``quantize_q4`` / ``quantize_fp8_ref``); this module only decides formats and
carries codes.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field
from typing import List

import numpy as np

# quant.rs:18-23
Q8_GROUP = 128
FP8_GROUP = 128
FP8_E4M3_MAX = 448.0

_BLOCK_FORMAT_ROLES = ("ffn.net.0.proj", "ffn.net.2")
_BLOCK_ATTN_ROLES = ("attn1.to_q", "attn1.to_k", "attn1.to_v", "attn1.to_out.0", "attn2.to_q",
                     "attn2.to_k", "attn2.to_v", "attn2.to_out.0", "to_gate_compress")
# Rust's usize::from_str: an optional '+', then ASCII digits only.
_USIZE = re.compile(r"\+?[0-9]+")


@dataclass(frozen=True)
class WeightQuant:
    """``WeightQuant`` (quant.rs:26-43): ``native``, ``int8``, ``fp8`` or
    ``int4`` with its group, HQQ flag and FFN-only flag."""

    kind: str = "native"
    group: int = 0
    hqq: bool = False
    ffn_only: bool = False

    @staticmethod
    def native() -> "WeightQuant":
        return WeightQuant("native")

    @staticmethod
    def int8() -> "WeightQuant":
        return WeightQuant("int8")

    @staticmethod
    def fp8() -> "WeightQuant":
        return WeightQuant("fp8")

    @staticmethod
    def int4(group: int = 64, hqq: bool = False, ffn_only: bool = False) -> "WeightQuant":
        return WeightQuant("int4", group, hqq, ffn_only)

    def attn(self) -> "WeightQuant":
        """The format of the non-FFN block linears (quant.rs:46-53)."""
        if self.kind == "int4" and self.ffn_only:
            return WeightQuant.int8()
        return self

    def for_key(self, key: str) -> "WeightQuant":
        """The format of block linear ``key`` (``blocks.N.<role>``, no
        ``.weight``), quant.rs:55-72: the FFN gets ``self``, attention and the
        gate get ``attn()``, everything else is native."""
        if not key.startswith("blocks."):
            return WeightQuant.native()
        rest = key[len("blocks."):]
        if "." not in rest:
            return WeightQuant.native()
        role = rest.split(".", 1)[1]
        if role in _BLOCK_FORMAT_ROLES:
            return self
        if role in _BLOCK_ATTN_ROLES:
            return self.attn()
        return WeightQuant.native()

    def __str__(self) -> str:  # quant.rs:74-92
        if self.kind == "int4":
            return "int4{}-g{}{}".format("-hqq" if self.hqq else "", self.group, "-ffn" if self.ffn_only else "")
        return {"native": "native", "int8": "int8", "fp8": "fp8-e4m3"}[self.kind]

    @staticmethod
    def parse(s: str) -> "WeightQuant":
        """``FromStr`` (quant.rs:94-132); raises ValueError with the
        reference's message."""
        if s in ("native", "bf16", "f16"):
            return WeightQuant.native()
        if s in ("int8", "q8"):
            return WeightQuant.int8()
        if s in ("fp8", "fp8-e4m3"):
            return WeightQuant.fp8()
        # int4[-hqq][-g<N>][-ffn]
        ffn_only = s.endswith("-ffn")
        if ffn_only:
            s = s[: -len("-ffn")]
        if not s.startswith("int4"):
            raise ValueError(f"unknown weight format `{s}` (native | int8 | fp8 | int4[-hqq][-gN][-ffn])")
        rest = s[len("int4"):]
        hqq = rest.startswith("-hqq")
        if hqq:
            rest = rest[len("-hqq"):]
        if rest.startswith("-g"):
            g = rest[2:]
            if not _USIZE.fullmatch(g) or int(g) >= 1 << 64:
                raise ValueError(f"bad group in `{s}`")
            group = int(g)
        elif rest == "":
            group = 64
        else:
            raise ValueError(f"bad weight format `{s}`")
        if group == 0 or group % 8 != 0:
            raise ValueError(f"int4 group must be a multiple of 8, got {group}")
        return WeightQuant.int4(group, hqq, ffn_only)


def group_or_cols(group: int, cols: int) -> int:
    """The reference quantizers' group: ``group`` when it divides ``cols``,
    else one group per row (quant.rs:155-159, 227-231, 424-428)."""
    return group if cols % group == 0 else cols


@dataclass
class StoredQ8:
    """``Q8`` (quant.rs:142-151): int8 codes [rows, cols], f32 scales [rows, cols / group]."""

    q: np.ndarray
    scales: np.ndarray
    rows: int
    cols: int
    group: int
    fmt: str = field(default="q8", init=False)

    @staticmethod
    def concat(parts: List["StoredQ8"]) -> "StoredQ8":
        """Stack by rows (fused QKV), quant.rs:189-200: columns and group must agree."""
        a = parts[0]
        for b in parts[1:]:
            if (a.cols, a.group) != (b.cols, b.group):
                raise ValueError(f"q8 concat: ({a.cols}, {a.group}) vs ({b.cols}, {b.group})")
        return StoredQ8(np.concatenate([p.q.reshape(-1) for p in parts]),
                        np.concatenate([p.scales.reshape(-1) for p in parts]),
                        sum(p.rows for p in parts), a.cols, a.group)


@dataclass
class StoredQ4:
    """``Q4`` (quant.rs:207-224): one 4-bit code per byte [rows * cols],
    f32 scales and zeros [rows, cols / group] (f16 values), ``w = (q - zero) * scale``."""

    q: np.ndarray
    scales: np.ndarray
    zeros: np.ndarray
    rows: int
    cols: int
    group: int
    fmt: str = field(default="q4", init=False)

    @staticmethod
    def from_packed(packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray, rows: int,
                    cols: int) -> "StoredQ4":
        """quant.rs:313-336: element 2i is the low nibble of byte i; the group
        is rows * cols / len(scales)."""
        n = rows * cols
        packed = np.asarray(packed, np.uint8).reshape(-1)
        scales = np.asarray(scales, np.float32).reshape(-1)
        zeros = np.asarray(zeros, np.float32).reshape(-1)
        if packed.size != (n + 1) // 2:
            raise ValueError(f"q4: {packed.size} packed bytes for {rows}x{cols}")
        if scales.size == 0 or scales.size != zeros.size or n % scales.size:
            raise ValueError(f"q4: {scales.size} scales / {zeros.size} zeros for {rows}x{cols}")
        q = np.empty(2 * packed.size, np.uint8)
        q[0::2] = packed & 15
        q[1::2] = packed >> 4
        return StoredQ4(q[:n], scales, zeros, rows, cols, n // scales.size)

    def packed(self) -> np.ndarray:
        """quant.rs:305-311."""
        q = self.q.reshape(-1)
        if q.size % 2:
            q = np.concatenate([q, np.zeros(1, np.uint8)])
        return (q[0::2] | (q[1::2] << 4)).astype(np.uint8)

    @staticmethod
    def concat(parts: List["StoredQ4"]) -> "StoredQ4":
        """quant.rs:339-351."""
        a = parts[0]
        for b in parts[1:]:
            if (a.cols, a.group) != (b.cols, b.group):
                raise ValueError(f"q4 concat: ({a.cols}, {a.group}) vs ({b.cols}, {b.group})")
        return StoredQ4(np.concatenate([p.q.reshape(-1) for p in parts]),
                        np.concatenate([p.scales.reshape(-1) for p in parts]),
                        np.concatenate([p.zeros.reshape(-1) for p in parts]),
                        sum(p.rows for p in parts), a.cols, a.group)


@dataclass
class StoredFp8:
    """``Fp8E4M3`` (quant.rs:364-373): e4m3 code bytes [rows, cols], f32 scales [rows * cols / group]."""

    q: np.ndarray
    scales: np.ndarray
    rows: int
    cols: int
    group: int
    fmt: str = field(default="fp8", init=False)

    @staticmethod
    def concat(parts: List["StoredFp8"]) -> "StoredFp8":
        """Row stacking as dit.rs:128-150 does it (codes and scales appended,
        the first part's group).  Parts whose columns or group differ would make
        a malformed struct there; here they are an error."""
        a = parts[0]
        for b in parts[1:]:
            if (a.cols, a.group) != (b.cols, b.group):
                raise ValueError(f"fp8 concat: ({a.cols}, {a.group}) vs ({b.cols}, {b.group})")
        return StoredFp8(np.concatenate([p.q.reshape(-1) for p in parts]),
                         np.concatenate([p.scales.reshape(-1) for p in parts]),
                         sum(p.rows for p in parts), a.cols, a.group)

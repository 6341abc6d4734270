"""Checkpoint ingest for the quantized linear path.

Host-side mirror of the parts of lightx2v-rs that feed ``Backend::linear``
its weights:

* ``SafetensorsSource`` -- ``SafetensorsDir`` as a ``WeightSource``
  (crates/lightx2v-core/src/weights.rs:17-35, 80-260): ``get`` converts an
  F32 / F16 / BF16 tensor to f32 after the size-1-dims-ignored shape check,
  ``stored`` reads ``<key>.weight.q8`` / ``.q4`` / ``.fp8`` with their
  ``.scale`` (and ``.zero``) exactly as the reference validates them;
* ``load_linear`` -- dit.rs:61-157: fused QKV / KV stacked by rows, stored
  codes handed to ``weight_q8/q4/fp8`` untouched, f32 rows quantized at load
  by ``WeightQuant.for_key`` (on the device, with the reference's
  arithmetic);
* ``quantized_linear_tensors`` / ``write_safetensors`` -- the tensors
  ``quantize_dit`` writes for one linear (export.rs:44-130) and the
  order-preserving writer (export.rs:161-252).

The safetensors format itself (8-byte little-endian header length, JSON
header of dtype / shape / data_offsets, then the data) is read and written
here directly, so BF16 and F16 need no framework.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from typing import Dict, Iterable, List, Optional, Sequence, Tuple, Union

import numpy as np

from . import DTYPE_F32, HipBackend, Buf, Weight
from .quant import (FP8_GROUP, Q8_GROUP, StoredFp8, StoredQ4, StoredQ8, WeightQuant, group_or_cols)

_NP = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "I64": np.int64, "I32": np.int32,
       "I16": np.int16, "I8": np.int8, "U8": np.uint8, "BOOL": np.bool_}
_SIZE = {"F64": 8, "F32": 4, "F16": 2, "BF16": 2, "I64": 8, "I32": 4, "I16": 2, "I8": 1, "U8": 1, "BOOL": 1}

Stored = Union[StoredQ8, StoredQ4, StoredFp8]


class WeightsError(ValueError):
    """``Error::Weights``: a missing tensor, a shape or dtype mismatch."""


def _squeeze(shape: Sequence[int]) -> List[int]:
    return [d for d in shape if d != 1]  # weights.rs:37-39


def bf16_to_f32(raw: np.ndarray) -> np.ndarray:
    return (raw.astype(np.uint32) << 16).view(np.float32)


class SafetensorsSource:
    """One or more .safetensors files as a ``WeightSource`` (weights.rs:80-130)."""

    def __init__(self, paths: Union[str, Iterable[str]]):
        if isinstance(paths, (str, os.PathLike)):
            p = str(paths)
            paths = sorted(os.path.join(p, f) for f in os.listdir(p) if f.endswith(".safetensors")) \
                if os.path.isdir(p) else [p]
        self._files = []
        self._index: Dict[str, int] = {}
        for i, path in enumerate(paths):
            with open(path, "rb") as f:
                n = int.from_bytes(f.read(8), "little")
                header = json.loads(f.read(n))
            data = np.memmap(path, np.uint8, "r", offset=8 + n) if os.path.getsize(path) > 8 + n \
                else np.zeros(0, np.uint8)
            header.pop("__metadata__", None)
            self._files.append((header, data))
            for name in header:
                self._index[name] = i
        if not self._files:
            raise WeightsError(f"no .safetensors in {paths}")

    def names(self):
        return self._index.keys()

    def contains(self, name: str) -> bool:
        return name in self._index

    def has_linear(self, key: str) -> bool:  # weights.rs:28-34
        return any(self.contains(f"{key}.weight{s}") for s in ("", ".q8", ".q4", ".fp8"))

    def raw(self, name: str) -> Tuple[str, List[int], np.ndarray]:
        """The stored bytes without conversion: (dtype, shape, uint8 data)."""
        if name not in self._index:
            raise WeightsError(f"missing tensor `{name}`")
        header, data = self._files[self._index[name]]
        t = header[name]
        b, e = t["data_offsets"]
        return t["dtype"], list(t["shape"]), data[b:e]

    def get(self, name: str, shape: Sequence[int]) -> np.ndarray:
        """The tensor as f32 (weights.rs:210-250): F32, F16 or BF16, shape
        checked with size-1 dims ignored."""
        dt, tshape, b = self.raw(name)
        if _squeeze(tshape) != _squeeze(shape):
            raise WeightsError(f"`{name}` is {tshape}, expected {list(shape)}")
        if dt == "F32":
            return np.frombuffer(b, "<f4").astype(np.float32)
        if dt == "F16":
            return np.frombuffer(b, "<f2").astype(np.float32)
        if dt == "BF16":
            return bf16_to_f32(np.frombuffer(b, "<u2"))
        raise WeightsError(f"`{name}`: unsupported dtype {dt}")

    def _f32s(self, name: str):
        _, shape, _ = self.raw(name)
        return shape, self.get(name, shape)

    def stored(self, key: str) -> Optional[Stored]:
        """The linear ``key`` if stored quantized, else None (weights.rs:131-208)."""
        def bad(m):
            return WeightsError(f"`{key}`: {m}")
        q8, q4, fp8 = f"{key}.weight.q8", f"{key}.weight.q4", f"{key}.weight.fp8"
        if self.contains(q8):
            dt, shape, data = self.raw(q8)
            if dt != "I8" or len(shape) != 2:
                raise bad(f"q8 is {dt} {shape}")
            sshape, scales = self._f32s(f"{key}.weight.scale")
            if len(sshape) != 2 or sshape[0] != shape[0] or shape[1] % sshape[1] != 0:
                raise bad(f"scale {sshape} for codes {shape}")
            return StoredQ8(np.frombuffer(data, np.int8).copy(), scales, shape[0], shape[1],
                            shape[1] // sshape[1])
        if self.contains(q4):
            dt, shape, data = self.raw(q4)
            if dt != "U8" or len(shape) != 2:
                raise bad(f"q4 is {dt} {shape}")
            rows, cols = shape[0], 2 * shape[1]
            sshape, scales = self._f32s(f"{key}.weight.scale")
            zshape, zeros = self._f32s(f"{key}.weight.zero")
            if sshape != zshape or len(sshape) != 2 or sshape[0] != rows or cols % sshape[1] != 0:
                raise bad(f"scale {sshape} / zero {zshape} for codes {shape}")
            return StoredQ4.from_packed(np.asarray(data), scales, zeros, rows, cols)
        if self.contains(fp8):
            dt, shape, data = self.raw(fp8)
            if dt != "U8" or len(shape) != 2:
                raise bad(f"fp8 is {dt} {shape}")
            sshape, scales = self._f32s(f"{key}.weight.scale")
            if len(sshape) != 2 or sshape[0] != shape[0] or shape[1] % sshape[1] != 0:
                raise bad(f"scale {sshape} for codes {shape}")
            return StoredFp8(np.asarray(data).copy(), scales, shape[0], shape[1], shape[1] // sshape[1])
        return None


@dataclass
class Linear:
    """dit.rs ``Linear``: the device weight and its uploaded bias."""

    w: Weight
    b: Buf


def quantize_on_device(be: HipBackend, w: np.ndarray, rows: int, cols: int, fmt: WeightQuant) -> Weight:
    """The weight ``load_linear`` makes from f32 rows (dit.rs:93-103): the
    reference's ``Q8::quantize`` / ``Q4::quantize`` / ``Fp8E4M3::quantize``
    run on the device with its arithmetic (groups as quant.rs picks them)."""
    if fmt.kind == "native":
        return be.weight(w, rows, cols)
    src = be.alloc(rows * cols, DTYPE_F32)
    try:
        be.write(src, w)
        if fmt.kind == "int8":
            return be.quantize_q8(src, rows, cols, group_or_cols(Q8_GROUP, cols))
        if fmt.kind == "int4":
            return be.quantize_q4(src, rows, cols, group_or_cols(fmt.group, cols), fmt.hqq)
        return be.quantize_fp8_ref(src, rows, cols, group_or_cols(FP8_GROUP, cols))
    finally:
        src.free()


def upload_stored(be: HipBackend, s: Stored) -> Weight:
    """``Backend::weight_q8 / weight_q4 / weight_fp8`` of a stored struct."""
    if isinstance(s, StoredQ8):
        return be.weight_q8(s.q, s.scales, s.rows, s.cols, s.group)
    if isinstance(s, StoredQ4):
        return be.weight_q4(s.q, s.scales, s.zeros, s.rows, s.cols, s.group)
    return be.weight_fp8(s.q, s.scales, s.rows, s.cols, s.group)


def load_linear(be: HipBackend, src, shapes: Dict[str, Sequence[int]], keys: Sequence[str],
                quant: WeightQuant) -> Linear:
    """Several ``nn.Linear``s stacked by rows into one matrix (fused QKV /
    KV), each checked against its manifest shape -- dit.rs:61-157, same
    checks, same messages."""
    w_rows: List[np.ndarray] = []
    bias: List[np.ndarray] = []
    stored: List[Stored] = []
    rows = cols = 0
    for k in keys:
        shape = shapes.get(f"{k}.weight")
        if shape is None:
            raise WeightsError(f"`{k}` is not in the manifest")
        o, i = shape[0], int(np.prod(shape[1:], dtype=np.int64))
        s = src.stored(k)
        if s is not None:
            if (s.rows, s.cols) != (o, i):
                raise WeightsError(f"`{k}` is stored {s.rows}x{s.cols}, expected {o}x{i}")
            stored.append(s)
        else:
            w_rows.append(src.get(f"{k}.weight", shape))
        bias.append(src.get(f"{k}.bias", [o]))
        rows += o
        cols = i
    if not stored:
        w = quantize_on_device(be, np.concatenate(w_rows), rows, cols, quant.for_key(keys[0]))
    elif len(stored) != len(keys):
        raise WeightsError(f"{list(keys)}: only some are stored quantized")
    elif all(isinstance(s, StoredQ8) for s in stored):
        w = upload_stored(be, StoredQ8.concat(stored))
    elif all(isinstance(s, StoredQ4) for s in stored):
        w = upload_stored(be, StoredQ4.concat(stored))
    elif all(isinstance(s, StoredFp8) for s in stored):
        w = upload_stored(be, StoredFp8.concat(stored))
    else:
        raise WeightsError(f"{list(keys)}: mixed quantized storage")
    return Linear(w, be.upload(np.concatenate(bias)))


# ---- writing a quantized checkpoint (export.rs) ------------------------------------

Tensor = Tuple[str, str, List[int], bytes]  # name, dtype, shape, little-endian bytes


def f16_bytes(v: np.ndarray) -> bytes:
    return np.asarray(v, np.float32).astype("<f2").tobytes()  # IEEE round to nearest even


def f32_bytes(v: np.ndarray) -> bytes:
    return np.asarray(v, "<f4").tobytes()


def quantized_linear_tensors(be: HipBackend, name: str, w: Weight) -> List[Tensor]:
    """The tensors ``quantize_dit`` writes for the linear weight ``name``
    (``X.weight``), export.rs:72-124: ``.q8`` I8 + ``.scale`` F32, ``.q4`` U8
    [out, in / 2] + ``.scale`` / ``.zero`` F16, ``.fp8`` U8 + ``.scale`` F32."""
    e = be.weight_export(w)
    rows, cols, ng = e["rows"], e["cols"], e["cols"] // e["group"]
    if e["fmt"] == 1:
        return [(f"{name}.q8", "I8", [rows, cols], e["q"].tobytes()),
                (f"{name}.scale", "F32", [rows, ng], f32_bytes(e["scales"]))]
    if e["fmt"] == 2:
        if cols % 2:
            raise WeightsError(f"`{name}`: 4-bit needs an even row length, got {cols}")
        return [(f"{name}.q4", "U8", [rows, cols // 2], e["q"].tobytes()),
                (f"{name}.scale", "F16", [rows, ng], f16_bytes(e["scales"])),
                (f"{name}.zero", "F16", [rows, ng], f16_bytes(e["zeros"]))]
    if e["fmt"] == 3:
        return [(f"{name}.fp8", "U8", [rows, cols], e["q"].tobytes()),
                (f"{name}.scale", "F32", [rows, ng], f32_bytes(e["scales"]))]
    raise WeightsError(f"`{name}` is not quantized")


def metadata(quant: WeightQuant) -> Dict[str, str]:
    """export.rs:262-274."""
    return {"lightx2v.format": "quant/1",
            "lightx2v.weights": "f16" if quant.kind == "native" else str(quant)}


def safetensors_bytes(tensors: Sequence[Tensor], meta: Optional[Dict[str, str]] = None) -> bytes:
    """One safetensors file, tensors in the given order (export.rs:161-252:
    the header is padded with spaces to a multiple of 8 bytes)."""
    header = {}
    if meta:
        header["__metadata__"] = dict(meta)
    off = 0
    for name, dt, shape, data in tensors:
        need = _SIZE[dt] * int(np.prod(shape, dtype=np.int64))
        if len(data) != need:
            raise WeightsError(f"`{name}`: {len(data)} bytes for {dt} {shape}")
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        off += len(data)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    return len(h).to_bytes(8, "little") + h + b"".join(t[3] for t in tensors)


def write_safetensors(path: str, tensors: Sequence[Tensor], meta: Optional[Dict[str, str]] = None):
    with open(path, "wb") as f:
        f.write(safetensors_bytes(tensors, meta))

"""FP8 checkpoint admission: safetensors files holding e4m3 weights.

LunaFlux's safetensors reader validates a header's tensors and accepts BF16
only (model/safetensors/metadata.mbt:90-123: name, dtype, rank, half-open
byte range inside the payload, size equal to the shape's, then
:133-175: no duplicate names, no overlapping ranges). This module applies
the same checks, raising SafetensorsError with the same error kinds, and
admits the dtypes an FP8 checkpoint adds: F8_E4M3 weight codes and their
F32 scales (BF16 stays admitted). A projection weight `<prefix>.weight`
[N, K] F8_E4M3 comes with either `<prefix>.weight_scale` (F32, N values:
per output channel) or `<prefix>.weight_scale_inv` (F32 [N/128, K/128]:
128 x 128 blocks), the dequantized weight being fp32(code) * scale in both
cases; load_fp8_linear returns what fp8.pack_weight takes.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass

import numpy as np

from . import fp8

ITEM_BYTES = {"F8_E4M3": 1, "BF16": 2, "F32": 4}
NUMPY = {"F8_E4M3": np.uint8, "BF16": np.uint16, "F32": np.float32}
MAX_HEADER_BYTES = 100 << 20
MAX_NAME_LENGTH = 512
MAX_RANK = 8


class SafetensorsError(ValueError):
    """kind: one of HeaderTooLarge, InvalidHeader, InvalidTensorName,
    InvalidDType, InvalidRank, InvalidByteRange, RangeOutsidePayload,
    RangeSizeMismatch, DuplicateTensor, OverlappingTensors, MissingTensor,
    InvalidScaleShape (the first ten as model/safetensors/errors.mbt names
    them); index: the tensor's position in the header, when one applies."""

    def __init__(self, kind: str, index: int | None = None, detail: str = ""):
        super().__init__(f"{kind}" + (f" (tensor {index})" if index is not None else "")
                         + (f": {detail}" if detail else ""))
        self.kind = kind
        self.index = index


@dataclass(frozen=True)
class TensorMetadata:
    name: str
    dtype: str
    shape: tuple
    start: int  # payload-relative, half-open
    end: int


def _valid_name(name) -> bool:
    return (isinstance(name, str) and 0 < len(name) <= MAX_NAME_LENGTH
            and all(ord(c) < 128 and 32 <= ord(c) != 127 for c in name))


def read_metadata(path: str) -> tuple[dict, int]:
    """(name -> TensorMetadata, payload offset in the file) of a safetensors
    file, validated as above."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise SafetensorsError("InvalidHeader", detail="no header length")
        n = struct.unpack("<Q", head)[0]
        if n > MAX_HEADER_BYTES or 8 + n > size:
            raise SafetensorsError("HeaderTooLarge")
        try:
            header = json.loads(f.read(n).decode("utf-8"), object_pairs_hook=_no_duplicates)
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise SafetensorsError("InvalidHeader", detail=str(e)) from None
    if not isinstance(header, dict):
        raise SafetensorsError("InvalidHeader", detail="not an object")
    payload = size - 8 - n
    tensors = {}
    for index, (name, raw) in enumerate((k, v) for k, v in header.items() if k != "__metadata__"):
        if not _valid_name(name):
            raise SafetensorsError("InvalidTensorName", index)
        if not isinstance(raw, dict) or raw.get("dtype") not in ITEM_BYTES:
            raise SafetensorsError("InvalidDType", index)
        shape = raw.get("shape")
        if (not isinstance(shape, list) or not 0 < len(shape) <= MAX_RANK
                or any(not isinstance(d, int) or d < 0 for d in shape)):
            raise SafetensorsError("InvalidRank", index)
        offsets = raw.get("data_offsets")
        if (not isinstance(offsets, list) or len(offsets) != 2
                or any(not isinstance(o, int) for o in offsets)
                or offsets[0] < 0 or offsets[1] < offsets[0]):
            raise SafetensorsError("InvalidByteRange", index)
        if offsets[1] > payload:
            raise SafetensorsError("RangeOutsidePayload", index)
        if offsets[1] - offsets[0] != int(np.prod(shape, dtype=np.int64)) * ITEM_BYTES[raw["dtype"]]:
            raise SafetensorsError("RangeSizeMismatch", index)
        t = TensorMetadata(name, raw["dtype"], tuple(shape), offsets[0], offsets[1])
        for j, prev in enumerate(tensors.values()):
            if prev.start < t.end and t.start < prev.end:
                raise SafetensorsError("OverlappingTensors", index, f"with tensor {j}")
        tensors[name] = t
    return tensors, 8 + n


def _no_duplicates(pairs):
    seen = {}
    for i, (k, v) in enumerate(pairs):
        if k in seen:
            raise SafetensorsError("DuplicateTensor", i, k)
        seen[k] = v
    return seen


def load_tensor(path: str, tensors: dict, payload_offset: int, name: str) -> np.ndarray:
    """A tensor's values (memory-mapped, read-only): F8_E4M3 as uint8 codes,
    BF16 as uint16 bit patterns, F32 as float32."""
    t = tensors.get(name)
    if t is None:
        raise SafetensorsError("MissingTensor", detail=name)
    count = int(np.prod(t.shape, dtype=np.int64))
    if count == 0:
        return np.zeros(t.shape, NUMPY[t.dtype])
    return np.memmap(path, dtype=NUMPY[t.dtype], mode="r", offset=payload_offset + t.start,
                     shape=t.shape)


def load_fp8_linear(path: str, prefix: str):
    """(codes [N, K] uint8, scales, scale mode) of the FP8 projection weight
    `<prefix>.weight` and its scales, ready for fp8.pack_weight."""
    tensors, off = read_metadata(path)
    w = tensors.get(prefix + ".weight")
    if w is None:
        raise SafetensorsError("MissingTensor", detail=prefix + ".weight")
    if w.dtype != "F8_E4M3" or len(w.shape) != 2:
        raise SafetensorsError("InvalidDType", detail=f"{w.name}: {w.dtype} {w.shape}")
    n, k = w.shape
    q = np.ascontiguousarray(load_tensor(path, tensors, off, w.name))
    if prefix + ".weight_scale" in tensors:
        s = tensors[prefix + ".weight_scale"]
        if s.dtype != "F32" or int(np.prod(s.shape)) != n or s.shape[0] != n:
            raise SafetensorsError("InvalidScaleShape", detail=f"{s.name}: {s.dtype} {s.shape}")
        scales = np.array(load_tensor(path, tensors, off, s.name), np.float32).reshape(n)
        return q, scales, fp8.PER_CHANNEL
    if prefix + ".weight_scale_inv" in tensors:
        s = tensors[prefix + ".weight_scale_inv"]
        if s.dtype != "F32" or s.shape != ((n + 127) // 128, (k + 127) // 128):
            raise SafetensorsError("InvalidScaleShape", detail=f"{s.name}: {s.dtype} {s.shape}")
        scales = np.array(load_tensor(path, tensors, off, s.name), np.float32)
        return q, scales, fp8.BLOCK128
    raise SafetensorsError("MissingTensor", detail=prefix + ".weight_scale[_inv]")


def upload_linear(rt, path: str, prefix: str) -> "fp8.Fp8Weight":
    """Loads, pre-swizzles and uploads one FP8 projection weight."""
    q, scales, mode = load_fp8_linear(path, prefix)
    return rt.upload_weight(q, scales, mode)

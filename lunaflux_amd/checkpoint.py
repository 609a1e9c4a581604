"""FP8 checkpoint admission: safetensors files holding e4m3 weights.

LunaFlux admits a safetensors file in two passes, both restated here with
the same checks in the same order and the same error kinds:

* the byte reader (model/safetensors_reader/reader.mbt:217-306): the
  8-byte little-endian header length, its bounds, the header envelope
  (``{`` ... ``}`` then only spaces), UTF-8, duplicate object keys at any
  depth up to 4 (internal/json_guard/guard.mbt:18-33, 107-145), the root
  object, ``__metadata__`` (an object of strings), and per tensor exactly the
  fields dtype / shape / data_offsets with exactly integral numbers
  (reader.mbt:66-187);
* metadata validation (model/safetensors/metadata.mbt:63-175): name, dtype,
  rank, positive dimensions, size overflow, the half-open byte range inside
  the payload and of the shape's size, no duplicate name, no overlap, the
  materialized-size budget; then the payload must be exactly covered
  (reader.mbt:269-271).

The limits are HeaderLimits (model/safetensors/limits.mbt:3-55). The only
deliberate difference is the dtype gate (metadata.mbt:100-102 admits BF16
only): an FP8 checkpoint adds F8_E4M3 weight codes and their F32 scales. A
projection weight ``<prefix>.weight`` [N, K] F8_E4M3 comes with
``<prefix>.weight_scale`` (F32: N values, per output channel, or one value
for the whole tensor, which is broadcast to every channel exactly) or
``<prefix>.weight_scale_inv`` (F32 [N/128, K/128]: 128 x 128 blocks); the
dequantized weight is fp32(code) * scale in every case. Codes and scales are
checked for the values a kernel cannot carry (the reference rejects
non-finite weights at decode, kernels/reference/bfloat16.mbt:24-26): no e4m3
NaN code (0x7F, 0xFF), scales finite and not negative.

bind_llama_fp8 then binds a whole dense Llama checkpoint in the TensorRef
order model/llama_weights/bind.mbt:53-113 emits, with the reference's exact
tensor count (3 + 9 L tensors, plus here one scale tensor per FP8
projection), names and shapes.
"""
from __future__ import annotations

import json
import math
import os
import struct
from dataclasses import dataclass

import numpy as np

from . import fp8

ITEM_BYTES = {"F8_E4M3": 1, "BF16": 2, "F32": 4}
NUMPY = {"F8_E4M3": np.uint8, "BF16": np.uint16, "F32": np.float32}
PREFIX_BYTES = 8
MAX_INT = 2 ** 31 - 1
MAX_INT64 = 2 ** 63 - 1
JSON_MAX_DEPTH = 4  # reader.mbt:254


class SafetensorsError(ValueError):
    """kind: a variant of SafetensorsReaderError (reader errors.mbt:13-34) or
    SafetensorsError (model/safetensors/errors.mbt:15-31), plus the FP8
    admission kinds MissingTensor, InvalidScaleShape, NonFiniteWeight and
    InvalidScale. index: the tensor's position among the header's tensors
    (``__metadata__`` excluded), when one applies; other: the earlier tensor
    of a DuplicateTensor / OverlappingTensors pair, or (depth, key index) of a
    DuplicateHeaderKey; field: DType, Shape or DataOffsets where the
    reference names one."""

    def __init__(self, kind: str, index: int | None = None, detail: str = "", other=None,
                 field: str | None = None):
        text = kind + (f" (tensor {index})" if index is not None else "")
        text += f" [{field}]" if field else ""
        text += f" with {other}" if other is not None else ""
        super().__init__(text + (f": {detail}" if detail else ""))
        self.kind = kind
        self.index = index
        self.other = other
        self.field = field


@dataclass(frozen=True)
class HeaderLimits:
    """model/safetensors/limits.mbt:3-55; the defaults are the worker
    recipe's header, rank and name bounds (engine/device_worker_bootstrap/
    recipe.mbt:5-20) and a 1 TiB payload."""

    max_header_bytes: int = 16 << 20
    max_tensor_count: int = 1 << 16
    max_rank: int = 2
    max_name_length: int = 256
    max_payload_bytes: int = 1 << 40
    max_materialized_tensor_bytes: int = 1 << 40

    def __post_init__(self):
        checks = [(self.max_header_bytes > 0, "HeaderBytes"),
                  (self.max_tensor_count > 0, "TensorCount"),
                  (self.max_rank > 0, "TensorRank"),
                  (self.max_name_length > 0, "TensorNameLength"),
                  (self.max_payload_bytes > 0, "PayloadBytes"),
                  (0 < self.max_materialized_tensor_bytes <= self.max_payload_bytes,
                   "MaterializedTensorBytes")]
        for ok, limit in checks:
            if not ok:
                raise SafetensorsError("InvalidLimit", detail=limit)


@dataclass(frozen=True)
class TensorMetadata:
    name: str
    dtype: str
    shape: tuple
    start: int  # payload-relative, half-open
    end: int


# -- the byte reader --------------------------------------------------------
def _envelope_ok(header: bytes) -> bool:
    """reader.mbt:45-59: starts with '{', ends with '}' and ASCII spaces."""
    if not header or header[0] != ord("{"):
        return False
    stripped = header.rstrip(b" ")
    return len(stripped) > 0 and stripped[-1] == ord("}")


class _Pairs(list):
    """An object's (key, value) pairs in document order, duplicates kept."""


def _duplicate_keys(value, depth: int):
    """internal/json_guard/guard.mbt:107-145 over the parsed tree: keys are
    checked in document order, each before its value is scanned; objects
    and arrays nest one level deeper than their container (the root object
    is depth 1); deeper than JSON_MAX_DEPTH is malformed for the reader."""
    if isinstance(value, _Pairs):
        depth += 1
        if depth > JSON_MAX_DEPTH:
            raise SafetensorsError("InvalidHeaderJson", detail="nesting deeper than 4")
        seen = set()
        for index, (key, item) in enumerate(value):
            if key in seen:
                raise SafetensorsError("DuplicateHeaderKey", other=(depth, index))
            seen.add(key)
            _duplicate_keys(item, depth)
    elif isinstance(value, list):
        depth += 1
        if depth > JSON_MAX_DEPTH:
            raise SafetensorsError("InvalidHeaderJson", detail="nesting deeper than 4")
        for item in value:
            _duplicate_keys(item, depth)


def _no_constant(name):
    """NaN, Infinity and -Infinity are not JSON."""
    raise ValueError(f"{name} is not JSON")


def _exact_int64(value, index: int, field: str) -> int:
    """reader.mbt:66-93: a JSON number with an exactly integral value in the
    int64 range (1.0 and 1e0 are accepted; fractions, booleans, strings and
    out-of-range values are not)."""
    if isinstance(value, bool) or not isinstance(value, (int, float)):
        raise SafetensorsError("InvalidInteger", index, field=field)
    if isinstance(value, float):
        if math.isnan(value) or math.isinf(value) or value != math.floor(value):
            raise SafetensorsError("InvalidInteger", index, field=field)
        if not -2.0 ** 63 <= value < 2.0 ** 63:
            raise SafetensorsError("InvalidInteger", index, field=field)
        value = int(value)
    if not -2 ** 63 <= value <= MAX_INT64:
        raise SafetensorsError("InvalidInteger", index, field=field)
    return value


def _decode_tensor(name, value, index: int, limits: HeaderLimits) -> tuple:
    """reader.mbt:153-187."""
    if not isinstance(value, _Pairs):
        raise SafetensorsError("InvalidTensor", index)
    fields = dict(value)
    for key, _ in value:
        if key not in ("dtype", "shape", "data_offsets"):
            raise SafetensorsError("UnexpectedTensorField", index)
    if "dtype" not in fields:
        raise SafetensorsError("MissingTensorField", index, field="DType")
    dtype = fields["dtype"]
    if not isinstance(dtype, str):
        raise SafetensorsError("InvalidTensorField", index, field="DType")
    if "shape" not in fields:
        raise SafetensorsError("MissingTensorField", index, field="Shape")
    shape = fields["shape"]
    if not isinstance(shape, list):
        raise SafetensorsError("InvalidTensorField", index, field="Shape")
    if len(shape) > limits.max_rank:
        raise SafetensorsError("InvalidRank", index)
    shape = [_exact_int64(d, index, "Shape") for d in shape]
    if "data_offsets" not in fields:
        raise SafetensorsError("MissingTensorField", index, field="DataOffsets")
    offsets = fields["data_offsets"]
    if not isinstance(offsets, list) or len(offsets) != 2:
        raise SafetensorsError("InvalidTensorField", index, field="DataOffsets")
    start = _exact_int64(offsets[0], index, "DataOffsets")
    end = _exact_int64(offsets[1], index, "DataOffsets")
    return name, dtype, shape, start, end


def _decode_entries(root, limits: HeaderLimits) -> list:
    """reader.mbt:190-209."""
    if not isinstance(root, _Pairs):
        raise SafetensorsError("InvalidRoot")
    entries = []
    for name, value in root:
        if name == "__metadata__":
            if not isinstance(value, _Pairs) or not all(isinstance(v, str) for _, v in value):
                raise SafetensorsError("InvalidMetadata")
            continue
        if len(entries) >= limits.max_tensor_count:
            raise SafetensorsError("TooManyTensors")
        entries.append(_decode_tensor(name, value, len(entries), limits))
    return entries


# -- metadata validation ----------------------------------------------------
def _valid_name(name: str, max_length: int) -> bool:
    """metadata.mbt:54-60 (MoonBit string length counts UTF-16 units; the
    name must be ASCII, where both counts agree)."""
    return (0 < len(name) <= max_length
            and all(ord(c) < 128 and not (ord(c) < 32 or ord(c) == 127) for c in name))


def _checked_bytes(shape, dtype: str, index: int, max_rank: int) -> int:
    """metadata.mbt:63-86 with the item size of the admitted dtype."""
    if not shape or len(shape) > max_rank:
        raise SafetensorsError("InvalidRank", index)
    elements = 1
    for d in shape:
        if d <= 0:
            raise SafetensorsError("InvalidDimension", index)
        if elements > MAX_INT64 // d:
            raise SafetensorsError("TensorSizeOverflow", index)
        elements *= d
    item = ITEM_BYTES[dtype]
    if elements > MAX_INT64 // item:
        raise SafetensorsError("TensorSizeOverflow", index)
    return elements * item


def validate_metadata(entries, header_bytes: int, payload_bytes: int,
                      limits: HeaderLimits) -> list:
    """metadata.mbt:125-175 over decoded entries (name, dtype, shape,
    start, end)."""
    if header_bytes < 0 or header_bytes > limits.max_header_bytes:
        raise SafetensorsError("HeaderTooLarge")
    if len(entries) > limits.max_tensor_count:
        raise SafetensorsError("TooManyTensors")
    if payload_bytes < 0 or payload_bytes > limits.max_payload_bytes:
        raise SafetensorsError("RangeOutsidePayload", 0)
    validated, total = [], 0
    for index, (name, dtype, shape, start, end) in enumerate(entries):
        if not _valid_name(name, limits.max_name_length):
            raise SafetensorsError("InvalidTensorName", index)
        if dtype not in ITEM_BYTES:
            raise SafetensorsError("InvalidDType", index)
        nbytes = _checked_bytes(shape, dtype, index, limits.max_rank)
        if start < 0 or end < start:
            raise SafetensorsError("InvalidByteRange", index)
        if end > payload_bytes:
            raise SafetensorsError("RangeOutsidePayload", index)
        if end - start != nbytes:
            raise SafetensorsError("RangeSizeMismatch", index)
        t = TensorMetadata(name, dtype, tuple(shape), start, end)
        for j, prev in enumerate(validated):
            if prev.name == t.name:
                raise SafetensorsError("DuplicateTensor", index, other=j)
            if prev.start < t.end and t.start < prev.end:
                raise SafetensorsError("OverlappingTensors", index, other=j)
        if nbytes > limits.max_materialized_tensor_bytes - total:
            raise SafetensorsError("MaterializedSizeExceeded")
        total += nbytes
        validated.append(t)
    return validated


def read_metadata(path: str, limits: HeaderLimits | None = None) -> tuple[dict, int]:
    """(name -> TensorMetadata in header order, payload offset in the file)
    of a safetensors file, admitted as reader.mbt:284-306 admits a whole
    file."""
    limits = limits or HeaderLimits()
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        prefix = f.read(PREFIX_BYTES)
        if len(prefix) < PREFIX_BYTES:
            raise SafetensorsError("MissingHeaderLength")
        n = struct.unpack("<Q", prefix)[0]
        if n > MAX_INT:
            raise SafetensorsError("HeaderLengthOverflow")
        if n > limits.max_header_bytes:
            raise SafetensorsError("HeaderTooLarge")
        if n > size - PREFIX_BYTES:
            raise SafetensorsError("TruncatedHeader")
        header = f.read(n)
    payload = size - PREFIX_BYTES - n
    if payload > limits.max_payload_bytes:
        raise SafetensorsError("RangeOutsidePayload", 0)
    if not _envelope_ok(header):
        raise SafetensorsError("InvalidHeaderEnvelope")
    try:
        text = header.decode("utf-8")
    except UnicodeDecodeError:
        raise SafetensorsError("InvalidHeaderEncoding") from None
    # The reference scans for duplicate keys before it parses; a header that
    # is malformed and also repeats a key is reported here as
    # InvalidHeaderJson rather than DuplicateHeaderKey.
    try:
        root = json.loads(text, object_pairs_hook=_Pairs, parse_constant=_no_constant)
    except (json.JSONDecodeError, RecursionError, ValueError) as e:
        raise SafetensorsError("InvalidHeaderJson", detail=str(e)) from None
    _duplicate_keys(root, 0)
    entries = _decode_entries(root, limits)
    tensors = validate_metadata(entries, n, payload, limits)
    if sum(t.end - t.start for t in tensors) != payload:
        raise SafetensorsError("PayloadSizeMismatch")
    return {t.name: t for t in tensors}, PREFIX_BYTES + n


def load_tensor(path: str, tensors: dict, payload_offset: int, name: str) -> np.ndarray:
    """A tensor's values (memory-mapped, read-only): F8_E4M3 as uint8 codes,
    BF16 as uint16 bit patterns, F32 as float32."""
    t = tensors.get(name)
    if t is None:
        raise SafetensorsError("MissingTensor", detail=name)
    return np.memmap(path, dtype=NUMPY[t.dtype], mode="r", offset=payload_offset + t.start,
                     shape=t.shape)


# -- FP8 projection weights --------------------------------------------------
def _fp8_linear(path, tensors, off, prefix, rows=None, columns=None):
    """Codes and scales of `<prefix>.weight` (F8_E4M3 [N, K], no NaN code)
    with `<prefix>.weight_scale`: F32, N values (one per output channel) or
    a single value for the whole tensor held as a rank-1 or rank-2 tensor of
    one element, broadcast to every channel; or `<prefix>.weight_scale_inv`:
    F32 [ceil(N / 128), ceil(K / 128)] (128 x 128 blocks). A rank-0 scale
    tensor never gets here: the metadata validation rejects every rank-0
    tensor with InvalidRank, as the reference's does (metadata.mbt:63-86;
    such files need their scalars stored as shape [1]). Scales must be
    finite and not negative."""
    w = tensors.get(prefix + ".weight")
    if w is None:
        raise SafetensorsError("MissingTensor", detail=prefix + ".weight")
    if w.dtype != "F8_E4M3" or len(w.shape) != 2:
        raise SafetensorsError("InvalidDType", detail=f"{w.name}: {w.dtype} {w.shape}")
    n, k = w.shape
    if (rows is not None and n != rows) or (columns is not None and k != columns):
        raise SafetensorsError("ShapeDimensionMismatch", detail=f"{w.name}: {w.shape}")
    q = np.ascontiguousarray(load_tensor(path, tensors, off, w.name))
    if np.any((q & 0x7F) == 0x7F):
        raise SafetensorsError("NonFiniteWeight", detail=f"{w.name}: e4m3 NaN code")
    if prefix + ".weight_scale" in tensors:
        s = tensors[prefix + ".weight_scale"]
        count = int(np.prod(s.shape))
        per_tensor = count == 1 and len(s.shape) <= 2
        per_channel = count == n and s.shape[0] == n
        if s.dtype != "F32" or not (per_tensor or per_channel):
            raise SafetensorsError("InvalidScaleShape", detail=f"{s.name}: {s.dtype} {s.shape}")
        scales = np.array(load_tensor(path, tensors, off, s.name), np.float32).reshape(-1)
        scales = np.broadcast_to(scales, (n,)).copy()
        mode = fp8.PER_CHANNEL
    elif prefix + ".weight_scale_inv" in tensors:
        s = tensors[prefix + ".weight_scale_inv"]
        if s.dtype != "F32" or s.shape != ((n + 127) // 128, (k + 127) // 128):
            raise SafetensorsError("InvalidScaleShape", detail=f"{s.name}: {s.dtype} {s.shape}")
        scales = np.array(load_tensor(path, tensors, off, s.name), np.float32)
        mode = fp8.BLOCK128
    else:
        raise SafetensorsError("MissingTensor", detail=prefix + ".weight_scale[_inv]")
    if not np.all(np.isfinite(scales)) or np.any(scales < 0):
        raise SafetensorsError("InvalidScale", detail=f"{s.name}: non-finite or negative")
    return q, scales, mode


def load_fp8_linear(path: str, prefix: str, limits: HeaderLimits | None = None):
    """(codes [N, K] uint8, scales, scale mode) of the FP8 projection weight
    `<prefix>.weight` and its scales, ready for fp8.pack_weight."""
    tensors, off = read_metadata(path, limits)
    return _fp8_linear(path, tensors, off, prefix)


def upload_linear(rt, path: str, prefix: str) -> "fp8.Fp8Weight":
    """Loads, pre-swizzles and uploads one FP8 projection weight."""
    q, scales, mode = load_fp8_linear(path, prefix)
    return rt.upload_weight(q, scales, mode)


# -- a whole dense Llama checkpoint -------------------------------------------
@dataclass(frozen=True)
class LlamaShape:
    """The dimensions model/llama_weights/bind.mbt:53-113 binds against
    (LlamaModelSpec, model/spec/llama.mbt:66-117)."""

    vocabulary: int
    hidden: int
    intermediate: int
    layers: int
    attention_heads: int
    kv_heads: int

    @property
    def kv_width(self) -> int:
        return self.kv_heads * (self.hidden // self.attention_heads)


class LlamaWeightsError(ValueError):
    """kind: TensorCountMismatch, MissingTensor, ShapeRankMismatch,
    ShapeDimensionMismatch (model/llama_weights/errors), or
    UnsupportedWeightDType; reference: the TensorRef index."""

    def __init__(self, kind: str, reference: int | None = None, detail: str = ""):
        super().__init__(kind + (f" (reference {reference})" if reference is not None else "")
                         + (f": {detail}" if detail else ""))
        self.kind = kind
        self.reference = reference


PROJECTIONS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
               "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


@dataclass(frozen=True)
class TensorBinding:
    """One TensorRef: a BF16 tensor, or an FP8 projection (codes + scales)
    whose region is the packed weight format."""

    reference: int
    name: str
    dtype: str          # "BF16" or "F8_E4M3"
    shape: tuple
    scale_name: str | None = None


def bind_llama_fp8(shape: LlamaShape, tensors: dict) -> list:
    """TensorRef bindings of an FP8 Llama checkpoint, in the order
    model/llama_weights/bind.mbt:53-113 emits (embedding; per layer input
    norm, q, k, v, o, post-attention norm, gate, up, down; final norm; LM
    head). Projections are F8_E4M3 with one scale tensor each; norms and the
    embedding stay BF16; the LM head may be either. The header must hold
    exactly these tensors: the count is checked first, as the reference's
    exact count is (bind.mbt:57-63), then each tensor in TensorRef order."""
    h, i, v, kv = shape.hidden, shape.intermediate, shape.vocabulary, shape.kv_width
    plan = [("model.embed_tokens.weight", (v, h), "BF16")]
    for layer in range(shape.layers):
        p = f"model.layers.{layer}"
        plan += [(f"{p}.input_layernorm.weight", (h,), "BF16"),
                 (f"{p}.self_attn.q_proj.weight", (h, h), "F8_E4M3"),
                 (f"{p}.self_attn.k_proj.weight", (kv, h), "F8_E4M3"),
                 (f"{p}.self_attn.v_proj.weight", (kv, h), "F8_E4M3"),
                 (f"{p}.self_attn.o_proj.weight", (h, h), "F8_E4M3"),
                 (f"{p}.post_attention_layernorm.weight", (h,), "BF16"),
                 (f"{p}.mlp.gate_proj.weight", (i, h), "F8_E4M3"),
                 (f"{p}.mlp.up_proj.weight", (i, h), "F8_E4M3"),
                 (f"{p}.mlp.down_proj.weight", (h, i), "F8_E4M3")]
    plan += [("model.norm.weight", (h,), "BF16"), ("lm_head.weight", (v, h), None)]
    # The count first, as bind.mbt:57-63 does before any per-tensor check:
    # 3 + 9 L tensors of the dense vocabulary plus one scale tensor per FP8
    # projection (7 L, and the LM head when it is F8_E4M3). A file holding
    # anything else (e.g. per-projection input_scale tensors) fails here.
    head = tensors.get("lm_head.weight")
    expected = 3 + 9 * shape.layers + 7 * shape.layers + (
        1 if head is not None and head.dtype == "F8_E4M3" else 0)
    if len(tensors) != expected:
        raise LlamaWeightsError("TensorCountMismatch",
                                detail=f"expected {expected}, found {len(tensors)}")
    bindings = []
    for name, dims, dtype in plan:
        ref = len(bindings)
        t = tensors.get(name)
        if t is None:
            raise LlamaWeightsError("MissingTensor", ref, name)
        if len(t.shape) != len(dims):
            raise LlamaWeightsError("ShapeRankMismatch", ref, name)
        for axis, d in enumerate(dims):
            if t.shape[axis] != d:
                raise LlamaWeightsError("ShapeDimensionMismatch", ref, f"{name} axis {axis}")
        want = dtype or t.dtype
        if t.dtype != want or want not in ("BF16", "F8_E4M3"):
            raise LlamaWeightsError("UnsupportedWeightDType", ref, f"{name}: {t.dtype}")
        scale = None
        if want == "F8_E4M3":
            base = name[:-len(".weight")]
            for suffix in (".weight_scale", ".weight_scale_inv"):
                if base + suffix in tensors:
                    scale = base + suffix
            if scale is None:
                raise LlamaWeightsError("MissingTensor", ref, base + ".weight_scale[_inv]")
        bindings.append(TensorBinding(ref, name, want, tuple(dims), scale))
    return bindings


def materialize_llama_fp8(rt, path: str, shape: LlamaShape,
                          limits: HeaderLimits | None = None) -> list:
    """Admits the file, binds it, and uploads one device region per
    TensorRef (model/device_materialize/layout.mbt:37-93 places them in this
    order): FP8 projections pre-swizzled into the packed weight format
    (fp8.Fp8Weight), BF16 tensors as they are (device Allocation)."""
    tensors, off = read_metadata(path, limits)
    out = []
    for b in bind_llama_fp8(shape, tensors):
        if b.dtype == "F8_E4M3":
            q, s, mode = _fp8_linear(path, tensors, off, b.name[:-len(".weight")], *b.shape)
            out.append(rt.upload_weight(q, s, mode))
        else:
            out.append(rt.context.upload(np.ascontiguousarray(
                load_tensor(path, tensors, off, b.name))))
    return out

"""The kernel artifact manifest for the gfx950 code object.

LunaFlux admits AOT kernels through a digest-pinned JSON manifest, schema
v1 (kernels/artifact_file/reader.mbt:2-40): exactly the root fields
schema_version, model_identity {content_sha256, plan_sha256}, device_target
{compute_major, compute_minor, supports_bf16, supports_cublas_lt},
catalog_version and modules [{sha256, path, entry_points [{family_id,
entry_point_id, symbol}]}] (schema_identity.mbt:1-115,
schema_modules.mbt:1-153), no unknown, missing or duplicate field at any
object (schema_fields.mbt:12-36, internal/json_guard), relative lexical
paths (path.mbt:1-40), bounded ASCII identifier symbols
(kernels/artifact/admit.mbt:56-92), and module bytes whose SHA-256 is the
declared digest (admit.mbt:94-96, 255-302).

write_manifest() describes lunaflux_fp8.hsaco in that schema: device target
{9, 5, true, false} (gfx950; no vendor GEMM), one module, one entry point per
kernel symbol of the code object, grouped into stable families (one catalog
AotKernelFamily per family of include/lunaflux_fp8.h). admit_manifest()
applies the reference's checks, in its order, to a manifest text and the
module bytes, raising ManifestError with the reference's error kinds.
"""
from __future__ import annotations

import hashlib
import json
import os
import re

PACKAGE = os.path.dirname(os.path.abspath(__file__))
CODE_OBJECT = "lunaflux_fp8.hsaco"
MANIFEST = "lunaflux_fp8.manifest.json"
SCHEMA_VERSION = 1
CATALOG_VERSION = 1
DEVICE_TARGET = {"compute_major": 9, "compute_minor": 5, "supports_bf16": True,
                 "supports_cublas_lt": False}
# kernels/artifact_file/limits.mbt and kernels/artifact/limits.mbt bounds
MAX_MANIFEST_BYTES = 1 << 20
MAX_JSON_DEPTH = 8
MAX_PATH_BYTES = 4096
MAX_MODULES = 16
MAX_ENTRY_POINTS = 4096
MAX_MODULE_BYTES = 1 << 30
MAX_SYMBOL_BYTES = 128  # the C ABI's bound (include/lunaflux_hip.h)

# Stable family ids (the integer a catalog AotKernelFamily names within the
# module), by symbol prefix and suffix; first match wins. The one-launch W8A8
# forms (_aq: x and a workspace in place of the quantized rows) are families
# of their own, since their operand lists differ.
FAMILIES = (
    # block-scaled forms first: their symbols share the per-channel prefixes
    (15, "lf_fp8_w8a16_dense_b128_"),
    (16, "lf_fp8_w8a16_qkv_b128_"),
    (17, "lf_fp8_w8a16_gate_up_b128_"),
    (18, "lf_fp8_w8a8_dense_b128"),
    (19, "lf_fp8_w8a8_qkv_b128"),
    (20, "lf_fp8_w8a8_gate_up_b128"),
    (21, "lf_fp8_w8a8_gated_mlp_b128"),
    (22, "lf_fp8_w8a16_gated_mlp_b128"),
    (12, "lf_fp8_w8a8_dense_", "_aq"),
    (13, "lf_fp8_w8a8_qkv_", "_aq"),
    (14, "lf_fp8_w8a8_gate_up_", "_aq"),
    (1, "lf_fp8_act_quant_rows"),
    (2, "lf_fp8_rms_norm_quant_rows_"),
    (3, "lf_fp8_w8a16_dense_"),
    (4, "lf_fp8_w8a16_qkv_"),
    (5, "lf_fp8_w8a16_gate_up_"),
    (6, "lf_fp8_w8a8_dense_"),
    (7, "lf_fp8_w8a8_qkv_"),
    (8, "lf_fp8_w8a8_gate_up_"),
    (9, "lf_moe_"),
    (10, "lf_fp8_w8a16_gated_mlp_"),
    (11, "lf_fp8_w8a8_gated_mlp_"),
)


class ManifestError(ValueError):
    """kind: a KernelArtifactFileError / KernelArtifactError variant
    (FileTooLarge, InvalidUtf8, MalformedJson, JsonDepthExceeded,
    DuplicateField, UnknownField, MissingField, InvalidField, IdentityMismatch,
    InvalidPath, InvalidFunctionSymbol, DuplicateModule, DuplicateEntryPoint,
    MissingModule, DigestMismatch, ModuleTooLarge); detail names the field,
    rule or identity."""

    def __init__(self, kind: str, detail: str = ""):
        super().__init__(kind + (f": {detail}" if detail else ""))
        self.kind = kind
        self.detail = detail


def kernel_symbols(image: bytes) -> list:
    """Kernel entry points of a code object we built: each kernel has a
    kernel-descriptor symbol `<name>.kd` in the ELF string table."""
    names = {m.group(1).decode("ascii") for m in re.finditer(rb"\x00([A-Za-z_][A-Za-z0-9_]*)\.kd\x00", image)}
    return sorted(n for n in names if family_of(n) is not None)


def family_of(symbol: str):
    for family, prefix, *suffix in FAMILIES:
        if symbol.startswith(prefix) and (not suffix or symbol.endswith(suffix[0])):
            return family
    return None


def build_manifest(image: bytes, content_sha256: str, plan_sha256: str,
                   path: str = CODE_OBJECT) -> dict:
    """The v1 manifest document for one code object and one model identity."""
    entries = []
    counters = {}
    for symbol in kernel_symbols(image):
        family = family_of(symbol)
        counters[family] = counters.get(family, 0) + 1
        entries.append({"family_id": family, "entry_point_id": counters[family], "symbol": symbol})
    return {
        "schema_version": SCHEMA_VERSION,
        "model_identity": {"content_sha256": content_sha256, "plan_sha256": plan_sha256},
        "device_target": dict(DEVICE_TARGET),
        "catalog_version": CATALOG_VERSION,
        "modules": [{"sha256": hashlib.sha256(image).hexdigest(), "path": path,
                     "entry_points": entries}],
    }


def write_manifest(content_sha256: str = "0" * 64, plan_sha256: str = "0" * 64,
                   directory: str = PACKAGE) -> str:
    """Writes lunaflux_fp8.manifest.json beside the built code object (the
    model identity defaults to a placeholder: the engine writes its own)."""
    with open(os.path.join(directory, CODE_OBJECT), "rb") as f:
        image = f.read()
    doc = build_manifest(image, content_sha256, plan_sha256)
    out = os.path.join(directory, MANIFEST)
    with open(out + ".tmp", "w") as f:
        json.dump(doc, f, indent=1)
        f.write("\n")
    os.replace(out + ".tmp", out)
    return out


# -- admission --------------------------------------------------------------
class _Pairs(list):
    pass


def _guard(value, depth):
    """internal/json_guard: duplicate keys by (depth, index), depth bound."""
    if isinstance(value, (_Pairs, list)):
        depth += 1
        if depth > MAX_JSON_DEPTH:
            raise ManifestError("JsonDepthExceeded", str(MAX_JSON_DEPTH))
    if isinstance(value, _Pairs):
        seen = set()
        for index, (key, item) in enumerate(value):
            if key in seen:
                raise ManifestError("DuplicateField", f"depth {depth}, index {index}")
            seen.add(key)
            _guard(item, depth)
    elif isinstance(value, list):
        for item in value:
            _guard(item, depth)


def _fields(obj, area, allowed):
    """schema_fields.mbt:12-36: unknown fields first (by position), then
    missing ones (in declaration order)."""
    if not isinstance(obj, _Pairs):
        raise ManifestError("InvalidField", f"{area}: expected object")
    for index, (name, _) in enumerate(obj):
        if name not in allowed:
            raise ManifestError("UnknownField", f"{area} index {index}")
    names = {k for k, _ in obj}
    for name in allowed:
        if name not in names:
            raise ManifestError("MissingField", f"{area}.{name}")
    return dict(obj)


def _nonnegative_int(value, where):
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ManifestError("InvalidField", f"{where}: expected a non-negative integer")
    return value


def _string(value, where):
    if not isinstance(value, str):
        raise ManifestError("InvalidField", f"{where}: expected a string")
    return value


def _lower_sha256(text):
    return len(text) == 64 and all(c in "0123456789abcdef" for c in text)


def validate_path(value: str, maximum: int = MAX_PATH_BYTES):
    """kernels/artifact_file/path.mbt:1-40."""
    if not value:
        raise ManifestError("InvalidPath", "EmptyPath")
    if len(value) > maximum:
        raise ManifestError("InvalidPath", "PathTooLong")
    if value[0] in "/\\":
        raise ManifestError("InvalidPath", "AbsolutePath")
    for segment in value.split("/"):
        if segment == "" or segment in (".", ".."):
            raise ManifestError("InvalidPath", "TraversalSegment")
        if not all(c.isascii() and (c.isalnum() or c in "_-.") for c in segment):
            raise ManifestError("InvalidPath", "InvalidPathCharacter")


def validate_symbol(symbol: str, maximum: int = MAX_SYMBOL_BYTES):
    """kernels/artifact/admit.mbt:56-92."""
    if not symbol:
        raise ManifestError("InvalidFunctionSymbol", "Empty")
    if len(symbol) > maximum:
        raise ManifestError("InvalidFunctionSymbol", "TooLong")
    for index, c in enumerate(symbol):
        if ord(c) > 127:
            raise ManifestError("InvalidFunctionSymbol", "NonAscii")
        initial = c.isalpha() or c == "_"
        if index == 0 and not initial:
            raise ManifestError("InvalidFunctionSymbol", "InvalidInitial")
        if index > 0 and not (initial or c.isdigit()):
            raise ManifestError("InvalidFunctionSymbol", "InvalidContinuation")


def admit_manifest(text: bytes, modules: dict, content_sha256: str, plan_sha256: str,
                   device_target: dict = None, catalog_version: int = CATALOG_VERSION) -> list:
    """Admits a manifest against the expected identities and the module files
    (path -> bytes): the reference's read_manifest (reader.mbt:2-40, 70-91)
    then module admission (digest of the bytes, admit.mbt:255-302). Returns
    [(family_id, entry_point_id, symbol, module path)]."""
    device_target = DEVICE_TARGET if device_target is None else device_target
    if len(text) > MAX_MANIFEST_BYTES:
        raise ManifestError("FileTooLarge", "manifest")
    try:
        doc_text = text.decode("utf-8")
    except UnicodeDecodeError:
        raise ManifestError("InvalidUtf8") from None
    try:
        root = json.loads(doc_text, object_pairs_hook=_Pairs,
                          parse_constant=lambda c: (_ for _ in ()).throw(ValueError(c)))
    except (ValueError, RecursionError):
        raise ManifestError("MalformedJson") from None
    _guard(root, 0)
    if not isinstance(root, _Pairs):
        raise ManifestError("MalformedJson")
    r = _fields(root, "ManifestRoot", ("schema_version", "model_identity", "device_target",
                                       "catalog_version", "modules"))
    if _nonnegative_int(r["schema_version"], "schema_version") != SCHEMA_VERSION:
        raise ManifestError("InvalidField", "schema_version: UnsupportedValue")
    ident = _fields(r["model_identity"], "ManifestModelIdentity", ("content_sha256", "plan_sha256"))
    content = _string(ident["content_sha256"], "content_sha256")
    plan = _string(ident["plan_sha256"], "plan_sha256")
    if not _lower_sha256(content):
        raise ManifestError("InvalidField", "content_sha256: InvalidSha256")
    if not _lower_sha256(plan):
        raise ManifestError("InvalidField", "plan_sha256: InvalidSha256")
    if content != content_sha256:
        raise ManifestError("IdentityMismatch", "ModelContentIdentity")
    if plan != plan_sha256:
        raise ManifestError("IdentityMismatch", "ModelPlanIdentity")
    target = _fields(r["device_target"], "ManifestDeviceTarget",
                     ("compute_major", "compute_minor", "supports_bf16", "supports_cublas_lt"))
    for name, mismatch in (("compute_major", "DeviceComputeMajor"),
                           ("compute_minor", "DeviceComputeMinor")):
        if _nonnegative_int(target[name], name) != device_target[name]:
            raise ManifestError("IdentityMismatch", mismatch)
    for name, mismatch in (("supports_bf16", "DeviceBf16Support"),
                           ("supports_cublas_lt", "DeviceCublasLtSupport")):
        if not isinstance(target[name], bool):
            raise ManifestError("InvalidField", f"{name}: expected a boolean")
        if target[name] != device_target[name]:
            raise ManifestError("IdentityMismatch", mismatch)
    if _nonnegative_int(r["catalog_version"], "catalog_version") != catalog_version:
        raise ManifestError("IdentityMismatch", "KernelCatalogVersion")
    module_values = r["modules"]
    if not isinstance(module_values, list):
        raise ManifestError("InvalidField", "modules: expected an array")
    if len(module_values) > MAX_MODULES:
        raise ManifestError("InvalidField", "modules: CountExceeded")
    admitted, seen_digests, seen_entries = [], set(), set()
    for index, value in enumerate(module_values):
        m = _fields(value, f"ManifestModule {index}", ("sha256", "path", "entry_points"))
        digest = _string(m["sha256"], "sha256")
        if not _lower_sha256(digest):
            raise ManifestError("InvalidField", f"module {index} sha256: InvalidSha256")
        path = _string(m["path"], "path")
        validate_path(path)
        entries = m["entry_points"]
        if not isinstance(entries, list):
            raise ManifestError("InvalidField", "entry_points: expected an array")
        if len(entries) > MAX_ENTRY_POINTS - len(admitted):
            raise ManifestError("InvalidField", "entry_points: CountExceeded")
        if digest in seen_digests:
            raise ManifestError("DuplicateModule", digest)
        seen_digests.add(digest)
        for e_index, e_value in enumerate(entries):
            e = _fields(e_value, f"ManifestEntryPoint {e_index}",
                        ("family_id", "entry_point_id", "symbol"))
            family = _nonnegative_int(e["family_id"], "family_id")
            entry_id = _nonnegative_int(e["entry_point_id"], "entry_point_id")
            symbol = _string(e["symbol"], "symbol")
            validate_symbol(symbol)
            key = (digest, family, entry_id)
            if key in seen_entries:
                raise ManifestError("DuplicateEntryPoint", f"family {family} entry {entry_id}")
            seen_entries.add(key)
            admitted.append((family, entry_id, symbol, path))
        image = modules.get(path)
        if image is None:
            raise ManifestError("MissingModule", path)
        if len(image) > MAX_MODULE_BYTES:
            raise ManifestError("ModuleTooLarge", path)
        if hashlib.sha256(image).hexdigest() != digest:
            raise ManifestError("DigestMismatch", path)
        present = set(kernel_symbols(image))
        for family, entry_id, symbol, p in admitted:
            if p == path and symbol not in present:
                raise ManifestError("InvalidFunctionSymbol", f"{symbol}: not in {path}")
    return admitted


if __name__ == "__main__":
    print(write_manifest())

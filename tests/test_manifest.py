"""The v1 kernel artifact manifest of the gfx950 code object
(lunaflux_amd/manifest.py), checked by the rules of
kernels/artifact_file/reader.mbt:2-40, schema_identity.mbt:1-115,
schema_modules.mbt:79-153, path.mbt:1-40 and kernels/artifact/admit.mbt:56-92
(symbols) and 255-302 (module digests). CPU only."""
import hashlib
import json
import os

import pytest

from lunaflux_amd import _abi, manifest

CONTENT, PLAN = "ab" * 32, "cd" * 32


@pytest.fixture(scope="module")
def image():
    return _abi.code_object_bytes()


def doc(image):
    return manifest.build_manifest(image, CONTENT, PLAN)


def admit(d, image, **kw):
    text = json.dumps(d).encode() if isinstance(d, dict) else d
    return manifest.admit_manifest(text, {manifest.CODE_OBJECT: image}, CONTENT, PLAN, **kw)


def test_manifest_describes_every_kernel_of_the_code_object(image):
    d = doc(image)
    assert d["schema_version"] == 1 and d["catalog_version"] == 1
    assert d["device_target"] == {"compute_major": 9, "compute_minor": 5, "supports_bf16": True,
                                  "supports_cublas_lt": False}
    (module,) = d["modules"]
    assert module["sha256"] == hashlib.sha256(image).hexdigest()
    symbols = {e["symbol"]: (e["family_id"], e["entry_point_id"]) for e in module["entry_points"]}
    for name, family in [("lf_fp8_act_quant_rows", 1), ("lf_fp8_rms_norm_quant_rows_eps1em5", 2),
                         ("lf_fp8_w8a16_gate_up_k4096_m32", 5), ("lf_fp8_w8a16_dense_m128", 3),
                         ("lf_fp8_w8a16_qkv_k4096_q4096_kv1024_m32", 4),
                         ("lf_fp8_w8a8_dense_t256", 6), ("lf_fp8_w8a8_gate_up_t128", 8),
                         ("lf_moe_route", 9), ("lf_moe_down_t256_b128", 9),
                         ("lf_fp8_w8a16_gated_mlp_h4096_i14336_m32", 10),
                         ("lf_fp8_w8a8_gated_mlp_t256_t256", 11), ("lf_fp8_w8a8_dense_t256_aq", 12),
                         ("lf_fp8_w8a8_qkv_t128_aq", 13), ("lf_fp8_w8a8_gate_up_t256x128_aq", 14),
                         ("lf_fp8_w8a16_dense_b128_m16", 15), ("lf_fp8_w8a16_qkv_b128_m128", 16),
                         ("lf_fp8_w8a16_gate_up_b128_m32", 17), ("lf_fp8_w8a8_dense_b128", 18),
                         ("lf_fp8_w8a8_qkv_b128", 19), ("lf_fp8_w8a8_gate_up_b128", 20),
                         ("lf_fp8_w8a8_gated_mlp_b128", 21)]:
        assert symbols[name][0] == family, name
    assert "lf_calibrate_copy" not in symbols          # a benchmark tool, not a plan kernel
    pairs = [(e["family_id"], e["entry_point_id"]) for e in module["entry_points"]]
    assert len(set(pairs)) == len(pairs)
    admitted = admit(d, image)
    assert len(admitted) == len(symbols) >= 55


def test_build_writes_an_admissible_manifest(image):
    path = os.path.join(os.path.dirname(_abi.CODE_OBJECT_PATH), manifest.MANIFEST)
    with open(path, "rb") as f:
        text = f.read()
    assert manifest.admit_manifest(text, {manifest.CODE_OBJECT: image}, "0" * 64, "0" * 64)


def mutated(image, change):
    d = doc(image)
    change(d)
    return d


@pytest.mark.parametrize("change,kind", [
    (lambda d: d.update(schema_version=2), "InvalidField"),
    (lambda d: d.update(extra=1), "UnknownField"),
    (lambda d: d.pop("catalog_version"), "MissingField"),
    (lambda d: d.update(catalog_version=2), "IdentityMismatch"),
    (lambda d: d["model_identity"].update(content_sha256="AB" * 32), "InvalidField"),
    (lambda d: d["model_identity"].update(plan_sha256="ef" * 32), "IdentityMismatch"),
    (lambda d: d["device_target"].update(compute_minor=4), "IdentityMismatch"),
    (lambda d: d["device_target"].update(compute_major=8), "IdentityMismatch"),
    (lambda d: d["device_target"].update(supports_cublas_lt=True), "IdentityMismatch"),
    (lambda d: d["device_target"].update(supports_bf16=1), "InvalidField"),
    (lambda d: d["modules"][0].update(sha256="0" * 64), "DigestMismatch"),
    (lambda d: d["modules"][0].update(path="../lunaflux_fp8.hsaco"), "InvalidPath"),
    (lambda d: d["modules"][0].update(path="/abs/x.hsaco"), "InvalidPath"),
    (lambda d: d["modules"][0].update(path="a//b"), "InvalidPath"),
    (lambda d: d["modules"][0].update(path="a b"), "InvalidPath"),
    (lambda d: d["modules"][0].update(path="other.hsaco"), "MissingModule"),
    (lambda d: d["modules"].append(dict(d["modules"][0])), "DuplicateModule"),
    (lambda d: d["modules"][0]["entry_points"][0].update(symbol="9bad"), "InvalidFunctionSymbol"),
    (lambda d: d["modules"][0]["entry_points"][0].update(symbol="a-b"), "InvalidFunctionSymbol"),
    (lambda d: d["modules"][0]["entry_points"][0].update(symbol="x" * 129), "InvalidFunctionSymbol"),
    (lambda d: d["modules"][0]["entry_points"][0].update(symbol="lf_not_a_kernel"),
     "InvalidFunctionSymbol"),
    (lambda d: d["modules"][0]["entry_points"][0].update(family_id=-1), "InvalidField"),
    (lambda d: d["modules"][0]["entry_points"][0].update(entry_point_id=True), "InvalidField"),
    (lambda d: d["modules"][0]["entry_points"].append(dict(d["modules"][0]["entry_points"][0])),
     "DuplicateEntryPoint"),
])
def test_manifest_rejections(image, change, kind):
    with pytest.raises(manifest.ManifestError) as err:
        admit(mutated(image, change), image)
    assert err.value.kind == kind, err.value


def test_manifest_text_rejections(image):
    good = json.dumps(doc(image))
    cases = [(b"\xff" + good.encode(), "InvalidUtf8"),
             (good.encode()[:-1], "MalformedJson"),
             (good.replace('"catalog_version": 1', '"catalog_version": 1, "catalog_version": 1')
              .encode(), "DuplicateField"),
             (b"[" * 20 + b"]" * 20, "JsonDepthExceeded"),
             (b" " * (manifest.MAX_MANIFEST_BYTES + 1), "FileTooLarge")]
    for text, kind in cases:
        with pytest.raises(manifest.ManifestError) as err:
            admit(text, image)
        assert err.value.kind == kind, (kind, err.value)

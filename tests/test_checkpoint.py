"""FP8 checkpoint admission (lunaflux_amd/checkpoint.py), CPU only: files
written here in the safetensors layout (8-byte little-endian header length,
JSON header, payload), read back bit for bit into the packed weight region,
and every header rejection of model/safetensors/metadata.mbt:90-175."""
import json
import struct

import numpy as np
import pytest

import oracle_lib as o
from lunaflux_amd import checkpoint, fp8, synth


def write_safetensors(path, tensors, header_edit=None):
    """tensors: name -> (dtype string, numpy array). Payload in given order."""
    header, blobs, pos = {}, [], 0
    for name, (dtype, arr) in tensors.items():
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [pos, pos + len(raw)]}
        blobs.append(raw)
        pos += len(raw)
    header["__metadata__"] = {"format": "pt"}
    if header_edit:
        header_edit(header)
    text = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + b"".join(blobs))


def test_per_channel_and_block_weights_round_trip(tmp_path):
    rng = np.random.default_rng(5)
    qc, sc = synth.weight(rng, 256, 384)
    qb, sb = synth.weight(rng, 256, 384, block=128)
    path = str(tmp_path / "model.safetensors")
    write_safetensors(path, {
        "layers.0.o_proj.weight": ("F8_E4M3", qc),
        "layers.0.o_proj.weight_scale": ("F32", sc.reshape(-1, 1)),
        "layers.0.mlp.down.weight": ("F8_E4M3", qb),
        "layers.0.mlp.down.weight_scale_inv": ("F32", sb.reshape(2, 3)),
        "layers.0.norm.weight": ("BF16", synth.bf16_bits(np.ones(384, np.float32))),
    })
    q, s, mode = checkpoint.load_fp8_linear(path, "layers.0.o_proj")
    assert mode == fp8.PER_CHANNEL and np.array_equal(q, qc) and np.array_equal(s, sc)
    q2, s2, info = fp8.unpack_weight(fp8.pack_weight(q, s, mode))
    assert np.array_equal(q2[0], qc) and np.array_equal(s2[0], sc)
    q, s, mode = checkpoint.load_fp8_linear(path, "layers.0.mlp.down")
    assert mode == fp8.BLOCK128 and np.array_equal(q, qb)
    assert np.array_equal(s.reshape(-1), sb.reshape(-1))
    # the dequantized weight is fp32(code) * scale, as the oracle defines it
    w = o.dequantize(q, s, mode=2, group=128)
    blk = o.e4m3_decode(qb[:128, :128]) * np.float32(sb.reshape(2, 3)[0, 0])
    assert np.array_equal(w[:128, :128], blk.astype(np.float32))
    tensors, off = checkpoint.read_metadata(path)
    assert tensors["layers.0.norm.weight"].dtype == "BF16"
    g = checkpoint.load_tensor(path, tensors, off, "layers.0.norm.weight")
    assert np.all(g == 0x3F80)


@pytest.mark.parametrize("edit,kind", [
    (lambda h: h["w.weight"].update(dtype="F16"), "InvalidDType"),
    (lambda h: h["w.weight"].update(shape=[]), "InvalidRank"),
    (lambda h: h["w.weight"].update(data_offsets=[10, 5]), "InvalidByteRange"),
    (lambda h: h["w.weight"].update(data_offsets=[0, 10 ** 9]), "RangeOutsidePayload"),
    (lambda h: h["w.weight"].update(shape=[16, 127]), "RangeSizeMismatch"),
    (lambda h: h["w.weight_scale"].update(data_offsets=[0, 64]), "OverlappingTensors"),
    (lambda h: h.update({"bad\nname": h.pop("w.weight")}), "InvalidTensorName"),
])
def test_header_rejections(tmp_path, edit, kind):
    rng = np.random.default_rng(6)
    q, s = synth.weight(rng, 16, 128)
    path = str(tmp_path / "bad.safetensors")
    write_safetensors(path, {"w.weight": ("F8_E4M3", q), "w.weight_scale": ("F32", s)}, edit)
    with pytest.raises(checkpoint.SafetensorsError) as err:
        checkpoint.read_metadata(path)
    assert err.value.kind == kind


def test_duplicate_names_and_scale_shapes(tmp_path):
    path = str(tmp_path / "dup.safetensors")
    text = b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}, ' \
           b'"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}'
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + bytes(8))
    with pytest.raises(checkpoint.SafetensorsError) as err:
        checkpoint.read_metadata(path)
    assert err.value.kind == "DuplicateTensor"
    rng = np.random.default_rng(7)
    q, s = synth.weight(rng, 16, 128)
    path = str(tmp_path / "scale.safetensors")
    write_safetensors(path, {"w.weight": ("F8_E4M3", q), "w.weight_scale": ("F32", s[:8])})
    with pytest.raises(checkpoint.SafetensorsError) as err:
        checkpoint.load_fp8_linear(path, "w")
    assert err.value.kind == "InvalidScaleShape"
    with pytest.raises(checkpoint.SafetensorsError) as err:
        checkpoint.load_fp8_linear(path, "missing")
    assert err.value.kind == "MissingTensor"

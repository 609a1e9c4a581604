"""FP8 checkpoint admission (lunaflux_amd/checkpoint.py), CPU only: files
written here in the safetensors layout (8-byte little-endian header length,
JSON header, payload), read back bit for bit into the packed weight region;
one case per rejection of the reference reader and validator
(model/safetensors_reader/reader.mbt:217-306,
model/safetensors/metadata.mbt:63-175), in their order; the FP8 value checks;
and the model-level binding in model/llama_weights/bind.mbt's TensorRef
order."""
import json
import struct

import numpy as np
import pytest

import oracle_lib as o
from lunaflux_amd import checkpoint, fp8, synth


def header_bytes(tensors, header_edit=None):
    header, blobs, pos = {}, [], 0
    for name, (dtype, arr) in tensors.items():
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [pos, pos + len(raw)]}
        blobs.append(raw)
        pos += len(raw)
    header["__metadata__"] = {"format": "pt"}
    if header_edit:
        header_edit(header)
    return json.dumps(header).encode(), b"".join(blobs)


def write_raw(path, text: bytes, payload: bytes, length=None):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text) if length is None else length) + text + payload)


def write_safetensors(path, tensors, header_edit=None):
    """tensors: name -> (dtype string, numpy array). Payload in given order."""
    text, payload = header_bytes(tensors, header_edit)
    write_raw(path, text, payload)


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
    assert list(tensors)[0] == "layers.0.o_proj.weight"  # header order kept
    assert tensors["layers.0.norm.weight"].dtype == "BF16"
    g = checkpoint.load_tensor(path, tensors, off, "layers.0.norm.weight")
    assert np.all(g == 0x3F80)


def test_per_tensor_scale_is_broadcast_to_every_channel(tmp_path):
    rng = np.random.default_rng(8)
    q, _ = synth.weight(rng, 32, 128)
    path = str(tmp_path / "t.safetensors")
    write_safetensors(path, {"w.weight": ("F8_E4M3", q),
                             "w.weight_scale": ("F32", np.array([0.0125], np.float32))})
    q2, s, mode = checkpoint.load_fp8_linear(path, "w")
    assert mode == fp8.PER_CHANNEL and s.shape == (32,) and np.all(s == np.float32(0.0125))


def _mutate(h, name, **fields):
    h[name].update(fields)


@pytest.mark.parametrize("edit,kind", [
    (lambda h: _mutate(h, "w.weight", dtype="F16"), "InvalidDType"),
    (lambda h: _mutate(h, "w.weight", shape=[]), "InvalidRank"),
    (lambda h: _mutate(h, "w.weight", shape=[1, 16, 128]), "InvalidRank"),
    (lambda h: _mutate(h, "w.weight", shape=[16, 0]), "InvalidDimension"),
    (lambda h: _mutate(h, "w.weight", shape=[-16, 128]), "InvalidDimension"),
    (lambda h: _mutate(h, "w.weight", shape=[2 ** 40, 2 ** 40]), "TensorSizeOverflow"),
    (lambda h: _mutate(h, "w.weight", shape=[16, True]), "InvalidInteger"),
    (lambda h: _mutate(h, "w.weight", shape=[16, 127.5]), "InvalidInteger"),
    (lambda h: _mutate(h, "w.weight", shape=[16, "128"]), "InvalidInteger"),
    (lambda h: _mutate(h, "w.weight", shape=[16, 2 ** 64]), "InvalidInteger"),
    (lambda h: _mutate(h, "w.weight", shape=16), "InvalidTensorField"),
    (lambda h: _mutate(h, "w.weight", dtype=8), "InvalidTensorField"),
    (lambda h: _mutate(h, "w.weight", data_offsets=[0]), "InvalidTensorField"),
    (lambda h: _mutate(h, "w.weight", data_offsets=[0, False]), "InvalidInteger"),
    (lambda h: _mutate(h, "w.weight", data_offsets=[10, 5]), "InvalidByteRange"),
    (lambda h: _mutate(h, "w.weight", data_offsets=[-1, 2047]), "InvalidByteRange"),
    (lambda h: _mutate(h, "w.weight", data_offsets=[0, 10 ** 9]), "RangeOutsidePayload"),
    (lambda h: _mutate(h, "w.weight", shape=[16, 127]), "RangeSizeMismatch"),
    (lambda h: _mutate(h, "w.weight_scale", data_offsets=[0, 64]), "OverlappingTensors"),
    (lambda h: h.update({"bad\nname": h.pop("w.weight")}), "InvalidTensorName"),
    (lambda h: h.update({"": h.pop("w.weight")}), "InvalidTensorName"),
    (lambda h: h.update({"x" * 257: h.pop("w.weight")}), "InvalidTensorName"),
    (lambda h: h.update({"café": h.pop("w.weight")}), "InvalidTensorName"),
    (lambda h: _mutate(h, "w.weight", extra=1), "UnexpectedTensorField"),
    (lambda h: h["w.weight"].pop("dtype"), "MissingTensorField"),
    (lambda h: h["w.weight"].pop("shape"), "MissingTensorField"),
    (lambda h: h["w.weight"].pop("data_offsets"), "MissingTensorField"),
    (lambda h: h.update({"w.weight": [1]}), "InvalidTensor"),
    (lambda h: h.update({"__metadata__": {"format": 1}}), "InvalidMetadata"),
    (lambda h: h.update({"__metadata__": "pt"}), "InvalidMetadata"),
    (lambda h: h.update({"z": {"dtype": "F32", "shape": [1], "data_offsets": [2112, 2116]}}),
     "RangeOutsidePayload"),
    (lambda h: _mutate(h, "w.weight", shape=[[16], [128]]), "InvalidInteger"),
])
def test_header_rejections(tmp_path, edit, kind):
    rng = np.random.default_rng(6)
    q, s = synth.weight(rng, 16, 128)
    path = str(tmp_path / "bad.safetensors")
    write_safetensors(path, {"w.weight": ("F8_E4M3", q), "w.weight_scale": ("F32", s)}, edit)
    with pytest.raises(checkpoint.SafetensorsError) as err:
        checkpoint.read_metadata(path)
    assert err.value.kind == kind


def test_check_order_reports_the_first_failing_check_of_the_first_bad_tensor(tmp_path):
    path = str(tmp_path / "order.safetensors")
    # tensor 0 has a bad dtype and a bad range: the dtype check comes first
    text = (b'{"a": {"dtype": "F64", "shape": [1], "data_offsets": [9, 1]}, '
            b'"b": {"dtype": "F33", "shape": [1], "data_offsets": [0, 4]}}')
    write_raw(path, text, bytes(4))
    with pytest.raises(checkpoint.SafetensorsError) as err:
        checkpoint.read_metadata(path)
    assert (err.value.kind, err.value.index) == ("InvalidDType", 0)
    # the rank bound of the reader comes before integer decoding
    text = b'{"a": {"dtype": "F32", "shape": [1, 1, true], "data_offsets": [0, 4]}}'
    write_raw(path, text, bytes(4))
    with pytest.raises(checkpoint.SafetensorsError) as err:
        checkpoint.read_metadata(path)
    assert err.value.kind == "InvalidRank"
    # an unexpected field is found before a missing one
    text = b'{"a": {"shape": [1], "data_offsets": [0, 4], "x": 0}}'
    write_raw(path, text, bytes(4))
    with pytest.raises(checkpoint.SafetensorsError) as err:
        checkpoint.read_metadata(path)
    assert err.value.kind == "UnexpectedTensorField"


def test_envelope_and_length_rejections(tmp_path):
    path = str(tmp_path / "env.safetensors")
    good = b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}'
    cases = [
        (lambda: open(path, "wb").write(b"\x01\x00"), "MissingHeaderLength"),
        (lambda: write_raw(path, good, bytes(4), length=2 ** 31), "HeaderLengthOverflow"),
        (lambda: write_raw(path, good, b"", length=len(good) + 100), "TruncatedHeader"),
        (lambda: write_raw(path, b" " + good, bytes(4)), "InvalidHeaderEnvelope"),
        (lambda: write_raw(path, good + b"\n", bytes(4)), "InvalidHeaderEnvelope"),
        (lambda: write_raw(path, good[:-1] + b"\xff}", bytes(4)), "InvalidHeaderEncoding"),
        (lambda: write_raw(path, b'{"a": NaN}', b""), "InvalidHeaderJson"),
        (lambda: write_raw(path, b'{"a": {"b": {"c": [[1]]}}}', b""), "InvalidHeaderJson"),
        (lambda: write_raw(path, good, bytes(5)), "PayloadSizeMismatch"),
    ]
    for write, kind in cases:
        write()
        with pytest.raises(checkpoint.SafetensorsError) as err:
            checkpoint.read_metadata(path)
        assert err.value.kind == kind, (kind, err.value)
    # trailing spaces after the closing brace are part of a valid envelope
    write_raw(path, good + b"   ", bytes(4))
    tensors, off = checkpoint.read_metadata(path)
    assert off == 8 + len(good) + 3 and tensors["a"].shape == (1,)
    # exactly integral numbers in float form are accepted
    write_raw(path, b'{"a": {"dtype": "F32", "shape": [1.0], "data_offsets": [0, 4e0]}}',
              bytes(4))
    assert checkpoint.read_metadata(path)[0]["a"].end == 4


def test_duplicate_keys_at_each_depth(tmp_path):
    path = str(tmp_path / "dup.safetensors")
    tensor = '{"dtype": "F32", "shape": [1], "data_offsets": [%d, %d]}'
    cases = [
        # two tensors of one name: depth 1 (the root object), second key
        ('{"a": %s, "a": %s}' % (tensor % (0, 4), tensor % (4, 8)), (1, 1)),
        # a repeated field inside a tensor entry: depth 2, its third key
        ('{"b": %s, "a": {"dtype": "F32", "shape": [1], "dtype": "F32", '
         '"data_offsets": [0, 4]}}' % (tensor % (4, 8)), (2, 2)),
        # a repeated __metadata__ key counts __metadata__'s own keys
        ('{"__metadata__": {"x": "1", "y": "2", "x": "3"}, "a": %s, "b": %s}'
         % (tensor % (0, 4), tensor % (4, 8)), (2, 2)),
    ]
    for text, where in cases:
        write_raw(path, text.encode(), bytes(8))
        with pytest.raises(checkpoint.SafetensorsError) as err:
            checkpoint.read_metadata(path)
        assert err.value.kind == "DuplicateHeaderKey" and err.value.other == where


def test_limits(tmp_path):
    rng = np.random.default_rng(9)
    q, s = synth.weight(rng, 16, 128)
    path = str(tmp_path / "lim.safetensors")
    write_safetensors(path, {"w.weight": ("F8_E4M3", q), "w.weight_scale": ("F32", s)})
    cases = [(checkpoint.HeaderLimits(max_header_bytes=32), "HeaderTooLarge"),
             (checkpoint.HeaderLimits(max_tensor_count=1), "TooManyTensors"),
             (checkpoint.HeaderLimits(max_name_length=7), "InvalidTensorName"),
             (checkpoint.HeaderLimits(max_rank=1), "InvalidRank"),
             (checkpoint.HeaderLimits(max_payload_bytes=2000, max_materialized_tensor_bytes=2000),
              "RangeOutsidePayload"),
             (checkpoint.HeaderLimits(max_materialized_tensor_bytes=2100), "MaterializedSizeExceeded")]
    for limits, kind in cases:
        with pytest.raises(checkpoint.SafetensorsError) as err:
            checkpoint.read_metadata(path, limits)
        assert err.value.kind == kind, kind
    for bad in [dict(max_header_bytes=0), dict(max_tensor_count=0), dict(max_rank=0),
                dict(max_name_length=0), dict(max_payload_bytes=0),
                dict(max_payload_bytes=10, max_materialized_tensor_bytes=11)]:
        with pytest.raises(checkpoint.SafetensorsError) as err:
            checkpoint.HeaderLimits(**bad)
        assert err.value.kind == "InvalidLimit"


def test_rank0_scale_is_rejected_by_metadata_validation(tmp_path):
    """A scalar (rank-0) weight_scale, the per-tensor form some FP8
    checkpoints use, fails the metadata validation with InvalidRank, as
    every rank-0 tensor does in the reference (metadata.mbt:63-86); the same
    scale stored as shape [1] is admitted and broadcast."""
    rng = np.random.default_rng(8)
    q, _ = synth.weight(rng, 16, 128)
    path = str(tmp_path / "scalar.safetensors")
    write_safetensors(path, {"w.weight": ("F8_E4M3", q),
                             "w.weight_scale": ("F32", np.array(0.5, np.float32))})
    with pytest.raises(checkpoint.SafetensorsError) as err:
        checkpoint.read_metadata(path)
    assert err.value.kind == "InvalidRank"
    write_safetensors(path, {"w.weight": ("F8_E4M3", q),
                             "w.weight_scale": ("F32", np.array([0.5], np.float32))})
    _, scales, mode = checkpoint.load_fp8_linear(path, "w")
    assert mode == fp8.PER_CHANNEL and np.all(scales == np.float32(0.5)) and scales.shape == (16,)


def test_scale_shapes_and_values(tmp_path):
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
    for bad_s, kind in [(np.where(np.arange(16) == 3, np.nan, s).astype(np.float32), "InvalidScale"),
                        (np.where(np.arange(16) == 3, np.inf, s).astype(np.float32), "InvalidScale"),
                        (-s, "InvalidScale")]:
        write_safetensors(path, {"w.weight": ("F8_E4M3", q), "w.weight_scale": ("F32", bad_s)})
        with pytest.raises(checkpoint.SafetensorsError) as err:
            checkpoint.load_fp8_linear(path, "w")
        assert err.value.kind == kind
    # an all-zero channel has scale 0 (absmax / 448): admitted
    z = q.copy()
    z[5] = 0
    s0 = s.copy()
    s0[5] = 0
    write_safetensors(path, {"w.weight": ("F8_E4M3", z), "w.weight_scale": ("F32", s0)})
    assert checkpoint.load_fp8_linear(path, "w")[1][5] == 0
    for code in (0x7F, 0xFF):   # e4m3 NaN, either sign
        bad_q = q.copy()
        bad_q[2, 9] = code
        write_safetensors(path, {"w.weight": ("F8_E4M3", bad_q), "w.weight_scale": ("F32", s)})
        with pytest.raises(checkpoint.SafetensorsError) as err:
            checkpoint.load_fp8_linear(path, "w")
        assert err.value.kind == "NonFiniteWeight"


TINY = checkpoint.LlamaShape(vocabulary=256, hidden=128, intermediate=256, layers=2,
                             attention_heads=4, kv_heads=2)


def tiny_llama_tensors(rng, shape=TINY, block_down=True, fp8_head=False):
    h, i, v, kv = shape.hidden, shape.intermediate, shape.vocabulary, shape.kv_width
    t = {"model.embed_tokens.weight": ("BF16", synth.bf16_bits(rng.standard_normal((v, h))))}

    def proj(name, n, k, block=False):
        q, s = synth.weight(rng, n, k, block=128 if block else None)
        t[name + ".weight"] = ("F8_E4M3", q)
        if block:
            t[name + ".weight_scale_inv"] = ("F32", s.reshape(n // 128, k // 128))
        else:
            t[name + ".weight_scale"] = ("F32", s)

    for layer in range(shape.layers):
        p = f"model.layers.{layer}"
        t[f"{p}.input_layernorm.weight"] = ("BF16", synth.bf16_bits(np.ones(h, np.float32)))
        proj(f"{p}.self_attn.q_proj", h, h)
        proj(f"{p}.self_attn.k_proj", kv, h)
        proj(f"{p}.self_attn.v_proj", kv, h)
        proj(f"{p}.self_attn.o_proj", h, h)
        t[f"{p}.post_attention_layernorm.weight"] = ("BF16", synth.bf16_bits(np.ones(h, np.float32)))
        proj(f"{p}.mlp.gate_proj", i, h)
        proj(f"{p}.mlp.up_proj", i, h)
        proj(f"{p}.mlp.down_proj", h, i, block=block_down)
    t["model.norm.weight"] = ("BF16", synth.bf16_bits(np.ones(h, np.float32)))
    if fp8_head:
        proj("lm_head", v, h)
    else:
        t["lm_head.weight"] = ("BF16", synth.bf16_bits(rng.standard_normal((v, h))))
    return t


def test_bind_llama_fp8_in_tensor_ref_order(tmp_path):
    rng = np.random.default_rng(10)
    path = str(tmp_path / "llama.safetensors")
    t = tiny_llama_tensors(rng, fp8_head=True)
    # the file's own order is not the binding order: shuffle the header
    names = list(t)
    rng.shuffle(names)
    write_safetensors(path, {n: t[n] for n in names})
    tensors, _ = checkpoint.read_metadata(path)
    b = checkpoint.bind_llama_fp8(TINY, tensors)
    assert len(b) == 3 + 9 * TINY.layers
    assert [x.reference for x in b] == list(range(len(b)))
    assert b[0].name == "model.embed_tokens.weight" and b[0].dtype == "BF16"
    layer0 = [x.name.split(".", 3)[-1] for x in b[1:10]]
    assert layer0 == ["input_layernorm.weight", "self_attn.q_proj.weight",
                      "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                      "self_attn.o_proj.weight", "post_attention_layernorm.weight",
                      "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"]
    assert b[2].shape == (128, 128) and b[3].shape == (64, 128) and b[9].shape == (128, 256)
    assert b[9].scale_name.endswith("weight_scale_inv") and b[2].scale_name.endswith("weight_scale")
    assert b[-2].name == "model.norm.weight" and b[-1].name == "lm_head.weight"
    assert b[-1].dtype == "F8_E4M3"


def _swap(t, name):
    """Replaces tensor `name` by an unrelated one: the count stays right."""
    t.pop(name)
    t["unrelated"] = ("F32", np.zeros(1, np.float32))


def _incomplete_and_misshapen(t):
    t.pop("model.layers.1.mlp.up_proj.weight_scale")
    t["model.layers.0.self_attn.k_proj.weight"] = ("F8_E4M3", np.zeros((128, 128), np.uint8))


@pytest.mark.parametrize("change,kind", [
    (lambda t: _swap(t, "model.layers.1.mlp.up_proj.weight_scale"), "MissingTensor"),
    (lambda t: _swap(t, "model.layers.0.self_attn.k_proj.weight"), "MissingTensor"),
    (lambda t: t.pop("model.layers.1.mlp.up_proj.weight_scale"), "TensorCountMismatch"),
    (lambda t: t.update({"extra": ("F32", np.zeros(1, np.float32))}), "TensorCountMismatch"),
    # the count is checked before any tensor (bind.mbt:57-63)
    (_incomplete_and_misshapen, "TensorCountMismatch"),
    # activation scales of static-quantized checkpoints are not part of the
    # bound vocabulary
    (lambda t: t.update({"model.layers.0.self_attn.q_proj.input_scale":
                         ("F32", np.ones(1, np.float32))}), "TensorCountMismatch"),
    (lambda t: t.update({"model.norm.weight": ("BF16", np.zeros((1, 128), np.uint16))}),
     "ShapeRankMismatch"),
    (lambda t: t.update({"model.layers.0.self_attn.k_proj.weight":
                         ("F8_E4M3", np.zeros((128, 128), np.uint8))}), "ShapeDimensionMismatch"),
    (lambda t: t.update({"model.layers.0.self_attn.o_proj.weight":
                         ("BF16", np.zeros((128, 128), np.uint16))}), "UnsupportedWeightDType"),
])
def test_bind_llama_fp8_rejections(tmp_path, change, kind):
    rng = np.random.default_rng(11)
    path = str(tmp_path / "llama.safetensors")
    t = tiny_llama_tensors(rng)
    change(t)
    write_safetensors(path, t)
    tensors, _ = checkpoint.read_metadata(path)
    with pytest.raises(checkpoint.LlamaWeightsError) as err:
        checkpoint.bind_llama_fp8(TINY, tensors)
    assert err.value.kind == kind

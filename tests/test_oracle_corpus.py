"""End-to-end pin of the oracle's projection semantics against an external
corpus: the reference's tiny Llama (stas/tiny-random-llama-2, 2 layers,
hidden 16, 4 heads, intermediate 64, vocabulary 3000, bf16 weights) run
forward through the oracle, compared with the logits and greedy
continuations transformers produced in fp32 (tests/reference_corpus/
corpus.json, MANIFEST.md:39-50; absolute and relative tolerance 1e-5).

The oracle supplies the bf16 decode of every tensor, RMSNorm, the fused QKV
projection, the output and vocabulary projections and the SiLU-gated MLP;
rotary embedding and causal attention, which are outside the FP8 projection
path, are restated here in numpy after kernels/reference/rotary.mbt:6-62 and
attention.mbt:7-87. The layer wiring follows the reference's dense Llama
builder (embedding, per layer x + o(attn(rope(qkv(norm(x))))) then
x + mlp(norm(x)), final norm, vocabulary head). A transposed weight, a
dropped residual or a wrong norm would move these logits far beyond 1e-5.

The fixtures are the reference corpus's data files, copied with their
SHA-256 checked (tests/golden/corpus/copy_corpus.py).
"""
import json
import os
import struct

import numpy as np
import pytest

import oracle_lib as o

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "corpus")


def load_model():
    config = json.load(open(os.path.join(HERE, "config.json")))
    raw = open(os.path.join(HERE, "model.safetensors"), "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    tensors = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        assert meta["dtype"] == "BF16", name
        a, b = meta["data_offsets"]
        shape = meta["shape"]
        rows, cols = (shape[0], shape[1]) if len(shape) == 2 else (1, shape[0])
        tensors[name] = o.decode_bfloat16_le(raw[8 + n + a:8 + n + b], rows, cols)
    return config, tensors


def rotary(qkv, heads, kv_heads, dim, theta):
    """kernels/reference/rotary.mbt:6-62: split-half rotation of the Q and K
    heads of each row (row index = position), fp32."""
    out = qkv.copy()
    half = dim // 2
    for row in range(qkv.shape[0]):
        pos = np.float32(row)
        for head in range(heads + kv_heads):
            base = head * dim
            for pair in range(half):
                exponent = np.float32(pair * 2) / np.float32(dim)
                angle = pos / np.power(np.float32(theta), exponent, dtype=np.float32)
                c, s = np.cos(angle, dtype=np.float32), np.sin(angle, dtype=np.float32)
                first, second = qkv[row, base + pair], qkv[row, base + pair + half]
                out[row, base + pair] = first * c - second * s
                out[row, base + pair + half] = second * c + first * s
    return out


def attention(qkv, heads, kv_heads, dim):
    """kernels/reference/attention.mbt:7-87: causal GQA, max-subtracted
    softmax, fp32."""
    rows = qkv.shape[0]
    qw, kvw = heads * dim, kv_heads * dim
    out = np.zeros((rows, qw), np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(dim))
    group = heads // kv_heads
    for r in range(rows):
        for h in range(heads):
            kvh = h // group
            q = qkv[r, h * dim:(h + 1) * dim]
            scores = np.array([np.float32(np.dot(q, qkv[j, qw + kvh * dim:qw + (kvh + 1) * dim])) * scale
                               for j in range(r + 1)], np.float32)
            p = np.exp(scores - scores.max(), dtype=np.float32)
            p = p / np.float32(p.sum(dtype=np.float32))
            v = qkv[:r + 1, qw + kvw + kvh * dim:qw + kvw + (kvh + 1) * dim]
            out[r, h * dim:(h + 1) * dim] = (p[:, None] * v).sum(axis=0, dtype=np.float32)
    return out


def forward(config, t, ids):
    """Last-position logits of the token ids."""
    dim = config["hidden_size"] // config["num_attention_heads"]
    heads, kv_heads = config["num_attention_heads"], config["num_key_value_heads"]
    eps, theta = config["rms_norm_eps"], config["rope_theta"]
    x = t["model.embed_tokens.weight"][np.asarray(ids)]
    for layer in range(config["num_hidden_layers"]):
        p = f"model.layers.{layer}."
        hn = o.rms_norm(x, t[p + "input_layernorm.weight"], eps)
        qkv = o.qkv_projection(hn, t[p + "self_attn.q_proj.weight"], t[p + "self_attn.k_proj.weight"],
                               t[p + "self_attn.v_proj.weight"])
        a = attention(rotary(qkv, heads, kv_heads, dim, theta), heads, kv_heads, dim)
        x = x + o.project_values(a, t[p + "self_attn.o_proj.weight"])
        hn = o.rms_norm(x, t[p + "post_attention_layernorm.weight"], eps)
        x = x + o.silu_gated_mlp(hn, t[p + "mlp.gate_proj.weight"], t[p + "mlp.up_proj.weight"],
                                 t[p + "mlp.down_proj.weight"])
    x = o.rms_norm(x, t["model.norm.weight"], eps)
    return o.project_values(x[-1:], t["lm_head.weight"])[0]


@pytest.fixture(scope="module")
def model():
    return load_model()


CORPUS = json.load(open(os.path.join(HERE, "corpus.json")))


@pytest.mark.parametrize("case", CORPUS["model_cases"], ids=lambda c: "ids" + "_".join(map(str, c["input_ids"])))
def test_tiny_llama_logits_and_greedy_tokens(model, case):
    config, t = model
    tol = CORPUS["logit_tolerance"]
    logits = forward(config, t, case["input_ids"])
    assert logits.shape == (config["vocab_size"],)
    for index, expected in case["sampled_logits"].items():
        np.testing.assert_allclose(logits[int(index)], expected, rtol=tol["relative"],
                                   atol=tol["absolute"], err_msg=f"logit {index}")
    assert int(np.argmax(logits)) == case["greedy_token"]
    ids = list(case["input_ids"])
    for expected in case["greedy_continuation"]:
        nxt = int(np.argmax(forward(config, t, ids)))
        assert nxt == expected
        ids.append(nxt)


def test_corpus_pin_catches_a_transposed_operand(model):
    """The pin is sensitive: the same forward with layer 0's output
    projection weight transposed (a layout mistake on a square weight, which
    no shape check catches) misses the sampled logits by far more than the
    tolerance."""
    config, t = model
    bad = dict(t)
    w = t["model.layers.0.self_attn.o_proj.weight"]
    bad["model.layers.0.self_attn.o_proj.weight"] = np.ascontiguousarray(w.T)
    case = CORPUS["model_cases"][2]
    good, wrong = forward(config, t, case["input_ids"]), forward(config, bad, case["input_ids"])
    idx = [int(i) for i in case["sampled_logits"]]
    exp = np.array([case["sampled_logits"][str(i)] for i in idx], np.float32)
    assert np.max(np.abs(good[idx] - exp)) <= 1e-5
    assert np.max(np.abs(wrong[idx] - exp)) > 1e-3

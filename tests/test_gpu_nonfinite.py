"""Non-finite inputs on the GPU path.

The reference rejects NaN and infinite values (decode:
kernels/reference/bfloat16.mbt:24-26; a non-finite sum:
kernels/reference/basic.mbt:91-93). A kernel cannot raise, so the device
contract these tests hold it to is:
* a row of activations holding a NaN or an infinity gives a row of outputs
  that are all non-finite (every output of that row depends on the value);
* every other row's outputs are bit-identical to a run without it (nothing
  leaks across rows, and no memory access moves);
* in routing, a NaN logit ranks as -inf (below every finite logit, ties to
  the lower expert id), so each token still gets k distinct experts in
  [0, E) and the sort still places all T k assignments; a token whose top
  logit is non-finite (+inf, or all NaN / -inf) gets NaN routing weights and
  a non-finite output row; every other token is bit-identical to a run with
  finite logits in that row.
"""
import numpy as np
import pytest

from lunaflux_amd import synth

pytestmark = pytest.mark.gpu

NAN, POS_INF, NEG_INF = 0x7FC0, 0x7F80, 0xFF80


@pytest.fixture(scope="module")
def rt():
    from lunaflux_amd.fp8 import ProjectionRuntime
    return ProjectionRuntime(0)


def non_finite(bits):
    return (np.asarray(bits, np.uint16) & 0x7F80) == 0x7F80


def poison(x):
    bad = x.copy()
    bad[1, 5] = NAN
    bad[3, x.shape[1] - 1] = POS_INF
    bad[4, x.shape[1] // 2] = NEG_INF
    return bad, [1, 3, 4]


@pytest.mark.parametrize("op,family,m,max_tokens,k", [
    ("o", "w8a16", 8, 16, 4096), ("o", "w8a16", 32, 32, 4096), ("o", "w8a16", 20, 128, 4096),
    ("o", "w8a16", 6, 16, 512), ("o", "w8a16", 40, 64, 512), ("o", "w8a8", 64, 64, 4096),
    ("o", "w8a8", 300, 512, 1024), ("gate_up", "w8a16", 32, 32, 4096),
    ("gate_up", "w8a8", 50, 64, 1024), ("qkv", "w8a16", 10, 16, 4096),
])
def test_nonfinite_activation_rows(rt, op, family, m, max_tokens, k):
    rng = np.random.default_rng(3100 + m + k)
    x = synth.activations(rng, m, k)
    bad, rows = poison(x)
    if op == "qkv":
        ws = [rt.upload_weight(*synth.weight(rng, n, k)) for n in (4096, 1024, 1024)]
        run = lambda xx: rt.qkv_projection(xx, *ws, family=family, max_tokens=max_tokens)
    elif op == "gate_up":
        wg, wu = (rt.upload_weight(*synth.weight(rng, 1536, k)) for _ in range(2))
        run = lambda xx: rt.gate_up_swiglu(xx, wg, wu, family=family, max_tokens=max_tokens)
    else:
        w = rt.upload_weight(*synth.weight(rng, 1536 if k == 512 else 4096, k))
        run = lambda xx: rt.dense_projection(xx, w, family=family, max_tokens=max_tokens)
    clean, dirty = run(x), run(bad)
    keep = np.setdiff1d(np.arange(m), rows)
    assert np.array_equal(dirty[keep], clean[keep]), "a non-finite row changed other rows"
    assert not non_finite(clean).any()
    for r in rows:
        assert non_finite(dirty[r]).all(), f"row {r}: finite outputs from a non-finite input"


def test_nonfinite_rows_in_the_fused_rms_norm_quantizer(rt):
    rng = np.random.default_rng(3200)
    m, k = 24, 4096
    x = synth.activations(rng, m, k)
    bad, rows = poison(x)
    gamma = synth.bf16_bits(rng.uniform(0.5, 1.5, k).astype(np.float32))
    w = rt.upload_weight(*synth.weight(rng, 256, k))
    q0, s0 = rt.rms_norm_quant(x, gamma, w, 1e-5)
    q1, s1 = rt.rms_norm_quant(bad, gamma, w, 1e-5)
    keep = np.setdiff1d(np.arange(m), rows)
    assert np.array_equal(q1[keep], q0[keep]) and np.array_equal(s1[keep], s0[keep])


def key_order(row, k):
    """Top-k expert ids by the device's ranking key (NaN as -inf, ties to the
    lower id)."""
    key = np.where(np.isnan(row), -np.inf, row)
    return sorted(range(len(row)), key=lambda e: (-key[e], e))[:k]


@pytest.mark.parametrize("mode", [0, 1])
def test_nonfinite_router_logits(rt, mode):
    from lunaflux_amd import moe
    rng = np.random.default_rng(3300 + mode)
    t, e, k, hidden, inter = 64, 8, 2, 256, 256
    x = synth.activations(rng, t, hidden)
    clean = (rng.standard_normal((t, e)) + rng.normal(0, 1.5, e)).astype(np.float32)
    bad = clean.copy()
    bad[3, :] = np.nan           # all NaN: picks 0, 1; NaN weights
    bad[7, 2] = np.nan           # one NaN: ranks last
    bad[11, 5] = np.inf          # +inf: picked first, NaN weights
    bad[12, 1] = -np.inf         # one -inf: ranks last
    bad[13, :] = -np.inf         # all -inf: picks 0, 1; NaN weights
    poisoned = [3, 11, 13]
    ws = []
    for rows, cols in ((inter, hidden), (inter, hidden), (hidden, inter)):
        drawn = [synth.weight(rng, rows, cols) for _ in range(e)]
        ws.append(rt.upload_weight(np.stack([q for q, _ in drawn]), np.stack([s for _, s in drawn])))
    out0, st0 = moe.moe_expert_mlp(rt, x, clean, *ws, k, mode, return_workspace=True)
    out1, st1 = moe.moe_expert_mlp(rt, x, bad, *ws, k, mode, return_workspace=True)
    ids = st1["topk_ids"]
    assert ((ids >= 0) & (ids < e)).all()
    assert all(len(set(r)) == k for r in ids.tolist())
    assert np.array_equal(np.sort(st1["sorted"]), np.arange(t * k))
    assert st1["offsets"][-1] == t * k
    for r in (3, 7, 11, 12, 13):
        assert ids[r].tolist() == key_order(bad[r], k), (r, ids[r])
    for r in (7, 12):
        assert np.isfinite(st1["topk_w"][r]).all()
    for r in poisoned:
        assert np.isnan(st1["topk_w"][r]).all()
        assert non_finite(out1[r]).all()
    keep = np.setdiff1d(np.arange(t), [3, 7, 11, 12, 13])
    assert np.array_equal(ids[keep], st0["topk_ids"][keep])
    assert np.array_equal(st1["topk_w"][keep], st0["topk_w"][keep])
    # tokens with finite logits: bit-identical outputs (rows are independent
    # in every GEMM, whatever the other tokens' routing)
    assert np.array_equal(out1[keep], out0[keep])

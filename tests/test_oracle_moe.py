"""Pins the oracle's MoE router, stable sort and grouped MLP (absent from the
reference) by brute force, invariants and reduction to the dense oracle.
CPU only.
"""
import numpy as np
import pytest

import oracle_lib as o


def brute_topk(logits, k):
    picks = []
    for row in logits:
        order = sorted(range(len(row)), key=lambda e: (-float(row[e]), e))
        picks.append(order[:k])
    return np.array(picks, np.int32)


@pytest.mark.parametrize("mode", [o.ROUTE_TOPK_SOFTMAX, o.ROUTE_SOFTMAX_TOPK])
def test_route_topk_brute_force(mode):
    rng = np.random.default_rng(21)
    logits = rng.standard_normal((50, 8)).astype(np.float32)
    logits[3, :] = 0.5           # all tied: lowest ids win
    logits[4, [2, 6]] = 9.0      # a tie at the top
    ex, w = o.route_topk(logits, 3, mode)
    np.testing.assert_array_equal(ex, brute_topk(logits, 3))
    assert ex[3].tolist() == [0, 1, 2] and ex[4, :2].tolist() == [2, 6]
    l64 = logits.astype(np.float64)
    picked = np.take_along_axis(l64, ex.astype(np.int64), axis=1)
    if mode == o.ROUTE_TOPK_SOFTMAX:
        expect = np.exp(picked - picked[:, :1]) / np.exp(picked - picked[:, :1]).sum(1, keepdims=True)
        np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)
    else:
        full = np.exp(l64 - l64.max(1, keepdims=True))
        full /= full.sum(1, keepdims=True)
        expect = np.take_along_axis(full, ex.astype(np.int64), axis=1)
        assert (w.sum(1) <= 1.0 + 1e-6).all()
    np.testing.assert_allclose(w, expect, rtol=1e-5)
    assert (np.diff(w, axis=1) <= 0).all()


def test_moe_sort_stable_and_offsets():
    rng = np.random.default_rng(22)
    te = rng.integers(0, 8, (100, 2)).astype(np.int32)
    te[:, 1] = (te[:, 0] + 1 + rng.integers(0, 7, 100)) % 8
    sorted_a, offsets = o.moe_sort(te, 8)
    flat = te.reshape(-1)
    expect = sorted(range(flat.size), key=lambda a: flat[a])  # Python sort is stable
    np.testing.assert_array_equal(sorted_a, expect)
    counts = np.bincount(flat, minlength=8)
    np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))
    assert sorted(sorted_a.tolist()) == list(range(200))  # a bijection


def test_moe_sort_special_cases():
    # every assignment to one expert; the other experts are empty
    te = np.full((10, 3), 5, np.int32)
    sorted_a, offsets = o.moe_sort(te, 8)
    np.testing.assert_array_equal(sorted_a, np.arange(30))
    assert offsets.tolist() == [0, 0, 0, 0, 0, 0, 30, 30, 30]
    with pytest.raises(o.OracleError):
        o.moe_sort(np.full((2, 1), 9, np.int32), 8)


def test_moe_mlp_reduces_to_dense_oracle():
    rng = np.random.default_rng(23)
    t, h, inter, e, k = 6, 32, 24, 4, 2
    x = rng.standard_normal((t, h)).astype(np.float32)
    wg = (rng.standard_normal((e, inter, h)) * 0.2).astype(np.float32)
    wu = (rng.standard_normal((e, inter, h)) * 0.2).astype(np.float32)
    wd = (rng.standard_normal((e, h, inter)) * 0.2).astype(np.float32)
    logits = rng.standard_normal((t, e)).astype(np.float32)
    ex, w = o.route_topk(logits, k, o.ROUTE_TOPK_SOFTMAX)
    for transform in (0, 1):
        out = o.moe_mlp(x, wg, wu, wd, ex, w, hidden_transform=transform, threads=3)
        for tok in range(t):
            acc = np.float32(0.0)
            for j in range(k):
                y = o.silu_gated_mlp(x[tok:tok + 1], wg[ex[tok, j]], wu[ex[tok, j]], wd[ex[tok, j]],
                                     round_hidden_bf16=bool(transform))
                acc = np.float32(acc + np.float32(w[tok, j] * y))
            np.testing.assert_array_equal(out[tok], acc[0])
    # threads never change the result
    np.testing.assert_array_equal(o.moe_mlp(x, wg, wu, wd, ex, w, threads=1),
                                  o.moe_mlp(x, wg, wu, wd, ex, w, threads=5))


def test_moe_mlp_hidden_quantization_transform():
    rng = np.random.default_rng(24)
    t, h, inter, e, k = 3, 16, 256, 2, 1
    x = rng.standard_normal((t, h)).astype(np.float32)
    wg = (rng.standard_normal((e, inter, h)) * 0.3).astype(np.float32)
    wu = (rng.standard_normal((e, inter, h)) * 0.3).astype(np.float32)
    wd = (rng.standard_normal((e, h, inter)) * 0.3).astype(np.float32)
    ex = np.array([[0], [1], [1]], np.int32)
    w = np.ones((t, 1), np.float32)
    for transform, group in ((3, None), (5, 128)):
        out = o.moe_mlp(x, wg, wu, wd, ex, w, hidden_transform=transform, threads=1)
        for tok in range(t):
            _, hid = o.silu_gated_mlp(x[tok:tok + 1], wg[ex[tok, 0]], wu[ex[tok, 0]], wd[ex[tok, 0]],
                                      return_hidden=True)
            hb = o.bf16_decode(o.bf16_round(hid))
            q, s = o.quantize_rows(hb, group=group)
            hq = o.dequantize(q, s if group else s, mode=1 if group else 0, group=group or 0)
            np.testing.assert_array_equal(out[tok], o.dense_projection(hq, wd[ex[tok, 0]])[0])


def test_moe_mlp_bf16_y_transform():
    """Bit 3 of hidden_transform rounds each y_a to bf16 before the combine
    (the device stores y in bf16): the result equals the per-token sum over
    the k picks of w_tj * bf16(y_a) with y_a from the dense oracle, and
    differs from the fp32-y result where a rounding changes a sum."""
    rng = np.random.default_rng(25)
    t, h, inter, e, k = 5, 32, 24, 4, 2
    x = rng.standard_normal((t, h)).astype(np.float32)
    wg = (rng.standard_normal((e, inter, h)) * 0.2).astype(np.float32)
    wu = (rng.standard_normal((e, inter, h)) * 0.2).astype(np.float32)
    wd = (rng.standard_normal((e, h, inter)) * 0.2).astype(np.float32)
    ex, w = o.route_topk(rng.standard_normal((t, e)).astype(np.float32), k, o.ROUTE_TOPK_SOFTMAX)
    for transform in (8, 9, 11):
        out = o.moe_mlp(x, wg, wu, wd, ex, w, hidden_transform=transform, threads=2)
        for tok in range(t):
            acc = np.zeros(h, np.float32)
            for j in range(k):
                _, hid = o.silu_gated_mlp(x[tok:tok + 1], wg[ex[tok, j]], wu[ex[tok, j]], wd[ex[tok, j]],
                                          return_hidden=True)
                if transform & 1:
                    hid = o.bf16_decode(o.bf16_round(hid))
                if transform & 2:
                    q, sc = o.quantize_rows(hid)
                    hid = o.dequantize(q, sc)
                y = o.bf16_decode(o.bf16_round(o.dense_projection(hid, wd[ex[tok, j]])))[0]
                acc = (acc + (w[tok, j] * y).astype(np.float32)).astype(np.float32)
            np.testing.assert_array_equal(out[tok], acc)
    assert not np.array_equal(o.moe_mlp(x, wg, wu, wd, ex, w, hidden_transform=8),
                              o.moe_mlp(x, wg, wu, wd, ex, w, hidden_transform=0))

"""Pins the oracle's restatement of kernels/reference against the reference's
own known-answer tests, plus closed forms and brute force for what they leave
open. CPU only.
"""
import numpy as np
import pytest

import oracle_lib as o


def ref_limits():
    # kernels/reference/values_test.mbt:2-4
    return o.limits(max_rows=16, max_columns=32, max_elements=256)


def test_dense_projection_kat():
    # kernels/reference/operations_test.mbt:12-35: [1,2] . W^T = [1,2,3]
    w = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    x = np.array([[1, 2]], np.float32)
    out = o.dense_projection(x, w, ref_limits())
    np.testing.assert_allclose(out, [[1, 2, 3]], atol=1e-5)


def test_qkv_concat_kat():
    # kernels/reference/operations_test.mbt:63-95: Q then K then V
    x = np.array([[1, 2]], np.float32)
    q = np.array([[1, 0], [0, 1]], np.float32)
    k = np.array([[1, 1]], np.float32)
    v = np.array([[2, 0]], np.float32)
    out = o.qkv_projection(x, q, k, v, ref_limits())
    np.testing.assert_allclose(out, [[1, 2, 3, 2]], atol=1e-5)


def test_qkv_rejects_unequal_kv_width():
    # kernels/reference/basic.mbt:125-127 (QkvOutputWidth)
    x = np.ones((1, 2), np.float32)
    with pytest.raises(o.OracleError) as err:
        o.qkv_projection(x, np.ones((2, 2)), np.ones((1, 2)), np.ones((2, 2)))
    assert err.value.status == o.INVALID_SHAPE


def test_silu_gated_mlp_kat():
    # kernels/reference/operations_test.mbt:208-217: 4.3863516 +- 2e-5
    one = np.array([[1.0]], np.float32)
    out = o.silu_gated_mlp(one, np.array([[1.0]]), np.array([[2.0]]), np.array([[3.0]]),
                           lim=ref_limits())
    assert abs(float(out[0, 0]) - 4.3863516) <= 2e-5


def test_bf16_decode_kat():
    # kernels/reference/values_test.mbt:56-65: [0x80,0x3f,0x00,0xc0] -> [1, -2]
    out = o.decode_bfloat16_le(bytes([0x80, 0x3F, 0x00, 0xC0]), 1, 2, ref_limits())
    assert out.tolist() == [[1.0, -2.0]]


def test_bf16_decode_rejects_nan_and_length():
    # kernels/reference/validation_test.mbt:46-53 and :101-113
    with pytest.raises(o.OracleError) as err:
        o.decode_bfloat16_le(bytes([0xC0, 0x7F]), 1, 1, ref_limits())
    assert err.value.status == o.NON_FINITE
    with pytest.raises(o.OracleError) as err:
        o.decode_bfloat16_le(bytes([0x80, 0x3F, 0x00]), 1, 2, ref_limits())
    assert err.value.status == o.INVALID_SHAPE


def test_computed_overflow_is_rejected():
    # kernels/reference/validation_test.mbt:54-71: 3.4e38 + 3.4e38 -> NonFinite
    x = np.array([[3.4e38, 3.4e38]], np.float32)
    w = np.array([[1.0, 1.0]], np.float32)
    with pytest.raises(o.OracleError) as err:
        o.dense_projection(x, w, ref_limits())
    assert err.value.status == o.NON_FINITE


def test_projection_width_mismatch():
    # kernels/reference/validation_test.mbt:83-94 (ProjectionInputWidth)
    with pytest.raises(o.OracleError) as err:
        o.dense_projection(np.ones((1, 2)), np.ones((1, 1)), ref_limits())
    assert err.value.status == o.INVALID_SHAPE


def test_limits():
    # kernels/reference/validation_test.mbt:2-30
    with pytest.raises(o.OracleError) as err:
        o.limits(max_rows=0, max_columns=2, max_elements=4)
    assert err.value.status == o.INVALID_LIMIT
    lim = o.limits(max_rows=1, max_columns=2, max_elements=2)
    with pytest.raises(o.OracleError) as err:
        o.dense_projection(np.ones((2, 1)), np.ones((1, 1)), lim)
    assert err.value.status == o.LIMIT_EXCEEDED


def test_sequential_k_accumulation_order():
    # The reference accumulates k = 0..K-1 left to right in binary32
    # (basic.mbt:86-90). (1e8 + 1) rounds back to 1e8 in fp32, so the
    # sequential sum of [1e8, 1, -1e8, 1] is 1.0; pairwise or reversed
    # orders give 0.0 or 2.0.
    x = np.array([[1e8, 1.0, -1e8, 1.0]], np.float32)
    w = np.ones((1, 4), np.float32)
    assert o.dense_projection(x, w)[0, 0] == np.float32(1.0)
    # and the multiply is rounded before the add (no fused multiply-add):
    a = np.float32(1.0 + 2.0 ** -12)
    x = np.array([[a, -1.0]], np.float32)
    w = np.array([[a, 1.0 + 2.0 ** -11]], np.float32)
    fused = np.float64(a) * np.float64(a) - (1.0 + 2.0 ** -11)
    got = o.dense_projection(x, w)[0, 0]
    assert got == np.float32(np.float32(a * a) - np.float32(1.0 + 2.0 ** -11))
    assert got != np.float32(fused)


def test_projection_closed_forms():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 8)).astype(np.float32)
    # identity weight copies x exactly
    np.testing.assert_array_equal(o.dense_projection(x, np.eye(8, dtype=np.float32)), x)
    # a permutation weight permutes columns
    perm = rng.permutation(8)
    np.testing.assert_array_equal(o.dense_projection(x, np.eye(8, dtype=np.float32)[perm]), x[:, perm])
    # one-hot rows of x select weight columns
    w = rng.standard_normal((5, 8)).astype(np.float32)
    np.testing.assert_array_equal(o.dense_projection(np.eye(8, dtype=np.float32), w), w.T)


def test_projection_brute_force_fp64():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    w = rng.standard_normal((7, 64)).astype(np.float32)
    got = o.dense_projection(x, w)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(got, exact, rtol=0, atol=64 * 2e-6 * np.abs(exact).max())
    # small integers: every partial sum is exact, so the result is exact
    xi = rng.integers(-8, 8, (3, 33)).astype(np.float32)
    wi = rng.integers(-8, 8, (5, 33)).astype(np.float32)
    np.testing.assert_array_equal(o.dense_projection(xi, wi), (xi.astype(np.int64) @ wi.astype(np.int64).T))


def test_silu_gated_mlp_matches_fp64_and_hidden():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 16)).astype(np.float32)
    wg = rng.standard_normal((12, 16)).astype(np.float32) * 0.3
    wu = rng.standard_normal((12, 16)).astype(np.float32) * 0.3
    wd = rng.standard_normal((16, 12)).astype(np.float32) * 0.3
    out, h = o.silu_gated_mlp(x, wg, wu, wd, return_hidden=True)
    g = x.astype(np.float64) @ wg.T
    u = x.astype(np.float64) @ wu.T
    h64 = g / (1 + np.exp(-g)) * u
    np.testing.assert_allclose(h, h64, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out, h64 @ wd.T, rtol=1e-4, atol=1e-5)
    # SiLU edge values: silu(0) * u == 0, silu(-large) -> -0.0 / tiny
    assert o.silu_mul(0.0, 5.0) == 0.0
    assert abs(o.silu_mul(-100.0, 1.0)) < 1e-30
    assert o.silu_mul(50.0, 2.0) == np.float32(100.0)
    # bf16-rounded hidden mirrors a two-launch device pipeline
    out_b = o.silu_gated_mlp(x, wg, wu, wd, round_hidden_bf16=True)
    hb = o.bf16_decode(o.bf16_round(h))
    np.testing.assert_array_equal(out_b, o.dense_projection(hb, wd))


def test_qkv_equals_three_dense_calls():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 32)).astype(np.float32)
    wq = rng.standard_normal((16, 32)).astype(np.float32)
    wk = rng.standard_normal((8, 32)).astype(np.float32)
    wv = rng.standard_normal((8, 32)).astype(np.float32)
    out = o.qkv_projection(x, wq, wk, wv)
    ref = np.concatenate([o.dense_projection(x, w) for w in (wq, wk, wv)], axis=1)
    np.testing.assert_array_equal(out, ref)


def test_multithreaded_projection_is_bit_identical():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((5, 300)).astype(np.float32)
    w = rng.standard_normal((37, 300)).astype(np.float32)
    single = o.project_values(x, w)
    for threads in (1, 3, 8):
        np.testing.assert_array_equal(o.project_values_mt(x, w, threads), single)


def test_rms_norm_kat():
    # kernels/reference/operations_test.mbt:38-60: [3, 4], weight [1, 1],
    # epsilon 1e-5 -> [0.8485277, 1.1313703] within 2e-5
    out = o.rms_norm(np.array([[3, 4]], np.float32), np.ones((1, 2), np.float32), 1e-5,
                     ref_limits())
    np.testing.assert_allclose(out, [[0.8485277, 1.1313703]], atol=2e-5)


def test_rms_norm_rejections():
    # kernels/reference/basic.mbt:38-47 (NormalizationWeight, Epsilon) and
    # :59-61 (a non-finite sum of squares)
    x = np.ones((2, 4), np.float32)
    for w in (np.ones((1, 3), np.float32), np.ones((2, 4), np.float32)):
        with pytest.raises(o.OracleError) as err:
            o.rms_norm(x, w, 1e-5)
        assert err.value.status == o.INVALID_SHAPE
    for eps, status in ((float("nan"), o.NON_FINITE), (float("inf"), o.NON_FINITE),
                        (0.0, o.INVALID_SCALAR), (-1e-5, o.INVALID_SCALAR)):
        with pytest.raises(o.OracleError) as err:
            o.rms_norm(x, np.ones(4, np.float32), eps)
        assert err.value.status == status
    with pytest.raises(o.OracleError) as err:
        o.rms_norm(np.full((1, 4), 1e20, np.float32), np.ones(4, np.float32), 1e-5)
    assert err.value.status == o.NON_FINITE


def test_rms_norm_sums_squares_in_column_order():
    # x = [4096, 1 x 1023]: adding 1 to 2^24 is a tie that rounds to even, so
    # the sequential sum stays 2^24 (any pairwise or blocked order would
    # reach 2^24 + 1023 or so); then 2^24 / 1024 + 2^-10 = 16384 (another
    # tie), sqrt 128, inverse 2^-7, all exact: out = x / 128 * w.
    x = np.ones((1, 1024), np.float32)
    x[0, 0] = 4096
    w = np.linspace(0.5, 2.0, 1024, dtype=np.float32)
    out = o.rms_norm(x, w, 2.0 ** -10)
    np.testing.assert_array_equal(out, (x / np.float32(128)) * w)


def test_rms_norm_closed_form():
    # against the float64 formula: each row within a few fp32 ulps of
    # x / sqrt(mean(x^2) + eps) * w, and the weight applied per column
    rng = np.random.default_rng(77)
    x = rng.standard_normal((5, 384)).astype(np.float32)
    w = rng.uniform(0.2, 3.0, 384).astype(np.float32)
    out = o.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(out, ref, rtol=2e-6, atol=0)
    # a row of equal magnitudes normalizes to +-1 (times w) up to epsilon
    out = o.rms_norm(np.full((1, 256), -3.0, np.float32), np.ones(256, np.float32), 1e-6)
    np.testing.assert_allclose(out, -1.0, rtol=1e-6)

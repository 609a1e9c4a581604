"""The GPU tests' parity helpers, on the CPU: each excuse they grant must be
one the summation bounds allow, and a planted mistake must fail."""
import numpy as np
import pytest

import oracle_lib as o
from parity import (abs_sum, combine, combine_tol, gamma, moved_codes_explained, parity,
                    swiglu_midpoint_tol)


def bf16(v):
    return o.bf16_round(np.asarray(v, np.float32))


def padded(gpu_value, ref_value, tol=None):
    """One element under test beside 1023 exact ones (so the relative L2 bar
    holds and only the max-abs bar decides); tol padded with zeros."""
    ref = np.full(1024, 6.0, np.float32)
    ref[0] = ref_value
    gpu = bf16(ref)
    gpu[0] = bf16([gpu_value])[0]
    if tol is None:
        return gpu, ref
    t = np.zeros(1024)
    t[0] = tol
    return gpu, ref, t


def test_exact_and_small_errors_pass():
    r = np.linspace(-3, 3, 64, dtype=np.float32)
    parity(bf16(r), r)
    parity(bf16(r + 1e-4), r)


def test_one_ulp_flip_needs_a_bound():
    # 6.0 + half a bf16 ulp (ulp at [4, 8) is 2^-5): the oracle rounds to
    # even (6.0), a GPU sum a hair above the midpoint rounds to 6.03125
    mid = 6.0 + 2.0 ** -6
    gpu, ref, s = padded(6.03125, mid - 1e-6, 64.0)
    assert o.bf16_decode(bf16(ref[:1]))[0] == 6.0
    with pytest.raises(AssertionError, match="max_abs"):
        parity(gpu, ref)
    # K = 4096 terms with S = 64: 2 gamma_K S ~ 3e-2 covers the 1e-6 gap
    parity(gpu, ref, k=4096, s_abs=s)
    # S so small that the bound cannot reach the midpoint
    with pytest.raises(AssertionError, match="max_abs"):
        parity(gpu, ref, k=4096, s_abs=s * 1e-6)


def test_two_ulp_difference_is_not_a_rounding_flip():
    gpu, ref, s = padded(6.0625, 6.0, 1.0)    # two bf16 ulp away
    with pytest.raises(AssertionError, match="max_abs"):
        parity(gpu, ref, k=4096, s_abs=s)


def test_value_tol_admits_only_the_stated_distance():
    gpu, ref, t = padded(3.03125, 3.0, 0.03125)   # two ulp of [2, 4)
    parity(gpu, ref, value_tol=t)
    with pytest.raises(AssertionError, match="max_abs"):
        parity(gpu, ref, value_tol=t * 0.3)


def test_rel_l2_has_no_exception():
    r = np.full(16, 6.0, np.float32)
    with pytest.raises(AssertionError, match="rel_l2"):
        parity(bf16(r * 1.01), r, value_tol=np.full(16, 1.0))


def test_combine_matches_sequential_fp32():
    rng = np.random.default_rng(0)
    w = rng.random((5, 2)).astype(np.float32)
    y = rng.standard_normal((5, 2, 7)).astype(np.float32)
    yb = o.bf16_decode(bf16(y))
    want = np.zeros((5, 7), np.float32)
    for t in range(5):
        for n in range(7):
            a = np.float32(0)
            for j in range(2):
                a = np.float32(a + np.float32(w[t, j] * yb[t, j, n]))
            want[t, n] = a
    np.testing.assert_array_equal(combine(w, y), want)


def test_combine_tol_flags_only_ambiguous_y():
    k = 4096
    s = np.array([[[16.0, 16.0]]])            # 2 gamma_K S ~ 7.8e-3
    # y near the [8,16) midpoint 8 + 2^-5 (ambiguous), and y = 8 exactly
    y = np.array([[[8.0 + 2.0 ** -5 - 1e-4, 8.0]]], np.float32)
    w = np.array([[0.5]])
    tol = combine_tol(w, y, s, k)
    assert tol[0, 0] >= 0.5 * 2.0 ** -4       # w ulp(y) for the ambiguous one
    assert tol[0, 1] < 1e-4                   # only the fp32 rounding term
    # with a tiny S neither is ambiguous
    tol = combine_tol(w, y, s * 1e-6, k)
    assert (tol < 1e-4).all()


def test_swiglu_tol_grows_with_the_summation_bound():
    g = np.array([1.0, 1.0])
    u = np.array([2.0, 2.0])
    t = swiglu_midpoint_tol(g, u, np.array([10.0, 1000.0]), np.array([10.0, 1000.0]), 4096)
    assert t[1] > 50 * t[0] > 0
    assert t[0] >= 1.1 * 2 * gamma(4096) * 10


def test_abs_sum():
    x = np.array([[1.0, -2.0]])
    w = np.array([[3.0, 4.0], [-1.0, 0.5]])
    np.testing.assert_array_equal(abs_sum(x, w), [[11.0, 2.0]])


def codes_case():
    rng = np.random.default_rng(3)
    h = rng.standard_normal((4, 256)).astype(np.float32)
    q, s = o.quantize_rows(o.bf16_decode(bf16(h)))
    return h, q, s


def test_moved_codes_explained_accepts_boundary_moves():
    h, q, s = codes_case()
    tol = np.full(h.shape, 1e-3)
    # the GPU's h one bf16 ulp up at element (1, 7): within 2 tol + ulp
    hg = o.bf16_decode(bf16(h)).copy()
    i = (1, 7)
    mag = abs(hg[i])
    hg[i] += np.sign(hg[i]) * 2.0 ** (np.floor(np.log2(mag)) - 7)
    qg, sg = o.quantize_rows(hg)
    assert moved_codes_explained(h, bf16(hg), tol, q, qg, s, sg, "case") >= 0


def test_moved_codes_explained_rejects_a_planted_error():
    h, q, s = codes_case()
    tol = np.full(h.shape, 1e-6)
    hg = o.bf16_decode(bf16(h)).copy()
    # a wrong value far beyond the bound, not the row's largest element
    row = hg[2]
    i = int(np.argmin(np.abs(row)))
    row[i] = row[i] + 0.5
    qg, sg = o.quantize_rows(hg)
    if (sg == s).all() and (qg == q).all():
        pytest.skip("the planted error did not move a code")
    with pytest.raises(AssertionError):
        moved_codes_explained(h, bf16(hg), tol, q, qg, s, sg, "case")

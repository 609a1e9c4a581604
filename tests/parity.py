"""The parity bar shared by the GPU tests.

relative L2 <= 1e-3 and max-abs <= 2e-2 between the bf16
GPU output and the oracle output rounded to bf16 (RNE).

Rounding-boundary flips. The oracle sums K products sequentially in fp32;
the GPU sums the same products in another order. Any fp32 summation order
is within gamma_K * S of the exact sum, where S = sum_k |x_k w_k| and
gamma_K = K u / (1 - K u), u = 2^-24 (Higham, Accuracy and Stability of
Numerical Algorithms, 2nd ed., eq. 4.4). When the exact result lies that
close to a bf16 rounding midpoint, the two fp32 results can round to
neighbouring bf16 values: a one-ulp difference that is the correct rounding
of an equally valid fp32 sum. At K = 14336 with |y| in [4, 8) one bf16 ulp is
0.03125 > 2e-2, so such flips are the only way an order-independent kernel
can exceed the max-abs bar. `parity` therefore excuses an element from the
max-abs bar only when the caller supplied a bound D on the distance between
the GPU's fp32 result and the oracle's, and the GPU's bf16 value is the
rounding of a value within D of the oracle's fp32 value:
|gpu - oracle32| <= D + ulp(gpu) / 2. With S (abs_sum) D = 2 gamma_K S: for
a plain dot product that admits only the neighbouring bf16 value, and only
when the oracle's fp32 value lies within 2 gamma_K S of the midpoint.
Everything else must meet the bar, the relative L2 bar has no exception, and
the number of excused elements is printed.

For an output that is not a plain dot product the caller passes the bound
itself: `midpoint_tol`, the largest distance from the exact value that
either side's fp32 result may have (D = 2 midpoint_tol; swiglu_midpoint_tol
derives it for SwiGLU h = silu(g) u from the summation bounds of g and u),
or `value_tol`, D itself (combine_tol derives it for the routing-weighted
sum of bf16 y rows, where one flipped y moves the sum by w ulp(y), which
can be several ulp of the sum).
"""
import numpy as np

import oracle_lib as o

REL_L2 = 1e-3
MAX_ABS = 2e-2
U32 = 2.0 ** -24


def abs_sum(x_values: np.ndarray, w_values: np.ndarray) -> np.ndarray:
    """S = sum_k |x[m,k] w[n,k]| per output element, in float64."""
    return np.abs(x_values.astype(np.float64)) @ np.abs(w_values.astype(np.float64)).T


def gamma(k: int) -> float:
    return k * U32 / (1 - k * U32)


def swiglu_midpoint_tol(g, u, s_g, s_u, k: int) -> np.ndarray:
    """Bound on |computed h - exact h| for h = silu(g) u, where g and u are
    K-term fp32 dot products with absolute-value sums s_g, s_u: each is
    within gamma_K S of its exact value in any summation order, |d silu /
    dg| <= 1.1 and |silu(g)| <= |g| + 0.3, and the silu evaluation itself
    (expf and a division, or exp2 and a reciprocal) adds at most a few fp32
    ulp of h, taken as 16 ulp."""
    g = np.abs(np.asarray(g, np.float64))
    u = np.abs(np.asarray(u, np.float64))
    dg = gamma(k) * np.asarray(s_g, np.float64)
    du = gamma(k) * np.asarray(s_u, np.float64)
    silu = g + 0.3
    h = silu * u
    return 1.1 * (u + du) * dg + (silu + 1.1 * dg) * du + 16 * U32 * h


def parity(gpu_bits, ref32, k: int = 0, s_abs=None, rel_l2=REL_L2, max_abs=MAX_ABS, label="",
           midpoint_tol=None, value_tol=None):
    g = o.bf16_decode(gpu_bits).astype(np.float64)
    r16 = o.bf16_round(ref32)
    r = o.bf16_decode(r16).astype(np.float64)
    assert g.shape == r.shape, label
    assert np.isfinite(g).all(), f"{label}: non-finite GPU output"
    if g.size == 0:
        return
    err = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)
    diff = np.abs(g - r)
    over = diff > max_abs
    excused = np.zeros_like(over)
    if over.any() and ((s_abs is not None and k > 0) or midpoint_tol is not None
                       or value_tol is not None):
        tol = 0.0
        if s_abs is not None and k > 0:
            tol = tol + 2 * gamma(k) * np.asarray(s_abs)
        if midpoint_tol is not None:
            tol = tol + 2 * np.asarray(midpoint_tol)
        if value_tol is not None:
            tol = tol + np.asarray(value_tol)
        # the GPU's bf16 value is the rounding of its fp32 value, which lies
        # within half an ulp of the GPU value's binade (the widest case)
        mag = np.abs(g)
        ulp = np.exp2(np.floor(np.log2(np.where(mag > 0, mag, 1.0))) - 7) * (mag > 0)
        excused = over & (np.abs(g - ref32.astype(np.float64)) <= tol + ulp / 2)
    strict = np.where(excused, 0.0, diff)
    mx = float(strict.max())
    print(f"{label}: rel_l2={err:.3e} max_abs={mx:.3e} boundary_flips={int(excused.sum())}"
          f"/{g.size} max_abs_incl_flips={float(diff.max()):.3e}", flush=True)
    assert err <= rel_l2, f"{label}: rel_l2 {err}"
    assert mx <= max_abs, f"{label}: max_abs {mx}"


def bf16_ordinal(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns as integers in value order (adjacent finite values
    differ by 1; +0 and -0 both map to 0)."""
    b = np.asarray(bits).astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)


def moved_codes_explained(h_oracle, h_gpu_bits, h_tol, q_oracle, q_gpu, s_oracle, s_gpu, label):
    """The e4m3 codes of a re-quantized bf16 h (one row per assignment) that
    differ between the oracle and the GPU must be rounding-boundary moves.
    h_oracle: the oracle's fp32 h; h_gpu_bits: the GPU's bf16 h; h_tol: the
    bound on either side's distance from the exact h (swiglu_midpoint_tol).
    An element is explained when the two bf16 values are within 2 h_tol plus
    one bf16 ulp of each other (both fp32 values lie within h_tol of the
    exact h, and each rounding moves at most half an ulp). Every moved code
    must be explained, or lie in a row whose scale moved because the row's
    largest |h| is explained on both sides (a moved scale can move any code
    of the row across its boundary). Returns the number of moved codes."""
    hb_o = o.bf16_decode(o.bf16_round(h_oracle)).astype(np.float64)
    hb_g = o.bf16_decode(h_gpu_bits).astype(np.float64)
    mag = np.maximum(np.abs(hb_o), np.abs(hb_g))
    ulp = np.exp2(np.floor(np.log2(np.where(mag > 0, mag, 1.0))) - 7)
    explained = np.abs(hb_o - hb_g) <= 2 * np.asarray(h_tol, np.float64) + ulp
    moved = q_oracle != q_gpu
    rows = len(q_oracle)
    scale_moved = np.any(s_oracle.reshape(rows, -1) != s_gpu.reshape(rows, -1), axis=1)
    for r in np.flatnonzero(scale_moved):
        for side in (hb_o[r], hb_g[r]):
            i = int(np.argmax(np.abs(side)))
            assert explained[r, i], f"{label}: row {r}'s scale moved with its amax beyond the bound"
    unexplained = moved & ~explained & ~scale_moved[:, None]
    assert not unexplained.any(), (f"{label}: {int(unexplained.sum())} h codes moved where the two h "
                                   f"values differ beyond the summation bound")
    return int(moved.sum())


def combine(weights: np.ndarray, y_rows: np.ndarray) -> np.ndarray:
    """out_t = sum_j w_tj * bf16(y_(t,j)), j ascending, each product and sum
    rounded to fp32 (the combine's arithmetic, from bf16 y). y_rows:
    [tokens, k, hidden] fp32."""
    acc = np.zeros((y_rows.shape[0], y_rows.shape[2]), np.float32)
    yb = o.bf16_decode(o.bf16_round(y_rows))
    for j in range(y_rows.shape[1]):
        acc = (acc + (weights[:, j:j + 1] * yb[:, j]).astype(np.float32)).astype(np.float32)
    return acc


def combine_tol(weights: np.ndarray, y32: np.ndarray, s_y: np.ndarray, k: int) -> np.ndarray:
    """value_tol for a combine over bf16 y (`combine`): the largest distance
    between the GPU's fp32 sum and the oracle's. y_(t,j) is a K-term fp32 dot
    product within gamma_K S of the exact value in any summation order, so
    the two sides' bf16 roundings of it can differ only when the oracle's
    fp32 value lies within 2 gamma_K S of a bf16 rounding midpoint, and then
    by one bf16 ulp of y; each such y moves the sum by w_tj ulp(y). The sum's
    own fp32 roundings (k products and k additions) add 2 k u sum_j |w y|.
    y32, s_y: [tokens, picks, hidden] (the oracle's fp32 y and its |h||w|
    sums)."""
    y = np.asarray(y32, np.float64)
    yb = o.bf16_decode(o.bf16_round(np.asarray(y32, np.float32))).astype(np.float64)
    mag = np.maximum(np.abs(y), np.abs(yb))
    ulp = np.exp2(np.floor(np.log2(np.where(mag > 0, mag, 1.0))) - 7)
    ambiguous = np.abs(y - yb) >= ulp / 2 - 2 * gamma(k) * np.asarray(s_y, np.float64)
    w = np.abs(np.asarray(weights, np.float64))[:, :, None]
    picks = y.shape[1]
    return np.sum(w * np.where(ambiguous, ulp, 0.0), axis=1) + 2 * picks * U32 * np.sum(w * (np.abs(y) + ulp), axis=1)

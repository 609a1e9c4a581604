"""GPU parity of the fused RmsNorm + per-token e4m3 quantizer
(lf_fp8_rms_norm_quant_rows_eps*) against the oracle: oracle.rms_norm
(kernels/reference/basic.mbt:32-68, sequential fp32) followed by the
oracle's per-token quantizer.

The kernel reduces the sum of squares across a wavefront, the reference sums
it in column order. Where every partial sum is exact (activations that are
multiples of 1/4 in [-4, 4]: squares are multiples of 1/16, sums stay below
2^17), both orders give the same fp32 value and the codes and scales must be
bit-identical to the oracle's. On general inputs the tests check (1) bit
identity with the reference formula applied to the sum of squares in the
kernel's documented order, and (2) closeness to the sequential-order oracle
within the fp32 summation error bound.
"""
import numpy as np
import pytest

import oracle_lib as o
from lunaflux_amd import synth
from parity import abs_sum, parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from lunaflux_amd.fp8 import ProjectionRuntime
    return ProjectionRuntime(0)


def oracle_rms_quant(x_bits, g_bits, eps):
    y = o.rms_norm(o.bf16_decode(x_bits), o.bf16_decode(g_bits), eps)
    q, s = o.quantize_rows(y)
    return q, s.reshape(-1), y


def norm_weight(rng, k):
    return synth.bf16_bits(rng.uniform(0.25, 2.0, k).astype(np.float32))


def consumer_weight(rt, rng, k, n=128):
    q, s = synth.weight(rng, n, k)
    return q, s, rt.upload_weight(q, s)


@pytest.mark.parametrize("k,m,max_rows,eps", [
    (4096, 37, 64, 1e-5), (8192, 9, 16, 1e-5), (1024, 130, 256, 1e-6), (384, 5, 8, 1e-6),
    (4352, 64, 64, 1e-5),
])
def test_rms_norm_quant_bit_exact_on_exact_sums(rt, k, m, max_rows, eps):
    rng = np.random.default_rng(500 + k + m)
    x = synth.bf16_bits(rng.integers(-16, 17, (m, k)).astype(np.float32) / 4)
    x[0, :] = 0  # a zero row: zero codes, scale 0
    g = norm_weight(rng, k)
    _, _, w = consumer_weight(rt, rng, k)
    codes, scales = rt.rms_norm_quant(x, g, w, eps, max_tokens=max_rows)
    q_ref, s_ref, _ = oracle_rms_quant(x, g, eps)
    assert np.array_equal(scales.view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(codes, q_ref)
    assert not codes[0].any() and scales[0] == 0


def wave_order_sum_of_squares(xf):
    """Sum of squares per row in the kernel's order, in fp32: lane l of the
    wavefront holds 16-byte chunks l, l + 64, ... (8 columns each) and sums
    their squares in column order, then a xor butterfly over offsets 32, 16,
    ..., 1 adds lane pairs (each pair gets the same value: fp32 addition is
    commutative)."""
    m, k = xf.shape
    chunks = k // 8
    per_lane = -(-chunks // 64)
    lanes = np.zeros((m, 64), np.float32)
    for c in range(per_lane):
        for j in range(8):
            idx = np.arange(64) + 64 * c
            live = idx < chunks
            col = np.where(live, idx * 8 + j, 0)
            sq = np.where(live, xf[:, col] * xf[:, col], np.float32(0)).astype(np.float32)
            lanes = (lanes + sq).astype(np.float32)
    for off in (32, 16, 8, 4, 2, 1):
        lanes = (lanes + lanes[:, np.arange(64) ^ off]).astype(np.float32)
    return lanes[:, 0]


def e4m3_step(v):
    """Distance between consecutive e4m3 values around |v| (v in [0, 448])."""
    v = np.maximum(np.abs(v), 2.0 ** -6)
    return 2.0 ** (np.floor(np.log2(v)) - 3)


@pytest.mark.parametrize("k,m,eps", [(4096, 200, 1e-5), (8192, 64, 1e-6), (2048, 33, 1e-5)])
def test_rms_norm_quant_random_rows(rt, k, m, eps):
    rng = np.random.default_rng(700 + k + m)
    x = synth.activations(rng, m, k)
    g = norm_weight(rng, k)
    _, _, w = consumer_weight(rt, rng, k)
    codes, scales = rt.rms_norm_quant(x, g, w, eps, max_tokens=m)

    # (1) Bit for bit against the reference formula evaluated on the sum of
    # squares taken in the kernel's order (each later step in fp32 with IEEE
    # rounding: numpy's float32 sqrt and division are correctly rounded, the
    # quantizer is the oracle's).
    xf, gf = o.bf16_decode(x), o.bf16_decode(g)
    ss = wave_order_sum_of_squares(xf)
    inv = (np.float32(1) / np.sqrt((ss / np.float32(k) + np.float32(eps)).astype(np.float32))
           ).astype(np.float32)
    y = ((xf * inv[:, None]).astype(np.float32) * gf).astype(np.float32)
    q_w, s_w = o.quantize_rows(y)
    assert np.array_equal(scales.view(np.uint32), s_w.reshape(-1).view(np.uint32))
    assert np.array_equal(codes, q_w)

    # (2) Against the reference's sequential sum. Any two fp32 summation
    # orders of K non-negative terms lie within gamma_K = K u / (1 - K u)
    # (u = 2^-24) of the exact sum (Higham, eq. 4.4), so inv, and the scale
    # amax(y) / 448 with it, differ by at most ~gamma_K relatively (half of
    # the 2 gamma_K between the two sums, through the square root), plus a
    # few roundings. The codes y * (448 / amax) do not depend on inv to first
    # order, so they agree except at rounding midpoints.
    q_ref, s_ref, y_ref = oracle_rms_quant(x, g, eps)
    u = 2.0 ** -24
    gamma = k * u / (1 - k * u)
    np.testing.assert_allclose(scales, s_ref, rtol=gamma + 8 * u, atol=0)
    diff = codes != q_ref
    if diff.any():
        dq, dr = o.e4m3_decode(codes[diff]), o.e4m3_decode(q_ref[diff])
        assert np.all(np.abs(dq - dr) <= e4m3_step(np.maximum(np.abs(dq), np.abs(dr))) * 1.0001)
        ratio = np.repeat((1.0 / s_ref.astype(np.float64))[:, None], k, 1)[diff]
        scaled = np.abs(y_ref[diff].astype(np.float64) * ratio)
        mid = (np.abs(dq) + np.abs(dr)) / 2
        assert np.all(np.abs(scaled - mid) <= 16 * u * mid), "a flip away from a rounding midpoint"
    # bf16 x times bf16 g has few significant bits, so many scaled values fall
    # exactly on an e4m3 midpoint, where either order's last-bit difference
    # decides the tie: about 1e-4 of the codes on N(0, 1) rows (measured).
    assert diff.mean() < 1e-3, f"{diff.sum()} codes differ"


def test_rms_norm_quant_feeds_the_w8a8_gemm(rt):
    """RmsNorm -> e4m3 rows -> W8A8 dense GEMM (a Llama-3 K-V width) through
    one xq region: the GEMM against the oracle on the rows the norm wrote, at
    the parity bar; the whole chain against oracle dense(dequant(quantize(
    rms_norm(x)))) within 1e-2, since a code that flips at a rounding
    midpoint (the sum-of-squares order) moves one input by an e4m3 step."""
    from lunaflux_amd.fp8 import _region, act_quant_bytes
    rng = np.random.default_rng(811)
    m, k, n, mt = 300, 4096, 1024, 512
    x = synth.activations(rng, m, k)
    g = norm_weight(rng, k)
    q, s, w = consumer_weight(rt, rng, k, n)
    ctx = rt.context
    xa = ctx.upload(np.concatenate([x, np.zeros((mt - m, k), np.uint16)]))
    ga = ctx.upload(g)
    xq = ctx.allocate(act_quant_bytes(mt, k))
    ya = ctx.allocate(mt * n * 2)
    counts = rt.step_counts(m)
    norm = rt.bind_rms_norm_quant(counts, _region(xa, alignment=256), _region(ga), w,
                                  _region(xq, alignment=256), mt, 1e-5)
    gemm = rt.bind_dense_quantized(counts, _region(xq, alignment=256), w,
                                   _region(ya, alignment=256), mt)
    norm.launch(rt.stream, synchronous=False)
    gemm.launch(rt.stream, synchronous=True)
    y = ya.read(np.uint16, (m, n))
    codes = xq.read(np.uint8, (m, k))
    scales = xq.read(np.float32, (m,), offset=(m * k + 255) // 256 * 256)
    wr = o.dequantize(q, s)
    xr = o.dequantize(codes, scales)
    parity(y, o.dense_projection(xr, wr), k=k, s_abs=abs_sum(xr, wr),
           label="w8a8 dense on the norm's rows")
    q_ref, s_ref, _ = oracle_rms_quant(x, g, 1e-5)
    ref = o.dense_projection(o.dequantize(q_ref, s_ref), wr)
    got = o.bf16_decode(y).astype(np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-2


def test_rms_norm_quant_zero_rows(rt):
    rng = np.random.default_rng(3)
    _, _, w = consumer_weight(rt, rng, 512)
    codes, scales = rt.rms_norm_quant(np.zeros((0, 512), np.uint16), norm_weight(rng, 512), w,
                                      1e-5, max_tokens=16)
    assert codes.shape == (0, 512) and scales.shape == (0,)

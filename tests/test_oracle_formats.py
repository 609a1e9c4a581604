"""Pins the oracle's FP8 / bf16 formats and quantizers, which the reference
does not have, against an independent library (torch's float8_e4m3fn and
bfloat16 casts on the CPU), closed-form special cases and invariants. CPU only.
"""
import numpy as np
import pytest

import oracle_lib as o


def torch_e4m3_encode(values: np.ndarray) -> np.ndarray:
    import torch

    # torch returns NaN above 480 instead of saturating; clamp first.
    t = torch.from_numpy(np.clip(values.astype(np.float32), -448.0, 448.0))
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_decode_all_codes_match_torch():
    import torch

    codes = np.arange(256, dtype=np.uint8)
    ours = o.e4m3_decode(codes)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    nan = np.isnan(theirs)
    assert nan.sum() == 2 and np.isnan(ours[nan]).all()
    assert (np.flatnonzero(nan) == [0x7F, 0xFF]).all()
    np.testing.assert_array_equal(ours[~nan], theirs[~nan])
    # closed-form anchors of the OCP E4M3 format
    assert ours[0x7E] == 448.0 and ours[0xFE] == -448.0
    assert ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6
    assert ours[0x38] == 1.0 and ours[0x80] == 0.0 and np.signbit(ours[0x80])


def test_e4m3_encode_anchors():
    cases = {
        464.0: 0x7E,      # tie between 448 and 480 goes to even (448)
        3.3: 0x45,        # 3.25 = 1.101b * 2^1
        2.0 ** -10: 0x00,  # half of the smallest subnormal ties to zero
        1.5 * 2.0 ** -10: 0x01,
        1e9: 0x7E,         # saturates
        -1e9: 0xFE,
        float("inf"): 0x7E,
        -0.0: 0x80,
        448.0: 0x7E,
        1.0: 0x38,
    }
    for value, code in cases.items():
        assert o.e4m3_encode(np.array([value], np.float32))[0] == code, value
    assert o.e4m3_encode(np.array([np.nan], np.float32))[0] & 0x7F == 0x7F


def test_e4m3_encode_exhaustive_bf16_patterns_match_torch():
    bits = np.arange(65536, dtype=np.uint32)
    values = (bits << 16).view(np.float32)
    values = values[np.isfinite(values)]
    for scale in (1.0, 448.0 / 3.0, 2.0 ** -7, 1.0 / 0.02):
        scaled = (values * np.float32(scale)).astype(np.float32)
        scaled = scaled[np.isfinite(scaled)]
        np.testing.assert_array_equal(o.e4m3_encode(scaled), torch_e4m3_encode(scaled))


def test_e4m3_encode_random_fp32_match_torch():
    rng = np.random.default_rng(11)
    raw = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    values = raw.view(np.float32)
    values = values[np.isfinite(values)]
    np.testing.assert_array_equal(o.e4m3_encode(values), torch_e4m3_encode(values))


def test_e4m3_roundtrip_is_identity_on_codes():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)
    np.testing.assert_array_equal(o.e4m3_encode(o.e4m3_decode(codes)), codes)


def test_bf16_rne_matches_torch():
    import torch

    rng = np.random.default_rng(12)
    raw = rng.integers(0, 2 ** 32, 1_000_000, dtype=np.uint64).astype(np.uint32)
    values = raw.view(np.float32)
    values = values[~np.isnan(values)]
    theirs = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(o.bf16_round(values), theirs)
    # ties to even, and the decode is the high half of a binary32
    assert o.bf16_round(np.array([1.0 + 2.0 ** -8], np.float32))[0] == 0x3F80
    assert o.bf16_round(np.array([1.0 + 3 * 2.0 ** -8], np.float32))[0] == 0x3F82
    assert o.bf16_decode(np.array([0xC000], np.uint16))[0] == -2.0


def test_quantize_rows_invariants_and_independent_restatement():
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    w[5] = 0.0  # an all-zero row gets scale 0 and zero codes
    q, s = o.quantize_rows(w)
    assert s[5] == 0.0 and (q[5] == 0).all()
    amax = np.abs(w).max(axis=1)
    nz = amax > 0
    np.testing.assert_array_equal(s[nz], (amax[nz] / np.float32(448.0)).astype(np.float32))
    # the absmax element of each row encodes as +-448
    arg = np.abs(w).argmax(axis=1)
    assert (q[np.arange(64)[nz], arg[nz]] & 0x7F == 0x7E).all()
    assert (q & 0x7F != 0x7F).all()
    # independent restatement through torch's cast
    ratio = (np.float32(448.0) / np.where(nz, amax, 1)).astype(np.float32)
    expect = torch_e4m3_encode((w * ratio[:, None]).astype(np.float32))
    expect[~nz] = 0
    np.testing.assert_array_equal(q, expect)
    # dequantization error is at most half an e4m3 step times the scale
    deq = o.dequantize(q, s)
    rel = np.abs(deq - w) / np.where(nz, s, 1)[:, None]
    assert rel.max() <= 16.0 + 1e-3  # half step at the top binade is 16
    np.testing.assert_array_equal(deq, (o.e4m3_decode(q) * s[:, None]).astype(np.float32))


def test_quantize_groups_and_blocks():
    rng = np.random.default_rng(14)
    x = rng.standard_normal((8, 384)).astype(np.float32)
    qg, sg = o.quantize_rows(x, group=128)
    assert sg.shape == (8, 3)
    for g in range(3):
        qq, ss = o.quantize_rows(x[:, 128 * g:128 * (g + 1)])
        np.testing.assert_array_equal(qg[:, 128 * g:128 * (g + 1)], qq)
        np.testing.assert_array_equal(sg[:, g], ss)
    w = (rng.standard_normal((300, 260)) * 0.02).astype(np.float32)
    qb, sb = o.quantize_blocks(w, 128)
    assert sb.shape == (3, 3)
    for rb in range(3):
        for cb in range(3):
            blk = w[128 * rb:128 * (rb + 1), 128 * cb:128 * (cb + 1)]
            assert sb[rb, cb] == np.float32(np.abs(blk).max() / np.float32(448.0))
    deq = o.dequantize(qb, sb, mode=2, group=128)
    scale_map = np.repeat(np.repeat(sb, 128, 0), 128, 1)[:300, :260]
    np.testing.assert_array_equal(deq, (o.e4m3_decode(qb) * scale_map).astype(np.float32))
    np.testing.assert_array_equal(o.dequantize(qg, sg, mode=1, group=128),
                                  (o.e4m3_decode(qg) * np.repeat(sg, 128, 1)).astype(np.float32))


def test_quantize_rejects_bad_group():
    with pytest.raises(o.OracleError):
        o.quantize_rows(np.ones((2, 100), np.float32), group=64)

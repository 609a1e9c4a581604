"""Seeded synthetic inputs for the FP8 path (no checkpoints or datasets are
available offline): bf16 activations drawn from N(0, 1), weights drawn from
N(0, std) and quantized to OCP e4m3 with fp32 scales, and MoE router logits.

The quantizer is the one a synthetic FP8 checkpoint is materialized with:
  amax = max |w| over the scale group; ratio = 448 / amax (fp32);
  q = e4m3_rne_saturate(w * ratio); scale = amax / 448; amax == 0 -> q = 0,
  scale = 0.
It is vectorized numpy; tests check it bit-exactly against the independent
C restatement used as the oracle.
"""
from __future__ import annotations

import numpy as np


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(values, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def bf16_values(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_encode(values: np.ndarray) -> np.ndarray:
    """fp32 -> OCP e4m3 codes, round to nearest even, saturating at +-448."""
    u = np.ascontiguousarray(values, np.float32).view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint8)
    a = u & np.uint32(0x7FFFFFFF)
    with np.errstate(over="ignore", invalid="ignore"):
        # only meaningful below 2^-6, where the product is < 8; clip the rest
        scaled = np.minimum(a.view(np.float32) * np.float32(512.0), np.float32(8.0))
        sub = np.rint(np.nan_to_num(scaled)).astype(np.uint8)
    a64 = a.astype(np.uint64)
    r = (a64 + 0x7FFFF + ((a64 >> 20) & 1)) & 0xFFF00000
    exponent = (r >> 23).astype(np.int64) - 120
    normal = ((exponent << 3) | ((r >> 20) & 7).astype(np.int64)) & 0x7F
    code = np.where(a < 0x3C800000, sub, normal.astype(np.uint8))
    code = np.where(a >= 0x43E00000, np.uint8(0x7E), code)
    code = np.where(a > 0x7F800000, np.uint8(0x7F), code)
    return (code | sign).astype(np.uint8)


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(codes, np.uint8).astype(np.int32)
    exponent = (c >> 3) & 15
    mantissa = c & 7
    value = np.where(exponent == 0, np.ldexp(mantissa.astype(np.float64), -9),
                     np.ldexp((8 + mantissa).astype(np.float64), exponent - 10))
    value = np.where((c & 0x7F) == 0x7F, np.nan, value)
    return np.where(c & 0x80, -value, value).astype(np.float32)


def quantize_rows(x: np.ndarray, group: int | None = None):
    """Per-row (group=None) or per-row-per-group quantization.
    Returns (codes like x, scales [rows] or [rows, columns/group])."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    g = cols if group is None else group
    if cols % g:
        raise ValueError("columns must be a multiple of the group")
    blocks = x.reshape(rows, cols // g, g)
    amax = np.abs(blocks).max(axis=2)
    zero = amax == 0
    ratio = (np.float32(448.0) / np.where(zero, np.float32(1.0), amax)).astype(np.float32)
    q = e4m3_encode((blocks * ratio[:, :, None]).astype(np.float32))
    q[zero] = 0
    scale = np.where(zero, np.float32(0.0), (amax / np.float32(448.0)).astype(np.float32))
    q = q.reshape(rows, cols)
    return q, (scale[:, 0].copy() if group is None else scale.astype(np.float32))


def quantize_blocks(w: np.ndarray, block: int = 128):
    """128 x 128 block quantization; rows and columns multiples of block."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    if rows % block or cols % block:
        raise ValueError("dimensions must be multiples of the block")
    tiles = w.reshape(rows // block, block, cols // block, block)
    amax = np.abs(tiles).max(axis=(1, 3))
    zero = amax == 0
    ratio = (np.float32(448.0) / np.where(zero, np.float32(1.0), amax)).astype(np.float32)
    q = e4m3_encode((tiles * ratio[:, None, :, None]).astype(np.float32))
    q[np.broadcast_to(zero[:, None, :, None], q.shape)] = 0
    scale = np.where(zero, np.float32(0.0), (amax / np.float32(448.0)).astype(np.float32))
    return q.reshape(rows, cols), scale.astype(np.float32)


def activations(rng: np.random.Generator, rows: int, columns: int) -> np.ndarray:
    """bf16 bits of N(0, 1) activations."""
    return bf16_bits(rng.standard_normal((rows, columns), dtype=np.float32))


def weight(rng: np.random.Generator, rows: int, columns: int, std: float = 0.02,
           block: int | None = None):
    """(codes [rows, columns], scales) of N(0, std) weights; per-channel
    scales unless block is given."""
    w = (rng.standard_normal((rows, columns), dtype=np.float32) * np.float32(std)).astype(np.float32)
    return quantize_blocks(w, block) if block else quantize_rows(w)

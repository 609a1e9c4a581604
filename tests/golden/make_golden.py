"""Writes the golden fixtures under tests/golden/ with the CPU oracle.

config1.npz: one FP8 projection y = x (s * W)^T with
M=4, K=512, N=1536; x bf16 from N(0,1); W from N(0,0.02) quantized to OCP e4m3
with per-output-channel fp32 absmax scales; fp32 accumulation (the oracle's
sequential-K loop over dequantized weights); seed 20261201.
Stored: x (bf16 bits), q (e4m3 codes), s (scales), y32 (oracle fp32), y16
(oracle rounded to bf16). The reference cannot be executed here (MoonBit,
no toolchain), so these vectors come from the oracle, whose own arithmetic is
pinned by the reference's known-answer tests (tests/test_oracle_*.py).

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle_lib as o  # noqa: E402

SEED = 20261201


def config1():
    rng = np.random.default_rng(SEED)
    m, k, n = 4, 512, 1536
    x32 = rng.standard_normal((m, k), dtype=np.float32)
    x = o.bf16_round(x32)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    q, s = o.quantize_rows(w)
    y32 = o.dense_projection(o.bf16_decode(x), o.dequantize(q, s))
    return dict(x=x, q=q, s=s, y32=y32, y16=o.bf16_round(y32), seed=np.int64(SEED))


if __name__ == "__main__":
    np.savez_compressed(os.path.join(HERE, "config1.npz"), **config1())
    print("wrote", os.path.join(HERE, "config1.npz"))

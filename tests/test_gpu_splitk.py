"""The W8A16 split-K exchange on every form that splits K across blocks:
the shape-specialized column-group entries of the Llama-3-8B decode layer
(down K = 14336 and QKV at 32 rows, four slices), the generic column-group
form (eight slices, the last block loading seven partials in two batches;
gate/up with sixteen, two weights per tile), and the 128-row GEMM form
(four slices at BN 64, and six at BN 128: a width the launch geometry no
longer splits, launched directly, as a caller of the entry may). Every
block stores its partial tile and counts
itself; the last to arrive sums the S partials in slice order and resets
the counter. So every launch must match the oracle, be bit-identical to the
launch before it on the same workspace (the counters back at zero), and
leave rows past M untouched.
"""
import numpy as np
import pytest

import oracle_lib as o
from lunaflux_amd import synth
from lunaflux_amd.fp8 import _region
from parity import abs_sum, parity

pytestmark = pytest.mark.gpu

SENTINEL = 0x7FC1


@pytest.fixture(scope="module")
def rt():
    from lunaflux_amd.fp8 import ProjectionRuntime
    return ProjectionRuntime(0)


def weight(rt, rng, n, k):
    q, s = synth.weight(rng, n, k)
    return q, s, rt.upload_weight(q, s)


# (op, n, k, max_tokens, m, symbol, slices)
CASES = [
    ("dense", 4096, 14336, 32, 32, "lf_fp8_w8a16_dense_k14336_m32", 4),
    ("qkv", 6144, 4096, 32, 27, "lf_fp8_w8a16_qkv_k4096_q4096_kv1024_m32", 4),
    ("dense", 4096, 2048, 32, 17, "lf_fp8_w8a16_dense_m32", 8),
    ("gate_up", 1024, 2048, 32, 30, "lf_fp8_w8a16_gate_up_m32", 16),
    ("dense", 4096, 4096, 128, 128, "lf_fp8_w8a16_dense_m128_n64", 4),
    ("dense", 4096, 14336, 128, 77, "lf_fp8_w8a16_dense_m128_n64", 4),
    ("dense", 4096, 14336, 128, 77, "lf_fp8_w8a16_dense_m128_n128", 6),
]


@pytest.mark.parametrize("op,n,k,max_tokens,m,symbol,slices", CASES)
def test_split_k_exchange(rt, op, n, k, max_tokens, m, symbol, slices):
    rng = np.random.default_rng(13000 + n + k + m)
    xa = rt.context.allocate(max_tokens * k * 2)
    ya = rt.context.allocate(max_tokens * n * 2)
    counts = rt.step_counts(m)
    xr_, yr_ = _region(xa, alignment=256), _region(ya, alignment=256)
    if op == "qkv":
        ws = [weight(rt, rng, nn, k) for nn in (4096, 1024, 1024)]
        bound = rt.bind_qkv("w8a16", counts, xr_, *(w for _, _, w in ws), yr_, max_tokens)
        wr = o.dequantize(np.concatenate([q for q, _, _ in ws]), np.concatenate([s for _, s, _ in ws]))
    elif op == "gate_up":
        ws = [weight(rt, rng, n, k) for _ in range(2)]
        bound = rt.bind_gate_up("w8a16", counts, xr_, ws[0][2], ws[1][2], yr_, max_tokens)
    else:
        ws = [weight(rt, rng, n, k)]
        bound = rt.bind_dense("w8a16", counts, xr_, ws[0][2], yr_, max_tokens)
        wr = o.dequantize(ws[0][0], ws[0][1])
    step = bound.steps[0]
    blocks_n = {"lf_fp8_w8a16_dense_m128_n64": n // 64, "lf_fp8_w8a16_dense_m128_n128": n // 128}
    if step.name != symbol and symbol in blocks_n:
        # the entry launched directly with `slices` K-slices, on a workspace
        # of its size: S x blocks x 8 waves x (2 BN / 32) 1 KiB fragments,
        # then a counter per column block
        from lunaflux_amd.device import KernelArguments, KernelLaunchDimensions
        from lunaflux_amd.fp8 import BoundOperation, LaunchStep
        bn, cb = int(symbol.rsplit("_n", 1)[1]), blocks_n[symbol]
        al = lambda v: -(-v // 256) * 256
        nbytes = al(slices * cb * 8 * 2 * (bn // 32) * 1024) + al(cb * 4)
        wsd = rt.context.allocate(nbytes)
        wsd.copy_from_host(np.zeros(nbytes, np.uint8))
        dims = KernelLaunchDimensions.new((cb * slices, 1, 1), (512, 1, 1), 0)
        args = KernelArguments(step.args.arguments[:-1] + [_region(wsd, alignment=256)])
        bound = BoundOperation([LaunchStep(rt.function(symbol), dims, args, symbol)], workspace=wsd)
        step = bound.steps[0]
    assert len(bound.steps) == 1 and step.name == symbol, step.name
    # the grid is column blocks x slices
    per_block = 16 * (8 if op == "qkv" else 4) if symbol not in blocks_n else None
    cols = blocks_n.get(symbol) or -(-(n // 16) // (per_block // 16))
    assert step.dims.grid[0] == cols * slices, step.dims.grid
    assert bound.workspace.byte_count > 256

    def run(x):
        xa.copy_from_host(np.concatenate([x, np.zeros((max_tokens - m, k), np.uint16)]))
        ya.copy_from_host(np.full(max_tokens * n, SENTINEL, np.uint16))
        bound.launch(rt.stream, synchronous=True)
        y = ya.read(np.uint16, (max_tokens, n))
        assert np.all(y[m:] == SENTINEL), "rows past M written"
        return y[:m]

    sample = np.sort(rng.choice(n, 128, replace=False))
    for it in range(2):
        x = synth.activations(rng, m, k)
        xr = o.bf16_decode(x)
        y = run(x)
        label = f"{symbol} m={m} launch {it}"
        if op == "gate_up":
            wg = o.dequantize(ws[0][0][sample], ws[0][1][sample])
            wu = o.dequantize(ws[1][0][sample], ws[1][1][sample])
            ref = o.silu_mul_array(o.dense_projection(xr, wg), o.dense_projection(xr, wu))
            parity(y[:, sample], ref, label=label)
        else:
            wc = wr[sample]
            parity(y[:, sample], o.dense_projection(xr, wc), k=k, s_abs=abs_sum(xr, wc), label=label)
        assert np.array_equal(run(x), y), "a second launch on the same workspace differs"

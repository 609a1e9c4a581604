"""GPU parity of the dense FP8 projections against the CPU oracle.

Every call goes through the C-ABI (liblunaflux_hip.so: module load, function
load, region-checked launch) into the gfx950 code object. The oracle is the
reference's fp32 arithmetic over dequantized weights (and, for the w8a8
family, over the same per-token-quantized activations). Bar (BASELINE
north star): relative L2 <= 1e-3 and max-abs <= 2e-2 between the bf16 GPU
output and the oracle output rounded to bf16; quantized activations must be
bit-identical.
"""
import numpy as np
import pytest

import oracle_lib as o
from lunaflux_amd import synth
from parity import MAX_ABS, abs_sum, parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from lunaflux_amd.fp8 import ProjectionRuntime
    return ProjectionRuntime(0)


def check_projection(y, xr, wr, label):
    """Parity of a plain projection y = xr wr^T, with the summation bound
    for rounding-boundary flips."""
    ref = o.dense_projection(xr, wr)
    parity(y, ref, k=xr.shape[1], s_abs=abs_sum(xr, wr), label=label)


def make_weight(rt, rng, n, k, std=0.02):
    q, s = synth.weight(rng, n, k, std)
    return q, s, rt.upload_weight(q, s)


def deq(q, s):
    return o.dequantize(q, s)


def x_ref(x_bits, family):
    """What the oracle multiplies: bf16 values (w8a16) or the per-token
    e4m3 dequantized values (w8a8)."""
    xf = o.bf16_decode(x_bits)
    if family == "w8a16":
        return xf
    q, s = o.quantize_rows(xf)
    return o.dequantize(q, s)


def test_e4m3_codes_decode_exactly_through_w8a16(rt):
    # Row n of the weight holds code n in column 0 (NaN codes replaced by 0),
    # the scales are 1 and x is one-hot at column 0, so y[0, n] is the
    # decoded code itself (exact in bf16).
    codes = np.arange(256, dtype=np.uint8)
    codes[[0x7F, 0xFF]] = 0
    q = np.zeros((256, 128), np.uint8)
    q[:, 0] = codes
    w = rt.upload_weight(q, np.ones(256, np.float32))
    x = np.zeros((1, 128), np.uint16)
    x[0, 0] = 0x3F80  # 1.0
    y = rt.dense_projection(x, w, "w8a16", max_tokens=16)
    np.testing.assert_array_equal(o.bf16_decode(y[0]), o.e4m3_decode(codes))


@pytest.mark.parametrize("k", [1024, 6144, 14336, 20480])
def test_act_quant_bit_exact(rt, k):
    # k covers each register-resident row form (up to 4096, 8192, 16384
    # columns) and the two-pass form beyond
    rng = np.random.default_rng(7 + k)
    m = 37
    x = synth.activations(rng, m, k)
    x[3] = 0                      # all-zero row: zero codes, zero scale
    x[5, 17] = synth.bf16_bits(np.array([3.0e4], np.float32))[0]   # dominant outlier
    x[6] = synth.bf16_bits(np.full(k, 1e-30, np.float32))          # tiny row
    _, _, w = make_weight(rt, rng, 16, k)
    codes, scales = rt.act_quant(x, w, max_tokens=64)
    q_ref, s_ref = o.quantize_rows(o.bf16_decode(x))
    np.testing.assert_array_equal(codes, q_ref)
    np.testing.assert_array_equal(scales, s_ref)


def test_act_quant_every_bf16_value(rt):
    # Rows whose amax is exactly 448 (ratio 1): together they hold every
    # finite bf16 value of magnitude <= 448 with both signs, so the encode
    # of each bf16 input (every tie between two e4m3 codes included) is
    # compared with the oracle's.
    k = 16384
    mags = np.arange(0, 0x43E0 + 1, dtype=np.uint32).astype(np.uint16)   # 0 .. 448
    vals = np.concatenate([mags, mags | np.uint16(0x8000)])
    per_row = k - 1
    rows = -(-len(vals) // per_row)
    x = np.zeros((rows, k), np.uint16)
    for r in range(rows):
        chunk = vals[r * per_row:(r + 1) * per_row]
        x[r, 0] = 0x43E0                     # 448: the row's amax
        x[r, 1:1 + len(chunk)] = chunk
    rng = np.random.default_rng(11)
    _, _, w = make_weight(rt, rng, 16, k)
    codes, scales = rt.act_quant(x, w, max_tokens=16)
    q_ref, s_ref = o.quantize_rows(o.bf16_decode(x))
    np.testing.assert_array_equal(scales, s_ref)
    assert np.all(s_ref == np.float32(1.0))
    np.testing.assert_array_equal(codes, q_ref)


def test_golden_config1(rt):
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "config1.npz"))
    w = rt.upload_weight(g["q"], g["s"])
    y = rt.dense_projection(g["x"], w, "w8a16", max_tokens=16)
    parity(y, g["y32"], label="config1 w8a16")
    # the stored bf16 rounding of the oracle
    diff = np.abs(o.bf16_decode(y) - o.bf16_decode(g["y16"]))
    assert diff.max() <= MAX_ABS


@pytest.mark.parametrize("m,k,n,max_tokens", [
    (4, 512, 1536, 16), (1, 4096, 4096, 16), (8, 1024, 2048, 16), (16, 512, 256, 16),
    (32, 2048, 1024, 32), (17, 1024, 512, 32), (50, 512, 256, 64), (128, 1024, 512, 128),
    (100, 512, 128, 128), (0, 512, 256, 16), (20, 512, 80, 32), (3, 128, 48, 16),
    (64, 896, 208, 64),
])
def test_dense_w8a16(rt, m, k, n, max_tokens):
    rng = np.random.default_rng(1000 + m * 7 + k + n)
    x = synth.activations(rng, m, k)
    q, s, w = make_weight(rt, rng, n, k)
    y = rt.dense_projection(x, w, "w8a16", max_tokens=max_tokens)
    if m == 0:
        assert y.shape == (0, n)
        return
    check_projection(y, x_ref(x, "w8a16"), deq(q, s), f"dense w8a16 {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n,max_tokens", [
    (128, 512, 256, 128), (200, 1024, 384, 256), (1, 512, 128, 1), (300, 2048, 512, 512),
    (4, 512, 1536, 4), (0, 512, 128, 128),
])
def test_dense_w8a8(rt, m, k, n, max_tokens):
    rng = np.random.default_rng(2000 + m * 7 + k + n)
    x = synth.activations(rng, m, k)
    q, s, w = make_weight(rt, rng, n, k)
    y = rt.dense_projection(x, w, "w8a8", max_tokens=max_tokens)
    if m == 0:
        assert y.shape == (0, n)
        return
    check_projection(y, x_ref(x, "w8a8"), deq(q, s), f"dense w8a8 {m}x{k}x{n}")


@pytest.mark.parametrize("family_op", ["dense", "gate_up"])
def test_w8a16_split_k_repeated_launches(rt, family_op):
    """The column-group form reduces split-K partials through the workspace
    and clears their slots at the end of every launch: three launches of
    one binding (one workspace) must each match the oracle and be
    bit-identical to each other (the slice sum order is fixed)."""
    from lunaflux_amd import _abi, fp8
    from lunaflux_amd.fp8 import _region
    rng = np.random.default_rng(7100)
    m, k, n, max_tokens = 29, 2048, 1024, 32
    entry = _abi.ENTRY_W8A16_DENSE if family_op == "dense" else _abi.ENTRY_W8A16_GATE_UP
    dims, sym = fp8.launch_geometry(entry, n, k, max_tokens)
    assert not sym.endswith("_t1") and dims.grid[0] > (n // 16) // 4  # split across blocks
    x = synth.activations(rng, m, k)
    q, s_, w = make_weight(rt, rng, n, k)
    xa = rt.context.upload(np.concatenate([x, np.zeros((max_tokens - m, k), np.uint16)]))
    ya = rt.context.allocate(max_tokens * n * 2)
    counts = rt.step_counts(m)
    if family_op == "dense":
        op = rt.bind_dense("w8a16", counts, _region(xa, alignment=256), w, _region(ya, alignment=256),
                           max_tokens)
        ref = o.dense_projection(x_ref(x, "w8a16"), deq(q, s_))
    else:
        qu, su, wu = make_weight(rt, rng, n, k)
        op = rt.bind_gate_up("w8a16", counts, _region(xa, alignment=256), w, wu,
                             _region(ya, alignment=256), max_tokens)
        xr = x_ref(x, "w8a16")
        ref = o.silu_mul_array(o.dense_projection(xr, deq(q, s_)), o.dense_projection(xr, deq(qu, su)))
    outs = []
    for _ in range(3):
        op.launch(rt.stream, synchronous=True)
        outs.append(ya.read(np.uint16, (m, n)))
    bound = dict(k=k, s_abs=abs_sum(x_ref(x, "w8a16"), deq(q, s_))) if family_op == "dense" else {}
    for y in outs:
        parity(y, ref, label=f"split-K {family_op} repeated", **bound)
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])


_LARGE_TILE_CASES = [
    ("dense", 300, 128), ("dense", 1, 256), ("dense", 511, 384), ("dense", 257, 1408),
    ("qkv", 513, 128), ("qkv", 256, 640), ("gate_up", 257, 256), ("gate_up", 40, 128),
]


@pytest.mark.parametrize("op,m,k,form,max_tokens", [
    c + f for f in (("_t256", 4096), ("_t256w8", 3072), ("_t256x128", 2048))
    for c in _LARGE_TILE_CASES if not (f[0] == "_t256x128" and c[0] == "gate_up")
] + [("dense", 2048, 384, "_t256x128", 2048), ("qkv", 700, 512, "_t256x128", 2048)])
def test_w8a8_large_tile_edges(rt, op, m, k, form, max_tokens):
    """The 256-row tiles at these widths: 256 x 256 on four waves for
    max_query_tokens = 4096 (256 tiles), on eight waves for 3072 (192
    tiles), and (QKV and dense) 256 x 128 on four waves with three stages for
    2048. Ragged live rows, the shortest K loops (K = 128: one k-tile, K =
    256: the prologue with nothing left to load, K = 384: three stages and
    nothing left; the eight-wave ring's prologue and tail cases), an odd
    k-tile count (K = 1408), full tiles, and qkv region boundaries that fall
    inside a block (Nq = 2176, Nk = Nv = 960)."""
    from lunaflux_amd import _abi, fp8
    rng = np.random.default_rng(7000 + m + k)
    x = synth.activations(rng, m, k)
    xr = x_ref(x, "w8a8")
    if op == "dense":
        n = 4096
        assert fp8.launch_geometry(_abi.ENTRY_W8A8_DENSE, n, k, max_tokens)[1].endswith(form)
        q, s, w = make_weight(rt, rng, n, k)
        y = rt.dense_projection(x, w, "w8a8", max_tokens=max_tokens)
        check_projection(y, xr, deq(q, s), f"{form} dense m={m} k={k}")
    elif op == "qkv":
        ns = (2176, 960, 960)
        assert fp8.launch_geometry(_abi.ENTRY_W8A8_QKV, sum(ns), k, max_tokens)[1].endswith(form)
        ws = [make_weight(rt, rng, n, k) for n in ns]
        y = rt.qkv_projection(x, *(w for _, _, w in ws), family="w8a8", max_tokens=max_tokens)
        ref = o.qkv_projection(xr, *(deq(q, s) for q, s, _ in ws))
        wall = np.concatenate([deq(q, s) for q, s, _ in ws])
        parity(y, ref, k=k, s_abs=abs_sum(xr, wall), label=f"{form} qkv m={m} k={k}")
    else:
        inter = 2048
        assert fp8.launch_geometry(_abi.ENTRY_W8A8_GATE_UP, inter, k, max_tokens)[1].endswith(form)
        qg, sg, wg = make_weight(rt, rng, inter, k)
        qu, su, wu = make_weight(rt, rng, inter, k)
        h = rt.gate_up_swiglu(x, wg, wu, family="w8a8", max_tokens=max_tokens)
        ref = o.silu_mul_array(o.dense_projection(xr, deq(qg, sg)), o.dense_projection(xr, deq(qu, su)))
        parity(h, ref, label=f"{form} gate_up m={m} k={k}")


@pytest.mark.parametrize("family,m,max_tokens", [("w8a16", 3, 16), ("w8a16", 32, 32),
                                                 ("w8a8", 130, 256), ("w8a8", 5, 128)])
def test_qkv(rt, family, m, max_tokens):
    rng = np.random.default_rng(3000 + m)
    k, nq, nkv = 512, 256, 128
    x = synth.activations(rng, m, k)
    ws = [make_weight(rt, rng, n, k) for n in (nq, nkv, nkv)]
    y = rt.qkv_projection(x, *(w for _, _, w in ws), family=family, max_tokens=max_tokens)
    ref = o.qkv_projection(x_ref(x, family), *(deq(q, s) for q, s, _ in ws))
    wall = np.concatenate([deq(q, s) for q, s, _ in ws])
    parity(y, ref, k=k, s_abs=abs_sum(x_ref(x, family), wall), label=f"qkv {family} m={m}")


@pytest.mark.parametrize("family,m,max_tokens", [("w8a16", 7, 16), ("w8a16", 64, 64),
                                                 ("w8a8", 150, 256)])
def test_gate_up_swiglu(rt, family, m, max_tokens):
    rng = np.random.default_rng(4000 + m)
    k, inter = 512, 384
    x = synth.activations(rng, m, k)
    qg, sg, wg = make_weight(rt, rng, inter, k)
    qu, su, wu = make_weight(rt, rng, inter, k)
    h = rt.gate_up_swiglu(x, wg, wu, family=family, max_tokens=max_tokens)
    xr = x_ref(x, family)
    ref = o.silu_mul_array(o.dense_projection(xr, deq(qg, sg)), o.dense_projection(xr, deq(qu, su)))
    parity(h, ref, label=f"gate_up {family} m={m}")


@pytest.mark.parametrize("family,m,max_tokens", [("w8a16", 5, 16), ("w8a8", 70, 128)])
def test_silu_gated_mlp(rt, family, m, max_tokens):
    rng = np.random.default_rng(5000 + m)
    hidden, inter = 256, 512
    x = synth.activations(rng, m, hidden)
    qg, sg, wg = make_weight(rt, rng, inter, hidden)
    qu, su, wu = make_weight(rt, rng, inter, hidden)
    qd, sd, wd = make_weight(rt, rng, hidden, inter)
    y = rt.silu_gated_mlp(x, wg, wu, wd, family=family, max_tokens=max_tokens)
    xr = x_ref(x, family)
    h = o.silu_mul_array(o.dense_projection(xr, deq(qg, sg)), o.dense_projection(xr, deq(qu, su)))
    # the device keeps h as bf16 between its two launches (and the w8a8
    # family then quantizes it per token like any activation)
    hb = o.bf16_round(h)
    ref = o.dense_projection(x_ref(hb, family), deq(qd, sd))
    parity(y, ref, label=f"mlp {family} m={m}")


@pytest.mark.parametrize("m,max_tokens", [(1, 16), (13, 16), (16, 16), (17, 32), (32, 32), (0, 32),
                                          (128, 128), (97, 128), (65, 128)])
def test_gated_mlp_one_launch(rt, m, max_tokens):
    """The one-launch W8A16 GatedMlp at the Llama-3-8B widths (H 4096, I
    14336): against the oracle on a column sample of y (h rounded to bf16
    between the GEMMs, as the two-launch form keeps it); bit-identical to
    the two-launch form where both use the same kernels (the 32-row profile's
    column groups, the 128-row profile's LDS-tiled GEMMs); three launches on
    one workspace agree bit for bit (the slice and done counters return to
    zero) and leave the error word 0; rows past M untouched; then new inputs
    on the same workspace."""
    from lunaflux_amd import _abi
    from lunaflux_amd.fp8 import _region
    rng = np.random.default_rng(7300 + m + max_tokens)
    hidden, inter = 4096, 14336
    x = synth.activations(rng, max(m, 1), hidden)[:m]
    qg, sg, wg = make_weight(rt, rng, inter, hidden)
    qu, su, wu = make_weight(rt, rng, inter, hidden)
    qd, sd, wd = make_weight(rt, rng, hidden, inter)
    xa = rt.context.upload(np.concatenate([x, np.zeros((max_tokens - m, hidden), np.uint16)]))
    counts = rt.step_counts(m)
    ya = rt.context.allocate(max_tokens * hidden * 2)
    one = rt.bind_gated_mlp("w8a16", counts, _region(xa, alignment=256), wg, wu, wd,
                            _region(ya, alignment=256), max_tokens)
    assert len(one.steps) == 1 and one.steps[0].name.startswith("lf_fp8_w8a16_gated_mlp_"), one.steps
    sentinel = np.full(max_tokens * hidden, 0x7FC1, np.uint16)
    ya.copy_from_host(sentinel)
    outs = []
    for _ in range(3):
        one.launch(rt.stream, synchronous=True)
        outs.append(ya.read(np.uint16, (max_tokens, hidden)))
    ws = one.workspace
    err = ws.read(np.int32, (1,), ws.byte_count - _abi.LF_FP8_GATED_MLP_ERROR_OFFSET_FROM_END)
    assert err[0] == 0, "a down block's wait for h ran out"
    assert all(np.array_equal(outs[0], y) for y in outs[1:]), "launches differ"
    assert np.all(outs[0][m:] == 0x7FC1), "rows past M written"
    if m:
        cols = np.sort(rng.choice(hidden, 256, replace=False))
        xr = x_ref(x, "w8a16")
        h = o.silu_mul_array(o.dense_projection(xr, deq(qg, sg)), o.dense_projection(xr, deq(qu, su)))
        hb = o.bf16_decode(o.bf16_round(h))
        wdc = deq(qd[cols], sd[cols])
        parity(outs[0][:m][:, cols], o.dense_projection(hb, wdc), k=inter, s_abs=abs_sum(hb, wdc),
               label=f"gated mlp one launch m={m}")
    if max_tokens in (32, 128):
        ya.copy_from_host(sentinel)
        two = rt.bind_gated_mlp("w8a16", counts, _region(xa, alignment=256), wg, wu, wd,
                                _region(ya, alignment=256), max_tokens, one_launch=False)
        assert len(two.steps) == 2
        two.launch(rt.stream, synchronous=True)
        assert np.array_equal(ya.read(np.uint16, (max_tokens, hidden)), outs[0])
        # new inputs on the same workspace: each launch starts from counters
        # at rest (a stale count would let down read h early)
        for _ in range(2):
            x2 = synth.activations(rng, max(m, 1), hidden)[:m]
            xa.copy_from_host(np.concatenate([x2, np.zeros((max_tokens - m, hidden), np.uint16)]))
            one.launch(rt.stream, synchronous=True)
            y1 = ya.read(np.uint16, (max_tokens, hidden))
            two.launch(rt.stream, synchronous=True)
            assert np.array_equal(y1, ya.read(np.uint16, (max_tokens, hidden)))


@pytest.mark.parametrize("op,m,family", [
    ("qkv", 32, "w8a16"), ("gate_up", 32, "w8a16"), ("down", 32, "w8a16"), ("o", 1, "w8a16"),
    ("qkv", 2048, "w8a8"), ("o", 2048, "w8a8"), ("gate_up", 2048, "w8a8"), ("down", 2048, "w8a8"),
    ("qkv", 8192, "w8a8"), ("o", 8192, "w8a8"), ("gate_up", 8192, "w8a8"), ("down", 8192, "w8a8"),
])
def test_llama3_8b_shapes_sampled(rt, op, m, family):
    """Full Llama-3-8B projection shapes (all four
    operations at M = 2048 and 8192, on whichever W8A8 tile form the
    geometry picks); the oracle checks a column sample (and, for prefill, a
    row sample that includes the first and last rows), which keeps it to
    seconds."""
    rng = np.random.default_rng(6000 + m)
    k = 14336 if op == "down" else 4096
    x = synth.activations(rng, m, k)
    rows = np.arange(m) if m <= 128 else np.unique(np.concatenate(
        [[0, m - 1], rng.choice(m, 94, replace=False)]))
    if op == "qkv":
        ws = [make_weight(rt, rng, n, k) for n in (4096, 1024, 1024)]
        y = rt.qkv_projection(x, *(w for _, _, w in ws), family=family, max_tokens=m)
        cols = np.sort(rng.choice(6144, 384, replace=False))
        wfull = np.concatenate([q for q, _, _ in ws]), np.concatenate([s for _, s, _ in ws])
        xr, wr = x_ref(x, family)[rows], deq(wfull[0][cols], wfull[1][cols])
    elif op == "gate_up":
        (qg, sg, wg), (qu, su, wu) = make_weight(rt, rng, 14336, k), make_weight(rt, rng, 14336, k)
        y = rt.gate_up_swiglu(x, wg, wu, family=family, max_tokens=m)
        cols = np.sort(rng.choice(14336, 256, replace=False))
        xr = x_ref(x, family)[rows]
        ref = o.silu_mul_array(o.dense_projection(xr, deq(qg[cols], sg[cols])),
                               o.dense_projection(xr, deq(qu[cols], su[cols])))
    else:
        q, s, w = make_weight(rt, rng, 4096, k)
        y = rt.dense_projection(x, w, family=family, max_tokens=m)
        cols = np.sort(rng.choice(4096, 256, replace=False))
        xr, wr = x_ref(x, family)[rows], deq(q[cols], s[cols])
    label = f"llama3-8b {op} {family} m={m}"
    if op == "gate_up":
        parity(y[rows][:, cols], ref, label=label)
    else:
        check_projection(y[rows][:, cols], xr, wr, label)


@pytest.mark.parametrize("op,m,max_tokens", [
    ("o", 1, 16), ("o", 16, 16), ("o", 17, 32), ("o", 32, 32), ("o", 0, 32),
    ("down", 5, 16), ("down", 20, 32), ("down", 32, 32),
    ("qkv", 1, 16), ("qkv", 13, 16), ("qkv", 32, 32),
    ("gate_up", 8, 16), ("gate_up", 25, 32), ("gate_up", 32, 32),
    ("o", 128, 128), ("o", 70, 128), ("down", 128, 128), ("down", 97, 128),
    ("qkv", 128, 128), ("qkv", 33, 128), ("gate_up", 128, 128), ("gate_up", 111, 128),
])
def test_w8a16_specialized_entries(rt, op, m, max_tokens):
    """Every shape-specialized W8A16 entry (Llama-3-8B widths, profiles of
    <= 16 and <= 32 rows) and the LDS-tiled GEMM form at 128 rows against the
    oracle on a column sample, with
    ragged live rows and M = 0; the column-group forms run three launches on
    one workspace, which must be bit-identical."""
    from lunaflux_amd import _abi, fp8
    from lunaflux_amd.fp8 import _region
    rng = np.random.default_rng(8100 + 97 * m + max_tokens + len(op))
    k = 14336 if op == "down" else 4096
    x = synth.activations(rng, max(m, 1), k)[:m]
    xa = rt.context.upload(np.concatenate([x, np.zeros((max_tokens - m, k), np.uint16)]))
    counts = rt.step_counts(m)
    # (M = 0: the oracle rejects an empty activation, so one row stands in)
    xr = x_ref(x if m else synth.activations(rng, 1, k), "w8a16")
    if op == "qkv":
        ws = [make_weight(rt, rng, n, k) for n in (4096, 1024, 1024)]
        n = 6144
        sym = fp8.launch_geometry(_abi.ENTRY_W8A16_QKV, n, k, max_tokens, qkv_split=(4096, 1024))[1]
        ya = rt.context.allocate(max_tokens * n * 2)
        bound = rt.bind_qkv("w8a16", counts, _region(xa, alignment=256), *(w for _, _, w in ws),
                            _region(ya, alignment=256), max_tokens)
        cols = np.sort(rng.choice(n, 512, replace=False))
        wq = np.concatenate([q for q, _, _ in ws])[cols]
        wsc = np.concatenate([s for _, s, _ in ws])[cols]
        ref = o.dense_projection(xr, deq(wq, wsc))
        extra = dict(k=k, s_abs=abs_sum(xr, deq(wq, wsc)))
    elif op == "gate_up":
        n = 14336
        (qg, sg, wg), (qu, su, wu) = make_weight(rt, rng, n, k), make_weight(rt, rng, n, k)
        sym = fp8.launch_geometry(_abi.ENTRY_W8A16_GATE_UP, n, k, max_tokens)[1]
        ya = rt.context.allocate(max_tokens * n * 2)
        bound = rt.bind_gate_up("w8a16", counts, _region(xa, alignment=256), wg, wu,
                                _region(ya, alignment=256), max_tokens)
        cols = np.sort(rng.choice(n, 256, replace=False))
        ref = o.silu_mul_array(o.dense_projection(xr, deq(qg[cols], sg[cols])),
                               o.dense_projection(xr, deq(qu[cols], su[cols])))
        extra = {}
    else:
        n = 4096
        q, s, w = make_weight(rt, rng, n, k)
        sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, n, k, max_tokens)[1]
        ya = rt.context.allocate(max_tokens * n * 2)
        bound = rt.bind_dense("w8a16", counts, _region(xa, alignment=256), w,
                              _region(ya, alignment=256), max_tokens)
        cols = np.sort(rng.choice(n, 384, replace=False))
        ref = o.dense_projection(xr, deq(q[cols], s[cols]))
        extra = dict(k=k, s_abs=abs_sum(xr, deq(q[cols], s[cols])))
    if max_tokens == 128:  # the LDS-tiled GEMM form
        assert "_m128_n" in sym, sym
    else:
        assert f"_k{k}_" in sym and sym.endswith(f"_m{max_tokens}"), sym
    sentinel = np.full(max_tokens * n, 0x7FC1, np.uint16)  # a NaN no kernel writes
    ya.copy_from_host(sentinel)
    outs = []
    for _ in range(3):
        bound.launch(rt.stream, synchronous=True)
        outs.append(ya.read(np.uint16, (max_tokens, n)))
    for y in outs:
        # rows past M stay untouched
        assert np.all(y[m:] == 0x7FC1), f"{sym}: rows past M written"
        if m:
            parity(y[:m][:, cols], ref, label=f"{sym} m={m}", **extra)
    assert all(np.array_equal(outs[0], y) for y in outs[1:]), f"{sym}: launches differ"


@pytest.mark.parametrize("op,n,k,qkv_split,m,max_tokens", [
    ("dense", 3072, 2048, None, 65, 80),        # BN 64, 48 blocks x 2 slices of 8 k-tiles
    ("dense", 24576, 1024, None, 128, 128),     # BN 128 (192 blocks), no split
    ("dense", 1024, 8192, None, 100, 128),      # BN 64, 16 blocks, S 8
    ("qkv", 3072, 4096, (2048, 512), 77, 128),  # BN 64, S 4; blocks straddle Q|K|V
    ("gate_up", 8192, 2048, None, 128, 128),    # BN 64 unsplit (256 blocks; ties BN 128 x 2)
    ("gate_up", 4096, 4096, None, 100, 128),    # BN 64, S 2 (256 blocks)
    ("dense", 40960, 1024, None, 128, 128),     # BN 128 unsplit, 320 blocks (> 256 either way)
    ("gate_up", 12288, 4096, None, 90, 96),     # BN 128 (192 blocks)
])
def test_w8a16_gemm_form(rt, op, n, k, qkv_split, m, max_tokens):
    """The LDS-tiled W8A16 GEMM (profiles of 65..128 rows) on shapes other
    than Llama-3-8B's: each block width, with and without the K split, QKV
    blocks across the Q|K|V boundaries, ragged M. Column sample against the
    oracle; rows past M untouched; three launches on one workspace agree
    bit for bit."""
    from lunaflux_amd import _abi, fp8
    from lunaflux_amd.fp8 import _region
    rng = np.random.default_rng(9100 + n + k + m)
    x = synth.activations(rng, m, k)
    xa = rt.context.upload(np.concatenate([x, np.zeros((max_tokens - m, k), np.uint16)]))
    counts = rt.step_counts(m)
    xr = x_ref(x, "w8a16")
    ya = rt.context.allocate(max_tokens * n * 2)
    cols = np.sort(rng.choice(n, 384, replace=False))
    extra = {}
    if op == "qkv":
        nq, nkv = qkv_split
        ws = [make_weight(rt, rng, r, k) for r in (nq, nkv, nkv)]
        sym = fp8.launch_geometry(_abi.ENTRY_W8A16_QKV, n, k, max_tokens, qkv_split=qkv_split)[1]
        bound = rt.bind_qkv("w8a16", counts, _region(xa, alignment=256), *(w for _, _, w in ws),
                            _region(ya, alignment=256), max_tokens)
        wq = np.concatenate([q for q, _, _ in ws])[cols]
        wsc = np.concatenate([s for _, s, _ in ws])[cols]
        ref = o.dense_projection(xr, deq(wq, wsc))
        extra = dict(k=k, s_abs=abs_sum(xr, deq(wq, wsc)))
    elif op == "gate_up":
        (qg, sg, wg), (qu, su, wu) = make_weight(rt, rng, n, k), make_weight(rt, rng, n, k)
        sym = fp8.launch_geometry(_abi.ENTRY_W8A16_GATE_UP, n, k, max_tokens)[1]
        bound = rt.bind_gate_up("w8a16", counts, _region(xa, alignment=256), wg, wu,
                                _region(ya, alignment=256), max_tokens)
        ref = o.silu_mul_array(o.dense_projection(xr, deq(qg[cols], sg[cols])),
                               o.dense_projection(xr, deq(qu[cols], su[cols])))
    else:
        q, s, w = make_weight(rt, rng, n, k)
        sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, n, k, max_tokens)[1]
        bound = rt.bind_dense("w8a16", counts, _region(xa, alignment=256), w,
                              _region(ya, alignment=256), max_tokens)
        ref = o.dense_projection(xr, deq(q[cols], s[cols]))
        extra = dict(k=k, s_abs=abs_sum(xr, deq(q[cols], s[cols])))
    assert "_m128_n" in sym, sym
    sentinel = np.full(max_tokens * n, 0x7FC1, np.uint16)
    ya.copy_from_host(sentinel)
    outs = []
    for _ in range(3):
        bound.launch(rt.stream, synchronous=True)
        outs.append(ya.read(np.uint16, (max_tokens, n)))
    for y in outs:
        assert np.all(y[m:] == 0x7FC1), f"{sym}: rows past M written"
        parity(y[:m][:, cols], ref, label=f"{sym} {op} n={n} k={k} m={m}", **extra)
    assert all(np.array_equal(outs[0], y) for y in outs[1:]), f"{sym}: launches differ"


def lm_head_weight(rt, rng, vocab, k):
    """A [vocab, k] head weight: a 2048-row N(0, 0.02) draw tiled down the
    vocabulary (drawing 525 M values would take most of the test's time),
    each copy's scales multiplied by its own factor so tiles differ."""
    q0, s0 = synth.weight(rng, 2048, k)
    reps = -(-vocab // 2048)
    q = np.tile(q0, (reps, 1))[:vocab]
    s = (np.tile(s0, reps) * np.repeat(np.linspace(0.5, 1.5, reps, dtype=np.float32), 2048))[:vocab]
    return q, s.astype(np.float32), rt.upload_weight(q, s.astype(np.float32))


@pytest.mark.parametrize("m,max_tokens,family", [(1, 16, "w8a16"), (13, 16, "w8a16"),
                                                (32, 32, "w8a16"), (100, 128, "w8a16"),
                                                (256, 256, "w8a8")])
def test_language_model_head(rt, m, max_tokens, family):
    """Llama-3 vocabulary head (hidden 4096 -> 128,256 logits = 8016
    16-column tiles, 501 256-column tiles): the dense entry at the widest
    shape it serves, checked on a column sample that includes the last 64
    columns, and for W8A16 on the K = 4096 wide-shape entries."""
    from lunaflux_amd import _abi, fp8
    vocab, k = 128256, 4096
    rng = np.random.default_rng(9100 + m)
    q, s, w = lm_head_weight(rt, rng, vocab, k)
    x = synth.activations(rng, m, k)
    if family == "w8a16":
        sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, vocab, k, max_tokens)[1]
        assert sym == f"lf_fp8_w8a16_dense_wide_k4096_m{max_tokens}", sym
    y = rt.language_model_head(x, w, family=family, max_tokens=max_tokens)
    assert y.shape == (m, vocab)
    cols = np.concatenate([np.sort(rng.choice(vocab - 64, 448, replace=False)),
                           np.arange(vocab - 64, vocab)])
    rows = np.arange(m) if m <= 128 else np.sort(rng.choice(m, 64, replace=False))
    check_projection(y[rows][:, cols], x_ref(x, family)[rows], deq(q[cols], s[cols]),
                     f"lm_head {family} m={m}")


def test_w8a16_specialized_entry_rejects_other_shape(rt):
    """A specialized entry checks the header against its compiled shape: a
    K = 8192 weight region launched on the K = 4096 dense entry (its reads
    stay inside the larger region) leaves the output untouched."""
    from lunaflux_amd.device import KernelArguments
    from lunaflux_amd.fp8 import _region, COUNTS_BYTES
    rng = np.random.default_rng(8200)
    m, k, n = 4, 4096, 4096
    _, _, w = make_weight(rt, rng, n, 2 * k)
    x = synth.activations(rng, 16, k)
    xa = rt.context.upload(x)
    ya = rt.context.upload(np.full(16 * n, 0x7FC1, np.uint16))
    ws = rt.context.allocate(256)
    counts = rt.step_counts(m)
    from lunaflux_amd import _abi, fp8
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, n, k, 16)
    assert sym == "lf_fp8_w8a16_dense_k4096_m16"
    args = KernelArguments([_region(counts, COUNTS_BYTES, alignment=4), _region(xa, alignment=256),
                            w.region, _region(ya, alignment=256), _region(ws, alignment=256)])
    rt.function(sym).launch_synchronous(dims, args, rt.stream)
    assert np.all(ya.read(np.uint16, (16 * n,)) == 0x7FC1)


def test_checkpoint_weight_through_the_dense_entry(rt, tmp_path):
    """An FP8 weight admitted from a safetensors file (per-channel scales),
    uploaded and run through the W8A16 and W8A8 dense entries."""
    import json
    import struct
    from lunaflux_amd import checkpoint
    rng = np.random.default_rng(4321)
    q, s = synth.weight(rng, 512, 1024)
    blobs = [q.tobytes(), s.reshape(-1, 1).tobytes()]
    header = {"proj.weight": {"dtype": "F8_E4M3", "shape": [512, 1024], "data_offsets": [0, len(blobs[0])]},
              "proj.weight_scale": {"dtype": "F32", "shape": [512, 1],
                                    "data_offsets": [len(blobs[0]), len(blobs[0]) + len(blobs[1])]}}
    text = json.dumps(header).encode()
    path = str(tmp_path / "proj.safetensors")
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + b"".join(blobs))
    w = checkpoint.upload_linear(rt, path, "proj")
    x = synth.activations(rng, 20, 1024)
    for family in ("w8a16", "w8a8"):
        y = rt.dense_projection(x, w, family, max_tokens=32)
        check_projection(y, x_ref(x, family), deq(q, s), f"checkpoint weight {family}")

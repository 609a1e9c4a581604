"""GPU parity of the block-scaled projections against the CPU oracle.

Weights carry 128 x 128 block scales (W = q s[n / 128][k / 128], the
weight_scale_inv checkpoint format; the oracle's lfo_dequantize mode 2).
W8A16 multiplies the bf16 activations; W8A8 quantizes them per token per
128-column group inside the launch (lfo_quantize_rows with group 128: codes
and scales bit-exact, read from the launch's workspace) and multiplies the
dequantized values. The weights' block magnitudes and the activations' group
magnitudes vary by up to 2^6 from one k-tile to the next, so a scale applied
to the wrong k-tile, row or column block moves outputs far past the bar.
Summation bound for rounding-boundary flips: gamma over K + 2 K / 128 terms
(each k-tile's fp32 sum is scaled and then added: two more roundings per
k-tile than a sequential dot product).
"""
import numpy as np
import pytest

import oracle_lib as o
from lunaflux_amd import _abi, fp8, synth
from lunaflux_amd.device import DeviceError
from lunaflux_amd.fp8 import _region
from parity import abs_sum, parity, swiglu_midpoint_tol

pytestmark = pytest.mark.gpu

SENTINEL = 0x7FC1


@pytest.fixture(scope="module")
def rt():
    from lunaflux_amd.fp8 import ProjectionRuntime
    return ProjectionRuntime(0)


def spread_weight(rng, n, k, zero_block=False):
    """Block-quantized N(0, 0.02) weights, each 128 x 128 block scaled by
    2^U(-3, 3); zero_block: the first block all zero (codes and scale 0)."""
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    f = np.exp2(rng.uniform(-3, 3, (n // 128, k // 128))).astype(np.float32)
    w = (w.reshape(n // 128, 128, k // 128, 128) * f[:, None, :, None]).reshape(n, k)
    if zero_block:
        w[:128, :128] = 0
    return synth.quantize_blocks(w, 128)


def spread_activations(rng, m, k, zero_groups=False):
    """bf16 N(0, 1) rows, each 128-column group scaled by 2^U(-3, 3);
    zero_groups: row 1's second group and all of row 2 zero."""
    x = rng.standard_normal((m, k), dtype=np.float32)
    x *= np.repeat(np.exp2(rng.uniform(-3, 3, (m, k // 128))), 128, axis=1).astype(np.float32)
    if zero_groups and m > 2:
        x[1, 128:256] = 0
        x[2] = 0
    return synth.bf16_bits(x)


def upload(rt, q, s):
    return rt.upload_weight(q, s, fp8.BLOCK128)


def deq(q, s):
    """The whole weight: s[n / 128][k / 128] (lfo_dequantize mode 2)."""
    return o.dequantize(q, s, mode=2, group=128)


def deq_rows(q, s, rows):
    """Rows `rows` of the weight: each with its block row's scales, as
    per-row per-group scales (lfo_dequantize mode 1)."""
    return o.dequantize(q[rows], s[rows // 128], mode=1, group=128)


def x_ref(x_bits, family):
    xf = o.bf16_decode(x_bits)
    if family == "w8a16":
        return xf
    q, s = o.quantize_rows(xf, group=128)
    return o.dequantize(q, s, mode=1, group=128)


def bound_k(k):
    return k + 2 * (k // 128)


SHAPES = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (14336, 4096), "down": (4096, 14336)}


def run_op(rt, rng, op, family, m, max_tokens, zero=False):
    """Binds the operation on block-scaled weights of the Llama-3-8B shape,
    launches it on m live rows of a max_tokens profile and returns (y, x,
    weights, bound operation); rows past m must stay untouched."""
    n, k = SHAPES[op]
    x = spread_activations(rng, max(m, 1), k, zero_groups=zero)[:m]
    xa = rt.context.allocate(max_tokens * k * 2)
    xa.copy_from_host(np.concatenate([x, np.zeros((max_tokens - m, k), np.uint16)]))
    ya = rt.context.allocate(max_tokens * n * 2)
    ya.copy_from_host(np.full(max_tokens * n, SENTINEL, np.uint16))
    counts = rt.step_counts(m)
    xr, yr = _region(xa, alignment=256), _region(ya, alignment=256)
    if op == "qkv":
        ws = [spread_weight(rng, nn, k, zero_block=zero) for nn in (4096, 1024, 1024)]
        bound = rt.bind_qkv(family, counts, xr, *(upload(rt, q, s) for q, s in ws), yr, max_tokens)
    elif op == "gate_up":
        ws = [spread_weight(rng, n, k, zero_block=zero) for _ in range(2)]
        bound = rt.bind_gate_up(family, counts, xr, *(upload(rt, q, s) for q, s in ws), yr, max_tokens)
    else:
        ws = [spread_weight(rng, n, k, zero_block=zero)]
        bound = rt.bind_dense(family, counts, xr, upload(rt, *ws[0]), yr, max_tokens)
    assert len(bound.steps) == 1 and "_b128" in bound.steps[0].name, bound.steps
    bound.launch(rt.stream, synchronous=True)
    y = ya.read(np.uint16, (max_tokens, n))
    assert np.all(y[m:] == SENTINEL), "rows past M written"
    # a second launch on the same workspace (its counters back at rest):
    # the same bits
    bound.launch(rt.stream, synchronous=True)
    assert np.array_equal(ya.read(np.uint16, (max_tokens, n)), y)
    return y[:m], x, ws, bound


def check_op(op, family, y, x, ws, rows, cols, label):
    k = SHAPES[op][1]
    xr = x_ref(x[rows], family)
    if op == "gate_up":
        wg, wu = (deq_rows(q, s, cols) for q, s in ws)
        g, u = o.dense_projection(xr, wg), o.dense_projection(xr, wu)
        tol = swiglu_midpoint_tol(g, u, abs_sum(xr, wg), abs_sum(xr, wu), bound_k(k))
        parity(y[rows][:, cols], o.silu_mul_array(g, u), label=label, midpoint_tol=tol)
        return
    if op == "qkv":
        wfull = np.concatenate([deq(q, s) for q, s in ws])[cols]
    else:
        wfull = deq_rows(*ws[0], cols)
    parity(y[rows][:, cols], o.dense_projection(xr, wfull), k=bound_k(k), s_abs=abs_sum(xr, wfull),
           label=label)


def sample(rng, m, n, nrows, ncols):
    rows = np.arange(m) if m <= nrows else np.unique(np.concatenate(
        [[0, 1, 2, m - 1], rng.choice(m, nrows, replace=False)]))
    # whole 128-column blocks' edges plus random columns
    cols = np.unique(np.concatenate([[0, 127, 128, n - 1], rng.choice(n, ncols, replace=False)]))
    return rows, cols


def test_block_scaled_dequantize_matches_block_layout():
    """The oracle's mode-2 dequantization applies s[n / 128][k / 128], and
    deq_rows (rows of q with their block row's scales) takes the same rows
    of it."""
    rng = np.random.default_rng(1)
    q, s = spread_weight(rng, 256, 384)
    full = deq(q, s)
    cols = np.array([0, 5, 130, 255])
    np.testing.assert_array_equal(deq_rows(q, s, cols), full[cols])
    np.testing.assert_array_equal(full, o.e4m3_decode(q) * np.repeat(np.repeat(s, 128, 0), 128, 1))


@pytest.mark.parametrize("op,m,max_tokens", [
    ("o", 1, 16), ("o", 13, 16), ("qkv", 16, 16), ("gate_up", 9, 16), ("down", 16, 16),
    ("qkv", 32, 32), ("gate_up", 20, 32), ("down", 32, 32), ("o", 64, 64),
    ("qkv", 100, 128), ("gate_up", 128, 128), ("down", 77, 128), ("o", 128, 128),
])
def test_block_scaled_w8a16(rt, op, m, max_tokens):
    rng = np.random.default_rng(12000 + 131 * m + max_tokens + len(op))
    y, x, ws, bound = run_op(rt, rng, op, "w8a16", m, max_tokens, zero=(m == 13 or m == 20))
    rows, cols = sample(rng, m, SHAPES[op][0], 128, 320)
    check_op(op, "w8a16", y, x, ws, rows, cols, f"b128 w8a16 {op} m={m}/{max_tokens}")


def w8a8_quantized_rows(bound, m, k, max_tokens):
    """(codes [m, K], scales [m, K / 128]) from the one-launch workspace:
    sync area (256 + 128 bands bytes), codes [cap, K], scales [K / 128][cap],
    with bands of 128 rows (256 on the 256-row forms, _t256 and _t256x128)
    and cap = bands x height."""
    height = 256 if "_t256" in bound.steps[0].name else 128
    bands = -(-max_tokens // height)
    cap = height * bands
    at = 256 + 128 * bands
    codes = bound.workspace.read(np.uint8, (cap, k), at)[:m]
    st = bound.workspace.read(np.float32, (k // 128, cap), at + -(-cap * k // 256) * 256)
    return codes, np.ascontiguousarray(st[:, :m].T)


# (qkv and gate/up at 2048 rows, and every case from 512 rows of gate/up or
# 3072 rows of o / down on, take the 256 x 256 form, the others the 256 x
# 128 one; the ragged and single-band cases leave bands without live rows)
T256 = {("qkv", 2048, 2048), ("gate_up", 2048, 2048), ("o", 4096, 4096), ("down", 3000, 3072),
        ("gate_up", 700, 1024), ("gate_up", 200, 1024), ("qkv", 1800, 2048)}


@pytest.mark.parametrize("op,m,max_tokens", [
    ("qkv", 2048, 2048), ("o", 2048, 2048), ("gate_up", 2048, 2048), ("down", 2048, 2048),
    ("o", 100, 256), ("down", 300, 512), ("qkv", 129, 256), ("gate_up", 1, 128),
    ("o", 4096, 4096), ("down", 3000, 3072), ("gate_up", 700, 1024), ("gate_up", 200, 1024),
    ("qkv", 1800, 2048),
])
def test_block_scaled_w8a8(rt, op, m, max_tokens):
    rng = np.random.default_rng(13000 + 7 * m + max_tokens + len(op))
    y, x, ws, bound = run_op(rt, rng, op, "w8a8", m, max_tokens, zero=m in (100, 700, 1800))
    form = "_t256" if (op, m, max_tokens) in T256 else "_t256x128"
    assert bound.steps[0].name.endswith(form), bound.steps[0].name
    k = SHAPES[op][1]
    codes, scales = w8a8_quantized_rows(bound, m, k, max_tokens)
    q_ref, s_ref = o.quantize_rows(o.bf16_decode(x), group=128)
    np.testing.assert_array_equal(codes, q_ref)
    np.testing.assert_array_equal(scales, s_ref.reshape(m, -1))
    rows, cols = sample(rng, m, SHAPES[op][0], 48, 256)
    check_op(op, "w8a8", y, x, ws, rows, cols, f"b128 w8a8 {op} m={m}/{max_tokens}")


@pytest.mark.parametrize("family,hidden,inter,m,max_tokens", [
    ("w8a8", 4096, 14336, 2048, 2048), ("w8a8", 512, 1024, 100, 256), ("w8a8", 4096, 14336, 300, 512),
    ("w8a8", 4096, 2048, 3000, 3072),
    ("w8a16", 4096, 14336, 32, 32), ("w8a16", 512, 1024, 100, 128),
])
def test_block_scaled_gated_mlp(rt, family, hidden, inter, m, max_tokens):
    """GatedMlp on block-scaled weights: W8A8 as one launch (four counted
    steps; both GEMMs on 256 x 256 tiles where the gate/up launch takes
    them and the hidden width is a multiple of 256: the Llama-3-8B widths
    from 257 rows on; else 128 x 128) against the two block-scaled launches
    it replaces, bit for bit where all of them have 256-row bands (the
    256 x 256 and 256 x 128 forms compute the same sums), else the chain
    checked against the oracle on its own h; W8A16 as those two launches. The oracle checks stage by stage on the device's own bf16
    h (read from the workspace): gate/up, the h quantizer (W8A8: codes and
    scales of the group quantizer), then down."""
    rng = np.random.default_rng(14000 + m + hidden)
    (qg, sg), (qu, su) = spread_weight(rng, inter, hidden), spread_weight(rng, inter, hidden)
    qd, sd = spread_weight(rng, hidden, inter)
    wg, wu, wd = upload(rt, qg, sg), upload(rt, qu, su), upload(rt, qd, sd)
    x = spread_activations(rng, m, hidden)
    xa = rt.context.upload(np.concatenate([x, np.zeros((max_tokens - m, hidden), np.uint16)]))
    ya = rt.context.allocate(max_tokens * hidden * 2)
    counts = rt.step_counts(m)
    xr_, yr_ = _region(xa, alignment=256), _region(ya, alignment=256)
    one = rt.bind_gated_mlp(family, counts, xr_, wg, wu, wd, yr_, max_tokens)
    two = rt.bind_gated_mlp(family, counts, xr_, wg, wu, wd, yr_, max_tokens, one_launch=False)
    assert len(two.steps) == 2
    wide = family == "w8a8" and hidden == 4096 and max_tokens > 256
    if family == "w8a8":
        assert len(one.steps) == 1, one.steps
        assert one.steps[0].name == "lf_fp8_w8a8_gated_mlp_b128" + ("_t256" if wide else ""), one.steps
    outs = []
    for op in (one, two, one):
        ya.copy_from_host(np.full(max_tokens * hidden, SENTINEL, np.uint16))
        op.launch(rt.stream, synchronous=True)
        outs.append(ya.read(np.uint16, (max_tokens, hidden)))
        assert np.all(outs[-1][m:] == SENTINEL), "rows past M written"
    assert np.array_equal(outs[0], outs[2])
    same_forms = all(("_t256" in st.name) == wide for st in two.steps)
    if same_forms:
        assert np.array_equal(outs[0], outs[1])
    y = outs[0][:m]
    # the device's h: the one-launch workspace (W8A8: sync area of three
    # steps, then the x rows: codes [cap, H], scales [H / 128][cap], cap =
    # bands x band height) or the chain's h allocation
    if family == "w8a8":
        height = 256 if wide else 128
        bands = -(-max_tokens // height)
        cap = height * bands
        at = 256 + 128 * 3 * bands
        at += -(-cap * hidden // 256) * 256 + -(-(hidden // 128) * cap * 4 // 256) * 256
        h_gpu = one.workspace.read(np.uint16, (m, inter), at)
        hq_at = at + -(-cap * inter * 2 // 256) * 256
        hq_gpu = one.workspace.read(np.uint8, (cap, inter), hq_at)[:m]
        hs_gpu = one.workspace.read(np.float32, (inter // 128, cap), hq_at + -(-cap * inter // 256) * 256)
        hs_gpu = np.ascontiguousarray(hs_gpu[:, :m].T)
    else:
        h_gpu = two.workspace.read(np.uint16, (m, inter))
    rows, hcols = sample(rng, m, inter, 24, 192)
    _, cols = sample(rng, m, hidden, 24, 128)
    xr = x_ref(x[rows], family)
    wgr, wur = deq_rows(qg, sg, hcols), deq_rows(qu, su, hcols)
    g, u = o.dense_projection(xr, wgr), o.dense_projection(xr, wur)
    tol = swiglu_midpoint_tol(g, u, abs_sum(xr, wgr), abs_sum(xr, wur), bound_k(hidden))
    wdr = deq_rows(qd, sd, cols)

    def check_stages(h_dev, y_dev, label, hq_dev=None, hs_dev=None):
        parity(h_dev[rows][:, hcols], o.silu_mul_array(g, u), label=label + " gate/up", midpoint_tol=tol)
        hb = o.bf16_decode(h_dev[rows])
        if family == "w8a8":
            hq_ref, hs_ref = o.quantize_rows(hb, group=128)
            if hq_dev is not None:
                np.testing.assert_array_equal(hq_dev[rows], hq_ref)
                np.testing.assert_array_equal(hs_dev[rows], hs_ref.reshape(len(rows), -1))
            hb = o.dequantize(hq_ref, hs_ref, mode=1, group=128)
        parity(y_dev[rows][:, cols], o.dense_projection(hb, wdr), k=bound_k(inter), s_abs=abs_sum(hb, wdr),
               label=label + " down")

    label = f"b128 gated mlp {family} h={hidden} m={m}"
    check_stages(h_gpu, y, label, *((hq_gpu, hs_gpu) if family == "w8a8" else ()))
    if not same_forms:
        check_stages(two.workspace.read(np.uint16, (m, inter)), outs[1][:m], label + " (two launches)")


@pytest.mark.parametrize("m,max_tokens", [(1, 16), (24, 32), (100, 128)])
def test_block_scaled_w8a16_gated_mlp_one_launch(rt, m, max_tokens):
    """W8A16 GatedMlp on block-scaled weights at the Llama-3-8B widths as one
    launch (LF_FP8_ENTRY_W8A16_GATED_MLP_B128): rows past M untouched, two
    launches on one workspace bit-identical, the same bits as the two
    block-scaled launches where both run the same down form (32 and 128
    rows; at 16 rows the two-launch down is the one-tile form, whose sum
    order differs), and the oracle stage by stage on the device's own h
    (the workspace's first [rows][I] bf16)."""
    hidden, inter = 4096, 14336
    rng = np.random.default_rng(14500 + m)
    (qg, sg), (qu, su) = spread_weight(rng, inter, hidden), spread_weight(rng, inter, hidden)
    qd, sd = spread_weight(rng, hidden, inter)
    wg, wu, wd = upload(rt, qg, sg), upload(rt, qu, su), upload(rt, qd, sd)
    x = spread_activations(rng, m, hidden)
    xa = rt.context.upload(np.concatenate([x, np.zeros((max_tokens - m, hidden), np.uint16)]))
    ya = rt.context.allocate(max_tokens * hidden * 2)
    counts = rt.step_counts(m)
    xr_, yr_ = _region(xa, alignment=256), _region(ya, alignment=256)
    one = rt.bind_gated_mlp("w8a16", counts, xr_, wg, wu, wd, yr_, max_tokens)
    two = rt.bind_gated_mlp("w8a16", counts, xr_, wg, wu, wd, yr_, max_tokens, one_launch=False)
    assert len(one.steps) == 1 and "gated_mlp_b128" in one.steps[0].name, one.steps
    assert len(two.steps) == 2
    outs = []
    for op in (one, one, two):
        ya.copy_from_host(np.full(max_tokens * hidden, SENTINEL, np.uint16))
        op.launch(rt.stream, synchronous=True)
        outs.append(ya.read(np.uint16, (max_tokens, hidden)))
        assert np.all(outs[-1][m:] == SENTINEL), "rows past M written"
    assert np.array_equal(outs[0], outs[1]), "a second launch on the same workspace differs"
    if max_tokens > 16:
        assert np.array_equal(outs[0], outs[2])
    y = outs[0][:m]
    h_gpu = one.workspace.read(np.uint16, (m, inter))
    rows, hcols = sample(rng, m, inter, 24, 192)
    xr = x_ref(x[rows], "w8a16")
    wgr, wur = deq_rows(qg, sg, hcols), deq_rows(qu, su, hcols)
    g, u = o.dense_projection(xr, wgr), o.dense_projection(xr, wur)
    tol = swiglu_midpoint_tol(g, u, abs_sum(xr, wgr), abs_sum(xr, wur), bound_k(hidden))
    label = f"b128 w8a16 gated mlp one launch m={m}/{max_tokens}"
    parity(h_gpu[rows][:, hcols], o.silu_mul_array(g, u), label=label + " gate/up", midpoint_tol=tol)
    hb = o.bf16_decode(h_gpu[rows])
    _, cols = sample(rng, m, hidden, 24, 128)
    wdr = deq_rows(qd, sd, cols)
    parity(y[rows][:, cols], o.dense_projection(hb, wdr), k=bound_k(inter), s_abs=abs_sum(hb, wdr),
           label=label + " down")


def test_block_scaled_admission(rt):
    """A per-channel weight is refused by the block-scaled entries, a
    block-scaled one by the per-channel entries (UNSUPPORTED), and each
    binding picks the entry of its weight's scale mode."""
    rng = np.random.default_rng(15000)
    qb, sb = spread_weight(rng, 256, 256)
    wb = upload(rt, qb, sb)
    qc, sc = synth.weight(rng, 256, 256)
    wc = rt.upload_weight(qc, sc)
    for entry in (_abi.ENTRY_W8A16_DENSE_B128, _abi.ENTRY_W8A8_DENSE_B128, _abi.ENTRY_W8A8_GATED_MLP_B128):
        with pytest.raises(DeviceError) as e:
            wc.admit(entry)
        assert e.value.status == _abi.LF_UNSUPPORTED
        wb.admit(entry)
    for entry in (_abi.ENTRY_W8A16_DENSE, _abi.ENTRY_W8A8_DENSE_AQ, _abi.ENTRY_W8A8_GATED_MLP):
        with pytest.raises(DeviceError) as e:
            wb.admit(entry)
        assert e.value.status == _abi.LF_UNSUPPORTED


@pytest.mark.parametrize("n,max_tokens,m,symbol", [
    (512, 256, 200, "lf_fp8_w8a8_dense_b128_t256x128"), (4096, 3072, 3000, "lf_fp8_w8a8_dense_b128_t256"),
])
def test_block_scaled_w8a8_sticky_error(rt, n, max_tokens, m, symbol):
    """The counted wait of the block-scaled one-launch entry (both tile
    forms), forced from the host as for the _aq entries: a band counter
    preset far below its target runs the wait out, the binding raises and
    zero-fills its workspace, and the next launch is correct."""
    rng = np.random.default_rng(15100 + n)
    k = 256
    q, s = spread_weight(rng, n, k)
    w = upload(rt, q, s)
    xa = rt.context.allocate(max_tokens * k * 2)
    ya = rt.context.allocate(max_tokens * n * 2)
    x = spread_activations(rng, m, k)
    xa.copy_from_host(np.concatenate([x, np.zeros((max_tokens - m, k), np.uint16)]))
    one = rt.bind_dense("w8a8", rt.step_counts(m), _region(xa, alignment=256), w,
                        _region(ya, alignment=256), max_tokens)
    assert one.steps[0].name == symbol, one.steps[0].name
    one.launch(rt.stream, synchronous=True)
    want = ya.read(np.uint16, (max_tokens, n))
    ws = one.workspace
    ws.copy_from_host(np.array([-(1 << 30)], np.int32), offset=256)
    ya.copy_from_host(np.full(max_tokens * n, SENTINEL, np.uint16))
    with pytest.raises(DeviceError):
        one.launch(rt.stream, synchronous=True)
    assert not ws.read(np.uint8, (ws.byte_count,)).any(), "workspace not zero-filled"
    one.launch(rt.stream, synchronous=True)
    assert np.array_equal(ya.read(np.uint16, (max_tokens, n))[:m], want[:m])


def test_block_scaled_w8a8_gated_mlp_sticky_error(rt):
    """The same for the block-scaled GatedMlp on 256 x 256 tiles (hidden 4096,
    intermediate 2048, 3072 rows): the x band counter preset far below its
    target runs the gate/up wait out, every later step's wait sees the error
    word, the binding raises and zero-fills the workspace, and the next
    launch gives the first launch's bits."""
    rng = np.random.default_rng(15200)
    hidden, inter, max_tokens, m = 4096, 2048, 3072, 3000
    (qg, sg), (qu, su) = spread_weight(rng, inter, hidden), spread_weight(rng, inter, hidden)
    qd, sd = spread_weight(rng, hidden, inter)
    wg, wu, wd = upload(rt, qg, sg), upload(rt, qu, su), upload(rt, qd, sd)
    x = spread_activations(rng, m, hidden)
    xa = rt.context.upload(np.concatenate([x, np.zeros((max_tokens - m, hidden), np.uint16)]))
    ya = rt.context.allocate(max_tokens * hidden * 2)
    one = rt.bind_gated_mlp("w8a8", rt.step_counts(m), _region(xa, alignment=256), wg, wu, wd,
                            _region(ya, alignment=256), max_tokens)
    assert len(one.steps) == 1 and one.steps[0].name == "lf_fp8_w8a8_gated_mlp_b128_t256", one.steps
    one.launch(rt.stream, synchronous=True)
    want = ya.read(np.uint16, (max_tokens, hidden))
    ws = one.workspace
    ws.copy_from_host(np.array([-(1 << 30)], np.int32), offset=256)
    ya.copy_from_host(np.full(max_tokens * hidden, SENTINEL, np.uint16))
    with pytest.raises(DeviceError):
        one.launch(rt.stream, synchronous=True)
    assert not ws.read(np.uint8, (ws.byte_count,)).any(), "workspace not zero-filled"
    one.launch(rt.stream, synchronous=True)
    assert np.array_equal(ya.read(np.uint16, (max_tokens, hidden))[:m], want[:m])


def al256(v):
    return -(-v // 256) * 256


def direct_b128(rt, symbol, operands, grid, block, ws_bytes):
    """A one-launch bound by hand (the 128 x 128 forms, which the geometry
    picks only for K >= 2^24): zero-filled workspace, error word at 0."""
    from lunaflux_amd.device import KernelArguments, KernelLaunchDimensions
    from lunaflux_amd.fp8 import BoundOperation, LaunchStep
    ws = rt.context.allocate(ws_bytes)
    ws.copy_from_host(np.zeros(ws_bytes, np.uint8))
    dims = KernelLaunchDimensions.new((grid, 1, 1), (block, 1, 1), 0)
    step = LaunchStep(rt.function(symbol), dims, KernelArguments(operands + [_region(ws, alignment=256)]), symbol)
    return BoundOperation([step], workspace=ws, error_offset=_abi.LF_FP8_AQ_ERROR_OFFSET)


@pytest.mark.parametrize("op,m,max_tokens", [("o", 300, 384), ("qkv", 129, 256), ("gate_up", 100, 128)])
def test_block_scaled_w8a8_t128_fallback(rt, op, m, max_tokens):
    """The 128 x 128 block-scaled entries (lf_fp8_w8a8_{op}_b128, the
    geometry's form for K >= 2^24), launched with the grid and workspace the
    geometry would give them (256 quantizer blocks, then column blocks x
    128-row bands; sync area of one step, codes [cap, K], scales [K / 128]
    [cap]): codes and scales bit-exact, outputs against the oracle, rows
    past M untouched, a second launch bit-identical."""
    from lunaflux_amd.fp8 import COUNTS_BYTES
    rng = np.random.default_rng(16000 + m + len(op))
    n, k = SHAPES[op]
    x = spread_activations(rng, m, k, zero_groups=True)
    xa = rt.context.upload(np.concatenate([x, np.zeros((max_tokens - m, k), np.uint16)]))
    ya = rt.context.allocate(max_tokens * n * 2)
    ya.copy_from_host(np.full(max_tokens * n, SENTINEL, np.uint16))
    counts = rt.step_counts(m)
    c = _region(counts, COUNTS_BYTES, alignment=4)
    if op == "qkv":
        ws = [spread_weight(rng, nn, k, zero_block=True) for nn in (4096, 1024, 1024)]
        regions = [upload(rt, q, s).region for q, s in ws]
        symbol, gx = "lf_fp8_w8a8_qkv_b128", n // 128
    elif op == "gate_up":
        ws = [spread_weight(rng, n, k) for _ in range(2)]
        regions = [upload(rt, q, s).region for q, s in ws]
        symbol, gx = "lf_fp8_w8a8_gate_up_b128", n // 64
    else:
        ws = [spread_weight(rng, n, k)]
        regions = [upload(rt, *ws[0]).region]
        symbol, gx = "lf_fp8_w8a8_dense_b128", n // 128
    bands = -(-max_tokens // 128)
    cap = 128 * bands
    ws_bytes = 256 + 128 * bands + al256(cap * k) + al256((k // 128) * cap * 4)
    bound = direct_b128(rt, symbol, [c, _region(xa, alignment=256), *regions, _region(ya, alignment=256)],
                        256 + gx * bands, 256, ws_bytes)
    bound.launch(rt.stream, synchronous=True)
    y = ya.read(np.uint16, (max_tokens, n))
    assert np.all(y[m:] == SENTINEL), "rows past M written"
    bound.launch(rt.stream, synchronous=True)
    assert np.array_equal(ya.read(np.uint16, (max_tokens, n)), y)
    codes, scales = w8a8_quantized_rows(bound, m, k, max_tokens)
    q_ref, s_ref = o.quantize_rows(o.bf16_decode(x), group=128)
    np.testing.assert_array_equal(codes, q_ref)
    np.testing.assert_array_equal(scales, s_ref.reshape(m, -1))
    rows, cols = sample(rng, m, n, 48, 256)
    check_op(op, "w8a8", y[:m], x, ws, rows, cols, f"b128 t128 w8a8 {op} m={m}/{max_tokens}")


@pytest.mark.parametrize("op,m,max_tokens", [("o", 2000, 2048), ("gate_up", 200, 256), ("qkv", 1000, 1024),
                                             ("down", 500, 512)])
def test_block_scaled_w8a8_256x128_matches_256x256(rt, op, m, max_tokens):
    """The 256 x 128 entries (which the geometry binds here) against the
    256 x 256 entry of the same operation launched by hand on the same
    inputs: both run the same per-element sums (the same k-tile rescales and
    MFMA order), so the former's launches (two on one workspace, one on a
    fresh one) must all give the latter's bits."""
    from lunaflux_amd.fp8 import COUNTS_BYTES
    rng = np.random.default_rng(17000 + m)
    y, x, ws, bound = run_op(rt, rng, op, "w8a8", m, max_tokens)
    assert bound.steps[0].name.endswith("_t256x128"), bound.steps[0].name
    n, k = SHAPES[op]
    xa = rt.context.upload(np.concatenate([x, np.zeros((max_tokens - m, k), np.uint16)]))
    ya = rt.context.allocate(max_tokens * n * 2)
    c = _region(rt.step_counts(m), COUNTS_BYTES, alignment=4)
    regions = [upload(rt, q, s).region for q, s in ws]
    bands = -(-max_tokens // 256)
    cap = 256 * bands
    gx = n // 128 if op == "gate_up" else n // 256
    symbol = "lf_fp8_w8a8_%s_b128_t256" % ("dense" if op in ("o", "down") else op)
    ws_bytes = 256 + 128 * bands + al256(cap * k) + al256((k // 128) * cap * 4)
    wide = direct_b128(rt, symbol, [c, _region(xa, alignment=256), *regions, _region(ya, alignment=256)],
                       256 + gx * bands, 512, ws_bytes)
    wide.launch(rt.stream, synchronous=True)
    want = ya.read(np.uint16, (max_tokens, n))[:m]
    assert np.array_equal(y, want)
    # (run_op launched twice on its workspace and compared; a fresh bind on
    # the same inputs)
    y2 = run_op(rt, np.random.default_rng(17000 + m), op, "w8a8", m, max_tokens)[0]
    assert np.array_equal(y2, want)

"""One launch per plan operation (kernels/launch_contract/types.mbt:16-27:
one AOT entry point per (profile, operation)).

The W8A8 operations quantize their bf16 input inside the launch (_aq
entries) and the W8A8 GatedMlp runs its four steps (x quantizer, gate/up +
SwiGLU, h quantizer, down) in one grid, ordered by counted waits
(csrc/kernels/phases.h). Each one-launch form must give the same bits as the
launches it replaces (the same quantizer and GEMM code run in both), on
every tile form the geometry picks, with ragged and zero live rows, rows past
M untouched, and a different x on every launch of one binding (its counters
must be back at rest after each launch). The error path is forced from the
host: a preset error word makes a launch store nothing; a band counter
preset far below its target makes the bounded wait run out (the kernel still
ends), and the binding then raises and zero-fills its workspace.
"""
import numpy as np
import pytest

import oracle_lib as o
from lunaflux_amd import _abi, fp8, synth
from lunaflux_amd.device import DeviceError
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


class Buffers:
    """Activation and output regions sized for a profile, as the engine's."""

    def __init__(self, rt, max_tokens, k, n):
        self.rt, self.max_tokens, self.k, self.n = rt, max_tokens, k, n
        self.xa = rt.context.allocate(max_tokens * k * 2)
        self.ya = rt.context.allocate(max_tokens * n * 2)
        self.counts = {}

    def counts_for(self, m):
        if m not in self.counts:
            self.counts[m] = self.rt.step_counts(m)
        return self.counts[m]

    def run(self, op, x):
        m = x.shape[0]
        self.xa.copy_from_host(np.concatenate([x, np.zeros((self.max_tokens - m, self.k), np.uint16)]))
        self.ya.copy_from_host(np.full(self.max_tokens * self.n, SENTINEL, np.uint16))
        op.launch(self.rt.stream, synchronous=True)
        y = self.ya.read(np.uint16, (self.max_tokens, self.n))
        assert np.all(y[m:] == SENTINEL), "rows past M written"
        return y[:m]


def bind(rt, op, buf, m, ws, one_launch):
    c = buf.counts_for(m)
    x, y = _region(buf.xa, alignment=256), _region(buf.ya, alignment=256)
    if op == "dense":
        return rt.bind_dense("w8a8", c, x, ws[0], y, buf.max_tokens, one_launch=one_launch)
    if op == "qkv":
        return rt.bind_qkv("w8a8", c, x, *ws, y, buf.max_tokens, one_launch=one_launch)
    return rt.bind_gate_up("w8a8", c, x, *ws, y, buf.max_tokens, one_launch=one_launch)


FORMS = [("_t256", 4096), ("_t256w8", 3072), ("_t256x128", 2048), ("_t128", 512)]


@pytest.mark.parametrize("op", ["dense", "qkv", "gate_up"])
@pytest.mark.parametrize("form,max_tokens", FORMS)
def test_aq_entry_equals_two_launches(rt, op, form, max_tokens):
    """The _aq entry of each tile form against act-quant + GEMM-only, three
    launches of one binding with a different x and live M each (the last a
    ragged band), then M = 0; the oracle on a sample of the first."""
    if op == "gate_up" and form == "_t256x128":
        pytest.skip("gate/up has no 256 x 128 form")
    rng = np.random.default_rng(9100 + max_tokens + len(op))
    k = 384
    if op == "dense":
        ns = (4096,)
    elif op == "qkv":
        ns = (2176, 960, 960)
    else:
        ns = (2048, 2048)
    n_out = sum(ns) if op != "gate_up" else ns[0]
    ws = [weight(rt, rng, n, k) for n in ns]
    entry = {"dense": _abi.ENTRY_W8A8_DENSE_AQ, "qkv": _abi.ENTRY_W8A8_QKV_AQ,
             "gate_up": _abi.ENTRY_W8A8_GATE_UP_AQ}[op]
    split = (ns[0], ns[1]) if op == "qkv" else None
    n_geo = sum(ns) if op == "qkv" else ns[0]
    dims, sym = fp8.launch_geometry(entry, n_geo, k, max_tokens, qkv_split=split)
    assert sym.endswith(form + "_aq"), sym
    buf = Buffers(rt, max_tokens, k, n_out)
    for m in (max_tokens, max_tokens - 37, 1, 0):
        one = bind(rt, op, buf, m, [w for _, _, w in ws], True)
        two = bind(rt, op, buf, m, [w for _, _, w in ws], False)
        assert len(one.steps) == 1 and one.steps[0].name == sym, one.steps
        assert len(two.steps) == 2
        x = synth.activations(rng, max(m, 1), k)[:m]
        y1 = buf.run(one, x)
        y2 = buf.run(two, x)
        assert np.array_equal(y1, y2), f"{op}{form} m={m}: one launch differs from two"
        if m == max_tokens - 37:
            # a second and third launch of the same binding, new inputs
            for _ in range(2):
                x = synth.activations(rng, m, k)
                assert np.array_equal(buf.run(one, x), buf.run(two, x))
            rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, 30, replace=False)]))
            xq, xs = o.quantize_rows(o.bf16_decode(x[rows]))
            xr = o.dequantize(xq, xs)
            y1 = buf.run(one, x)
            if op == "gate_up":
                (qg, sg, _), (qu, su, _) = ws
                cols = np.sort(rng.choice(ns[0], 128, replace=False))
                ref = o.silu_mul_array(o.dense_projection(xr, o.dequantize(qg[cols], sg[cols])),
                                       o.dense_projection(xr, o.dequantize(qu[cols], su[cols])))
                parity(y1[rows][:, cols], ref, label=f"{op}{form}_aq")
            else:
                qall = np.concatenate([q for q, _, _ in ws])
                sall = np.concatenate([s for _, s, _ in ws])
                cols = np.sort(rng.choice(n_out, 128, replace=False))
                wr = o.dequantize(qall[cols], sall[cols])
                parity(y1[rows][:, cols], o.dense_projection(xr, wr), k=k, s_abs=abs_sum(xr, wr),
                       label=f"{op}{form}_aq")


GATED = [
    # (hidden, inter, max_tokens, symbol): each the forms the separate
    # launches also pick, so the outputs are bit-identical
    (2048, 2048, 8192, "lf_fp8_w8a8_gated_mlp_t256_t256"),
    (1024, 2048, 4096, "lf_fp8_w8a8_gated_mlp_t256_t256x128"),
    (512, 1024, 256, "lf_fp8_w8a8_gated_mlp_t128_t128"),
]


@pytest.mark.parametrize("hidden,inter,max_tokens,symbol", GATED)
def test_w8a8_gated_mlp_one_launch(rt, hidden, inter, max_tokens, symbol):
    """W8A8 GatedMlp as one launch against its four launches (x act-quant,
    gate/up, h act-quant, down), bit for bit, over successive launches with
    new x and live M; the oracle stage by stage on sampled rows and columns:
    gate/up against the oracle, the h codes and scales bit-exact against the
    oracle quantizer on the device's bf16 h, down on those codes."""
    rng = np.random.default_rng(9300 + max_tokens)
    qg, sg, wg = weight(rt, rng, inter, hidden)
    qu, su, wu = weight(rt, rng, inter, hidden)
    qd, sd, wd = weight(rt, rng, hidden, inter)
    buf = Buffers(rt, max_tokens, hidden, hidden)
    for m in (max_tokens, max_tokens - 200, 17, 0):
        c = buf.counts_for(m)
        x_r, y_r = _region(buf.xa, alignment=256), _region(buf.ya, alignment=256)
        one = rt.bind_gated_mlp("w8a8", c, x_r, wg, wu, wd, y_r, max_tokens)
        four = rt.bind_gated_mlp("w8a8", c, x_r, wg, wu, wd, y_r, max_tokens, one_launch=False)
        assert len(one.steps) == 1 and one.steps[0].name == symbol, one.steps
        assert len(four.steps) == 4
        for _ in range(2):
            x = synth.activations(rng, max(m, 1), hidden)[:m]
            y1 = buf.run(one, x)
            y4 = buf.run(four, x)
            assert np.array_equal(y1, y4), f"{symbol} m={m}: one launch differs from four"
        if m == max_tokens - 200:
            # Stage by stage on the device's own intermediates (read from the
            # workspace: sync area, xq, h bf16 [cap, I], hq): an h that
            # differs from the oracle's by one bf16 ulp can move an e4m3
            # code of the re-quantized h, so the end-to-end check runs on the
            # GPU's h, as the separate launches would be checked.
            bm = 128 if "t128_t128" in symbol else 256
            bands = -(-max_tokens // bm)
            cap = bands * bm
            sync = 256 + 128 * 3 * bands   # error, done, one line per band counter
            xq_bytes = -(-cap * hidden // 256) * 256 + -(-cap * 4 // 256) * 256
            h_gpu = one.workspace.read(np.uint16, (m, inter), sync + xq_bytes)
            hq_at = sync + xq_bytes + -(-cap * inter * 2 // 256) * 256
            hq_gpu = one.workspace.read(np.uint8, (m, inter), hq_at)
            hs_gpu = one.workspace.read(np.float32, (m,), hq_at + -(-m * inter // 256) * 256)
            rows = np.unique(np.concatenate([[0, m - 1], rng.choice(m, 12, replace=False)]))
            xq, xs = o.quantize_rows(o.bf16_decode(x[rows]))
            xr = o.dequantize(xq, xs)
            hcols = np.sort(rng.choice(inter, 128, replace=False))
            h = o.silu_mul_array(o.dense_projection(xr, o.dequantize(qg[hcols], sg[hcols])),
                                 o.dense_projection(xr, o.dequantize(qu[hcols], su[hcols])))
            parity(h_gpu[rows][:, hcols], h, label=f"{symbol} gate/up")
            hq_ref, hs_ref = o.quantize_rows(o.bf16_decode(h_gpu[rows]))
            np.testing.assert_array_equal(hq_gpu[rows], hq_ref)
            np.testing.assert_array_equal(hs_gpu[rows], hs_ref)
            hr = o.dequantize(hq_ref, hs_ref)
            cols = np.sort(rng.choice(hidden, 96, replace=False))
            wdr = o.dequantize(qd[cols], sd[cols])
            parity(y1[rows][:, cols], o.dense_projection(hr, wdr), k=inter, s_abs=abs_sum(hr, wdr),
                   label=f"{symbol} down")


def test_aq_sticky_error_and_timeout(rt):
    """The counted waits' failure path, forced from the host. (1) An error
    word left set: the launch stores nothing, the binding raises and
    zero-fills its workspace, and the next launch is correct. (2) A band
    counter preset far below its target: the GEMM tiles of that band poll
    until their bound runs out (every kernel still ends), the error word is
    set, the binding raises and restores the workspace, and the next launch
    is correct again."""
    rng = np.random.default_rng(9500)
    k, n, max_tokens, m = 256, 512, 256, 200
    _, _, w = weight(rt, rng, n, k)
    buf = Buffers(rt, max_tokens, k, n)
    c = buf.counts_for(m)
    one = rt.bind_dense("w8a8", c, _region(buf.xa, alignment=256), w, _region(buf.ya, alignment=256),
                        max_tokens)
    two = rt.bind_dense("w8a8", c, _region(buf.xa, alignment=256), w, _region(buf.ya, alignment=256),
                        max_tokens, one_launch=False)
    x = synth.activations(rng, m, k)
    want = buf.run(two, x)
    ws = one.workspace
    # (1) error word set before the launch
    ws.copy_from_host(np.array([1], np.int32), offset=_abi.LF_FP8_AQ_ERROR_OFFSET)
    buf.xa.copy_from_host(np.concatenate([x, np.zeros((max_tokens - m, k), np.uint16)]))
    buf.ya.copy_from_host(np.full(max_tokens * n, SENTINEL, np.uint16))
    with pytest.raises(DeviceError):
        one.launch(rt.stream, synchronous=True)
    assert np.all(buf.ya.read(np.uint16, (max_tokens, n)) == SENTINEL), "a failed workspace wrote y"
    assert not ws.read(np.uint8, (ws.byte_count,)).any(), "workspace not zero-filled"
    assert np.array_equal(buf.run(one, x), want)
    # (2) band 0's counter can never reach its target: the sync area is
    # [error line, done line, one 128-byte line per band counter]
    ws.copy_from_host(np.array([-(1 << 30)], np.int32), offset=256)
    buf.ya.copy_from_host(np.full(max_tokens * n, SENTINEL, np.uint16))
    with pytest.raises(DeviceError):
        one.launch(rt.stream, synchronous=True)
    y = buf.ya.read(np.uint16, (max_tokens, n))
    assert np.all(y[:128] == SENTINEL), "band 0 stored after its wait ran out"
    assert np.array_equal(buf.run(one, x), want)
    one.check()


@pytest.mark.parametrize("max_tokens,m", [(32, 24), (128, 100)])
def test_w8a16_gated_mlp_sticky_error_and_timeout(rt, max_tokens, m):
    """The same failure path for the one-launch W8A16 GatedMlp: a preset
    error word stores nothing; a slice counter preset far below its target
    makes the down blocks of that slice run out of polls without loading h
    or storing; the binding raises, zero-fills, and the next launch is
    bit-identical to the two launches."""
    rng = np.random.default_rng(9600 + max_tokens)
    hidden, inter = 4096, 14336
    _, _, wg = weight(rt, rng, inter, hidden)
    _, _, wu = weight(rt, rng, inter, hidden)
    _, _, wd = weight(rt, rng, hidden, inter)
    buf = Buffers(rt, max_tokens, hidden, hidden)
    c = buf.counts_for(m)
    args = (c, _region(buf.xa, alignment=256), wg, wu, wd, _region(buf.ya, alignment=256), max_tokens)
    one = rt.bind_gated_mlp("w8a16", *args)
    two = rt.bind_gated_mlp("w8a16", *args, one_launch=False)
    assert len(one.steps) == 1 and len(two.steps) == 2
    x = synth.activations(rng, m, hidden)
    want = buf.run(two, x)
    ws = one.workspace
    err_at = ws.byte_count - _abi.LF_FP8_GATED_MLP_ERROR_OFFSET_FROM_END
    ws.copy_from_host(np.array([1], np.int32), offset=err_at)
    buf.ya.copy_from_host(np.full(max_tokens * hidden, SENTINEL, np.uint16))
    with pytest.raises(DeviceError):
        one.launch(rt.stream, synchronous=True)
    assert np.all(buf.ya.read(np.uint16, (max_tokens, hidden)) == SENTINEL)
    assert np.array_equal(buf.run(one, x), want)
    # slice counter 0 opens the sync area: 768 bytes (four slice lines, done,
    # error, spare) in the column-group form, 128 S + 256 in the 128-row form
    if max_tokens == 32:
        sync = 768
    else:
        dn_dims, dn_sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, hidden, inter, max_tokens)
        bn = int(dn_sym.rsplit("_n", 1)[1])  # the down GEMM's block width
        sync = 128 * (dn_dims.grid[0] // (hidden // bn)) + 256
    ws.copy_from_host(np.array([-(1 << 30)], np.int32), offset=ws.byte_count - sync)
    with pytest.raises(DeviceError):
        one.launch(rt.stream, synchronous=True)
    assert np.array_equal(buf.run(one, x), want)
    for _ in range(2):
        x = synth.activations(rng, m, hidden)
        assert np.array_equal(buf.run(one, x), buf.run(two, x))

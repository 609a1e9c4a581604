"""Benchmark of the FP8 projection hot path on one MI355X.

Metric: FP8 projection GB/s & TFLOP/s (% roofline),
Llama-3-8B shapes, 1 GPU. Workload of `value`: one
Llama-3-8B decode layer's four projection calls on the W8A16 family - fused
QKV (4096 -> 6144), O (4096 -> 4096), gate/up with SwiGLU (4096 -> 2 x 14336
-> 14336) and down (14336 -> 4096) - at M = 32 tokens, bf16 activations from
N(0, 1), e4m3 weights from N(0, 0.02) with per-output-channel fp32 scales
(synthetic, seeded; no checkpoint exists offline). One step = the four calls.
Weights are rotated over 24 device copies of the layer (5.2 GB, 20x the
256 MB MALL) so each step streams its weights from HBM.

value = algorithmic bytes of the step / step time, with algorithmic bytes per
call = N*K (e4m3 weights) + 4*N (scales) + 2*M*K (x) + 2*M*N_out (y), each
weight byte counted once. The roofline object is the dominant kernel (gate/up)
timed with HIP events on the launch stream. `detail` holds the other decode
M values (and the GatedMlp operation as one launch against two), the
prefill (W8A8) GEMMs in TFLOP/s, the act-quant pass, each
operation's TFLOP/s with it as two launches and as the plan's one launch
(act-quant inside), and the W8A8 GatedMlp as one launch against four. cpu_baseline times the
CPU oracle (C restatement of kernels/reference over dequantized weights) on
the host cores, with one-thread figures for configs 1 and 2 beside it.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
ROTATIONS = 24  # weight copies cycled per call: 24 x 218 MB keeps the 256 MB MALL from serving reuse
HIDDEN, INTER, NQ, NKV = 4096, 14336, 4096, 1024
METRIC = "FP8 proj GB/s & TFLOP/s (% roofline), Llama-3-8B shapes M=1..8192, 1 GPU"
PMC_COPY_BYTES = 512 << 20  # calibration copy of the counter passes


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def call_shapes():
    """(name, K, N weight rows, N_out) for the four calls of one layer."""
    return [("qkv", HIDDEN, NQ + 2 * NKV, NQ + 2 * NKV), ("o", HIDDEN, HIDDEN, HIDDEN),
            ("gate_up", HIDDEN, 2 * INTER, INTER), ("down", INTER, HIDDEN, HIDDEN)]


def call_bytes(m, k, n, n_out):
    return n * k + 4 * n + 2 * m * k + 2 * m * n_out


def layer_bytes(m):
    return sum(call_bytes(m, k, n, no) for _, k, n, no in call_shapes())


def call_flops(m, k, n):
    return 2 * m * n * k


def roofline_kernel():
    """Symbol of the dominant kernel of the headline workload: the W8A16
    gate/up launch of a 32-row profile (host-side geometry, no GPU needed)."""
    from lunaflux_amd import _abi, fp8
    return fp8.launch_geometry(_abi.ENTRY_W8A16_GATE_UP, INTER, HIDDEN, 32)[1]


class Layer:
    """Device-resident weights of one layer, `rotations` copies each."""

    def __init__(self, rt, seed=1234, rotations=ROTATIONS, block=False):
        """block: 128 x 128 block scales (the _b128 entries) instead of
        per-channel scales."""
        from lunaflux_amd import fp8, synth
        rng = np.random.default_rng(seed)
        t0 = time.time()
        self.rotations = rotations
        self.regions = {}
        for name, rows, cols in [("q", NQ, HIDDEN), ("k", NKV, HIDDEN), ("v", NKV, HIDDEN),
                                 ("o", HIDDEN, HIDDEN), ("gate", INTER, HIDDEN),
                                 ("up", INTER, HIDDEN), ("down", HIDDEN, INTER)]:
            q, s = synth.weight(rng, rows, cols, block=128 if block else None)
            region = fp8.pack_weight(q, s, fp8.BLOCK128 if block else fp8.PER_CHANNEL)
            self.regions[name] = [rt.weight_from_region(region) for _ in range(rotations)]
        log(f"weights ready ({rotations} copies of one {'block-scaled ' if block else ''}layer) "
            f"in {time.time() - t0:.1f}s")

    def w(self, name, r):
        return self.regions[name][r % self.rotations]


class Bench:
    """One profile's bound calls over the rotated weights. one_launch: the
    plan's binding, one launch per operation (the W8A8 calls quantize their
    input inside the launch); False: the W8A8 calls as an act-quant launch
    plus a GEMM-only launch. `share`: another Bench of the same profile whose
    activation and output buffers this one reuses."""

    def __init__(self, rt, layer, max_tokens, family, one_launch=True, share=None):
        from lunaflux_amd import synth
        from lunaflux_amd.fp8 import _region
        self.rt, self.layer, self.family, self.one_launch = rt, layer, family, one_launch
        ctx = rt.context
        if share is not None:
            self.x, self.xd, self.out = share.x, share.xd, share.out
        else:
            rng = np.random.default_rng(99 + max_tokens)
            self.x = ctx.upload(synth.activations(rng, max_tokens, HIDDEN))
            self.xd = ctx.upload(synth.activations(rng, max_tokens, INTER))
            self.out = {n: ctx.allocate(max_tokens * no * 2) for n, _, _, no in call_shapes()}
        self.max_tokens = max_tokens
        self._region = _region
        self.ops = {}
        self.mlp_ops = {}

    def bind(self, m):
        rt, L, R = self.rt, self.layer, self._region
        counts = rt.step_counts(m)
        ops = []
        for r in range(L.rotations):
            fam, mt = self.family, self.max_tokens
            x, xd = R(self.x, alignment=256), R(self.xd, alignment=256)
            one = self.one_launch
            ops.append({
                "qkv": rt.bind_qkv(fam, counts, x, L.w("q", r), L.w("k", r), L.w("v", r),
                                   R(self.out["qkv"], alignment=256), mt, one_launch=one),
                "o": rt.bind_dense(fam, counts, x, L.w("o", r), R(self.out["o"], alignment=256), mt,
                                   one_launch=one),
                "gate_up": rt.bind_gate_up(fam, counts, x, L.w("gate", r), L.w("up", r),
                                           R(self.out["gate_up"], alignment=256), mt, one_launch=one),
                "down": rt.bind_dense(fam, counts, xd, L.w("down", r),
                                      R(self.out["down"], alignment=256), mt, one_launch=one),
            })
        self.ops[m] = (counts, ops)
        return ops

    def bind_mlp(self, m, one_launch):
        """The GatedMlp operation (gate/up + SwiGLU + down, x [M, 4096] ->
        y [M, 4096]) for each weight rotation."""
        key = (m, one_launch)
        if key not in self.mlp_ops:
            rt, L, R = self.rt, self.layer, self._region
            counts = rt.step_counts(m)
            self.mlp_ops[key] = [
                rt.bind_gated_mlp(self.family, counts, R(self.x, alignment=256), L.w("gate", r),
                                  L.w("up", r), L.w("down", r), R(self.out["o"], alignment=256),
                                  self.max_tokens, one_launch=one_launch)
                for r in range(L.rotations)]
        return self.mlp_ops[key]

    def time_ops(self, ops, launches, warmup=3):
        """Average time of one whole bound operation (all of its launch steps),
        `launches` back to back over the rotations: HIP events on the launch
        stream. Checks the counted waits' error words afterwards."""
        stream, ctx = self.rt.stream, self.rt.context
        for i in range(warmup):
            ops[i % len(ops)].launch(stream, synchronous=False)
        start, stop = ctx.create_event(), ctx.create_event()
        start.record(stream)
        for i in range(launches):
            ops[i % len(ops)].launch(stream, synchronous=False)
        stop.record(stream)
        stop.synchronize()
        for op in ops:
            op.check()
        return start.elapsed_milliseconds(stop) / launches

    def run(self, m, steps, warmup, calls=("qkv", "o", "gate_up", "down"), probe="gate_up"):
        """Times `steps` steps of the given calls; returns (total ms, mean ms of
        each launch step of `probe` (events around it), per-step ms)."""
        rt = self.rt
        ops = self.ops.get(m, (None, None))[1] or self.bind(m)
        stream = rt.stream
        for i in range(warmup):
            for c in calls:
                ops[i % ROTATIONS][c].launch(stream, synchronous=False)
        stream.synchronize()
        ctx = rt.context
        start, stop = ctx.create_event(), ctx.create_event()
        probe_events = [(ctx.create_event(), ctx.create_event()) for _ in range(steps)]
        start.record(stream)
        for i in range(steps):
            for c in calls:
                op = ops[i % ROTATIONS][c]
                if c == probe:
                    pre = op.steps[:-1]
                    for s in pre:
                        s.launch(stream, synchronous=False)
                    probe_events[i][0].record(stream)
                    op.steps[-1].launch(stream, synchronous=False)
                    probe_events[i][1].record(stream)
                else:
                    op.launch(stream, synchronous=False)
        stop.record(stream)
        stop.synchronize()
        total = start.elapsed_milliseconds(stop)
        probe_ms = (sum(a.elapsed_milliseconds(b) for a, b in probe_events) / steps
                    if probe in calls else None)
        return total, probe_ms, total / steps


    def time_kernel(self, m, call, launches, warmup=5, step=-1):
        """Average duration of one launch of kernel `step` of `call` (by
        default the last, the GEMM): HIP events on the launch stream around
        `launches` back-to-back launches (rotating over the weight copies);
        the call's earlier steps (the act-quant prologue) run once
        beforehand, as their output is reused."""
        ops = self.ops.get(m, (None, None))[1] or self.bind(m)
        stream, ctx = self.rt.stream, self.rt.context
        for r in range(ROTATIONS):
            for s in ops[r][call].steps[:-1]:
                s.launch(stream, synchronous=False)
        for i in range(warmup):
            ops[i % ROTATIONS][call].steps[step].launch(stream, synchronous=False)
        start, stop = ctx.create_event(), ctx.create_event()
        start.record(stream)
        for i in range(launches):
            ops[i % ROTATIONS][call].steps[step].launch(stream, synchronous=False)
        stop.record(stream)
        stop.synchronize()
        return start.elapsed_milliseconds(stop) / launches


def block_scaled_bench(rt):
    """The Llama-3-8B layer on 128 x 128 block-scaled weights (the _b128
    entries the bindings pick for weight_scale_inv checkpoints): each
    operation as the plan binds it (one launch; W8A16 GatedMlp as its two
    block-scaled launches), decode in GB/s of algorithmic bytes (plus the
    block scales), prefill in TFLOP/s."""
    layer = Layer(rt, seed=4321, block=True)
    out = {}
    for mm, mt, fam in [(1, 16, "w8a16"), (32, 32, "w8a16"), (128, 128, "w8a16"),
                        (2048, 2048, "w8a8"), (8192, 8192, "w8a8")]:
        b = Bench(rt, layer, mt, fam)
        n = 20 if fam == "w8a16" else 5
        if fam == "w8a16":
            b.run(mm, 3 * ROTATIONS, 0, probe=None)  # untimed, as in the decode rows
        row = {}
        for c, k, nn, no in call_shapes():
            p = b.time_kernel(mm, c, n, warmup=2)
            if fam == "w8a16":
                byts = call_bytes(mm, k, nn, no) + (nn // 128) * (k // 128) * 4
                row[c] = {"us": round(p * 1e3, 2), "GB/s": round(byts / (p * 1e-3) / 1e9, 1)}
            else:
                tf = call_flops(mm, k, nn) / (p * 1e-3) / 1e12
                row[c] = {"us": round(p * 1e3, 1), "TFLOP/s": round(tf, 1),
                          "fp8_frac": round(tf / FP8_PEAK_TFLOPS, 4)}
        mlp = b.bind_mlp(mm, True)
        t1 = b.time_ops(mlp, n)
        row["gated_mlp"] = {"launches": len(mlp[0].steps), "us": round(t1 * 1e3, 1 if fam == "w8a8" else 2)}
        row["layer_us"] = round(row["qkv"]["us"] + row["o"]["us"] + t1 * 1e3, 2)
        out[f"{fam} M={mm}"] = row
        log(f"block-scaled {fam} M={mm}: {row}")
        del b
    return out


def rms_norm_quant_bench(rt, bench, m, launches=20):
    """The fused RmsNorm + per-token quantizer (eps 1e-5, K = 4096, the input
    of qkv and gate/up) at prefill size m: average launch time, rotating over
    enough bf16 input copies (>= 1 GB) that the MALL cannot serve them, and
    GB/s of algorithmic bytes (2 M K read + 2 K norm weight + M K codes + 4 M
    scales)."""
    from lunaflux_amd import synth
    from lunaflux_amd.fp8 import _region, act_quant_bytes
    ctx, stream = rt.context, rt.stream
    rng = np.random.default_rng(55)
    copies = min(32, max(2, -(-(1 << 30) // (2 * m * HIDDEN))))
    x0 = synth.activations(rng, m, HIDDEN)
    xs = [ctx.upload(x0) for _ in range(copies)]
    g = ctx.upload(synth.bf16_bits(rng.uniform(0.5, 1.5, HIDDEN).astype(np.float32)))
    xq = ctx.allocate(act_quant_bytes(m, HIDDEN))
    counts = rt.step_counts(m, decode=False)
    w = bench.layer.w("q", 0)
    steps = [rt.bind_rms_norm_quant(counts, _region(x, alignment=256), _region(g), w,
                                    _region(xq, alignment=256), m, 1e-5) for x in xs]
    for i in range(3):
        steps[i % copies].launch(stream, synchronous=False)
    start, stop = ctx.create_event(), ctx.create_event()
    start.record(stream)
    for i in range(launches):
        steps[i % copies].launch(stream, synchronous=False)
    stop.record(stream)
    stop.synchronize()
    us = start.elapsed_milliseconds(stop) / launches * 1e3
    nbytes = 3 * m * HIDDEN + 2 * HIDDEN + 4 * m
    return {"us": round(us, 1), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "kernel": steps[0].name}


VOCAB = 128256
LM_HEAD_ROTATIONS = 4  # 4 x 525 MB head weights: 8x the MALL


def lm_head_bench(rt, launches=20):
    """The Llama-3 vocabulary head (4096 -> 128,256, the dense entry) at
    decode sizes on the W8A16 family: average launch time over launches
    rotating between LM_HEAD_ROTATIONS weight copies, and algorithmic GB/s.
    The weight is a 2048-row draw tiled down the vocabulary (the values do
    not change the kernel's time)."""
    from lunaflux_amd import fp8, synth
    from lunaflux_amd.fp8 import _region
    rng = np.random.default_rng(31)
    q0, s0 = synth.weight(rng, 2048, HIDDEN)
    reps = VOCAB // 2048 + 1
    region = fp8.pack_weight(np.tile(q0, (reps, 1))[:VOCAB], np.tile(s0, reps)[:VOCAB])
    ws = [rt.weight_from_region(region) for _ in range(LM_HEAD_ROTATIONS)]
    del region
    ctx, stream = rt.context, rt.stream
    out = {}
    for m, mt in [(1, 16), (8, 16), (32, 32), (128, 128)]:
        x = ctx.upload(synth.activations(rng, mt, HIDDEN))
        y = ctx.allocate(mt * VOCAB * 2)
        counts = rt.step_counts(m)
        ops = [rt.bind_dense("w8a16", counts, _region(x, alignment=256), w,
                             _region(y, alignment=256), mt) for w in ws]
        # untimed launches first: at 128 rows 20-launch windows read 176,
        # 153, 147, 147 us one after another (the decode rows' warm-up)
        for i in range(60):
            ops[i % len(ops)].launch(stream, synchronous=False)
        start, stop = ctx.create_event(), ctx.create_event()
        start.record(stream)
        for i in range(launches):
            ops[i % len(ops)].launch(stream, synchronous=False)
        stop.record(stream)
        stop.synchronize()
        us = start.elapsed_milliseconds(stop) / launches * 1e3
        gbs = call_bytes(m, HIDDEN, VOCAB, VOCAB) / (us * 1e-6) / 1e9
        out[f"M={m}"] = {"us": round(us, 2), "GB/s": round(gbs, 1),
                         "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "kernel": ops[0].steps[-1].name}
    return out


def host_threads():
    """The host cores this process may use: the CPU affinity set, capped by
    OMP_NUM_THREADS where the machine sets it (the GPU box gives each GPU a
    share of its cores and says so there)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(cap))) if cap.isdigit() and int(cap) > 0 else n


def cpu_single_thread(seconds=4.0):
    """One-thread figures of the CPU oracle: BASELINE config 1 (M=4, K=512,
    N=1536) repeated for about `seconds`, and one config-2 decode layer at
    M=32 (the four calls once)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as o
    from lunaflux_amd import synth
    rng = np.random.default_rng(11)
    x = o.bf16_decode(synth.activations(rng, 4, 512))
    q, s = synth.weight(rng, 1536, 512)
    w = o.dequantize(q, s)
    reps, t_total = 0, 0.0
    while t_total < seconds:
        t0 = time.perf_counter()
        o.project_values(x, w)
        t_total += time.perf_counter() - t0
        reps += 1
    c1 = reps * call_bytes(4, 512, 1536, 1536) / t_total / 1e9
    xs = {HIDDEN: o.bf16_decode(synth.activations(rng, 32, HIDDEN)),
          INTER: o.bf16_decode(synth.activations(rng, 32, INTER))}
    t_layer = 0.0
    for name, k, n, n_out in call_shapes():
        qw, sw = synth.weight(rng, n, k)
        wd = o.dequantize(qw, sw)
        t0 = time.perf_counter()
        y = o.project_values(xs[k], wd)
        if name == "gate_up":
            o.silu_mul_array(y[:, :n_out], y[:, n_out:])
        t_layer += time.perf_counter() - t0
    return {"config1_GB/s": round(c1, 4), "config1_calls": reps,
            "config2_m32_layer_GB/s": round(layer_bytes(32) / t_layer / 1e9, 4),
            "config2_m32_layer_s": round(t_layer, 2), "threads": 1}


def cpu_baseline(m=32, threads=None):
    """The CPU oracle on this host: the four decode calls of one layer at
    M=m over dequantized fp32 weights (sequential-K fp32, as the reference),
    output elements split across threads."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as o
    from lunaflux_amd import synth
    threads = threads or host_threads()
    rng = np.random.default_rng(7)
    x = o.bf16_decode(synth.activations(rng, m, HIDDEN))
    xd = o.bf16_decode(synth.activations(rng, m, INTER))
    weights = []
    for name, k, n, n_out in call_shapes():
        q, s = synth.weight(rng, n, k)
        weights.append((name, n_out, o.dequantize(q, s)))
    passes, total_s = 0, 0.0
    # Repeat whole layers until about 20 s of CPU work (wall x threads).
    while passes == 0 or total_s * threads < 20.0:
        for name, n_out, w in weights:
            t0 = time.perf_counter()
            y = o.project_values_mt(xd if name == "down" else x, w, threads)
            if name == "gate_up":
                o.silu_mul_array(y[:, :n_out], y[:, n_out:])
            total_s += time.perf_counter() - t0
        passes += 1
    gbs = passes * layer_bytes(m) / total_s / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{passes} decode layers (qkv, o, gate/up+SwiGLU, down) at M={m}, full "
                      f"shapes: the CPU oracle's sequential-K fp32 project_values over dequantized "
                      f"weights; {total_s:.2f} s wall on {threads} threads",
            "single_thread": cpu_single_thread()}


MOE_CONFIGS = {
    # Mixtral-style, 8 experts, top-2, per-channel scales.
    "mixtral_e8_k2_t1024": dict(tokens=1024, experts=8, top_k=2, hidden=4096, inter=14336,
                                group=0, route_mode=0, popularity="bias"),
    # 64 experts, top-6, 128x128 block scales, Zipf(1.1).
    "fine_e64_k6_t4096": dict(tokens=4096, experts=64, top_k=6, hidden=2048, inter=1408,
                              group=128, route_mode=1, popularity="zipf"),
    "fine_e64_k6_t32": dict(tokens=32, experts=64, top_k=6, hidden=2048, inter=1408,
                            group=128, route_mode=1, popularity="zipf"),
}


def moe_flops(c):
    a = c["tokens"] * c["top_k"]
    return 2 * a * c["hidden"] * 2 * c["inter"] + 2 * a * c["inter"] * c["hidden"]


MOE_ROTATION_BYTES = 1 << 30  # expert weights cycled per step: 4x the 256 MB MALL


def moe_bench(rt, c, steps=12, warmup=3, seed=4242):
    """Times the launches of one MoE expert-MLP operation with events
    between them. Expert weights are E copies of one seeded draw (kernel time
    does not depend on the values; it keeps setup short); enough such weight
    sets to total MOE_ROTATION_BYTES are cycled over the steps, so no step
    finds its experts' weights in the MALL from the step before."""
    from lunaflux_amd import fp8, moe, synth
    from lunaflux_amd.fp8 import _region
    rng = np.random.default_rng(seed)
    e, k, h, i, t = c["experts"], c["top_k"], c["hidden"], c["inter"], c["tokens"]
    block = 128 if c["group"] else None
    mode = fp8.BLOCK128 if block else fp8.PER_CHANNEL
    regions = []
    for rows, cols in ((i, h), (i, h), (h, i)):
        q, s = synth.weight(rng, rows, cols, block=block)
        regions.append(fp8.pack_weight(np.broadcast_to(q, (e,) + q.shape),
                                       np.broadcast_to(s, (e,) + s.shape), mode))
    sets = max(1, -(-MOE_ROTATION_BYTES // sum(r.size for r in regions)))
    weight_sets = [[rt.weight_from_region(r) for r in regions] for _ in range(sets)]
    logits = rng.standard_normal((t, e)).astype(np.float32)
    if c["popularity"] == "bias":
        logits += rng.normal(0.0, 1.5, e).astype(np.float32)
    else:  # Zipf(1.1) popularity: log-probability bias by expert rank
        logits += np.log(1.0 / np.arange(1, e + 1) ** 1.1).astype(np.float32)[rng.permutation(e)]
    desc = moe.moe_descriptor(e, k, c["route_mode"], h, i, c["group"])
    ctx = rt.context
    xa = ctx.upload(synth.activations(rng, t, h))
    la = ctx.upload(logits)
    da = ctx.upload(desc.as_bytes())
    oa = ctx.allocate(t * h * 2)
    counts = rt.step_counts(t, decode=False)
    ops = [moe.bind_moe(rt, counts, desc, _region(da, 32, alignment=4), _region(la, alignment=256),
                        _region(xa, alignment=256), *weights, _region(oa, alignment=256), t)
           for weights in weight_sets]
    op = ops[0]
    stream = rt.stream
    for it in range(warmup):
        ops[it % sets].launch(stream, synchronous=False)
    stream.synchronize()
    events = [[ctx.create_event() for _ in range(len(op.steps) + 1)] for _ in range(steps)]
    for it in range(steps):
        events[it][0].record(stream)
        for s_i, step in enumerate(ops[it % sets].steps):
            step.launch(stream, synchronous=False)
            events[it][s_i + 1].record(stream)
    events[-1][-1].synchronize()
    per = [sum(events[it][s_i].elapsed_milliseconds(events[it][s_i + 1]) for it in range(steps)) / steps
           for s_i in range(len(op.steps))]
    names = [s.name for s in op.steps]
    total_ms = sum(per)
    gemm_ms = sum(p for n, p in zip((s.name for s in op.steps), per)
                  if n.startswith(("lf_moe_gate_up", "lf_moe_down")))
    fl = moe_flops(c)
    return {"total_us": round(total_ms * 1e3, 1),
            "steps_us": {n: round(p * 1e3, 1) for n, p in zip(names, per)},
            "gemm_us": round(gemm_ms * 1e3, 1),
            "gemm_TFLOP/s": round(fl / (gemm_ms * 1e-3) / 1e12, 1),
            "gemm_fp8_frac": round(fl / (gemm_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
            "total_TFLOP/s": round(fl / (total_ms * 1e-3) / 1e12, 1),
            "GFLOP": round(fl / 1e9, 1), "weight_sets": sets}


def pmc_pass():
    """Short run for hardware-counter passes: the roofline kernel (W8A16
    gate/up at M=32) 10 times, then the calibration copy of 512 MiB 3 times."""
    from lunaflux_amd import _abi, fp8, synth
    from lunaflux_amd.device import KernelArguments, KernelLaunchDimensions
    from lunaflux_amd.fp8 import ProjectionRuntime, _region
    rt = ProjectionRuntime(0)
    rng = np.random.default_rng(5)
    ws = [rt.weight_from_region(fp8.pack_weight(*synth.weight(rng, INTER, HIDDEN))) for _ in range(2)]
    x = rt.context.upload(synth.activations(rng, 32, HIDDEN))
    h = rt.context.allocate(32 * INTER * 2)
    counts = rt.step_counts(32)
    op = rt.bind_gate_up("w8a16", counts, _region(x, alignment=256), ws[0], ws[1],
                         _region(h, alignment=256), 32)
    for _ in range(10):
        op.launch(rt.stream, synchronous=False)
    n = PMC_COPY_BYTES
    src, dst = rt.context.allocate(n), rt.context.allocate(n)
    cnt = rt.context.upload(np.array([n // 16], np.int64))
    copy = rt.function("lf_calibrate_copy")
    args = KernelArguments([_region(cnt, 8, alignment=8), _region(src, alignment=256),
                            _region(dst, alignment=256)])
    for _ in range(3):
        copy.launch_async(KernelLaunchDimensions.new((4096,), (256,)), args, rt.stream)
    rt.stream.synchronize()
    log(f"pmc pass done (gate_up x10, copy {n} bytes x3)")


# (M, K, N) of the dense GEMMs pmc_pass_prefill launches, in order.
# (operation, M, K, N): N is the packed QKV width, or I for gate/up (whose
# GEMM computes 2 I columns)
PREFILL_PASS_SHAPES = (("down", 8192, INTER, HIDDEN), ("o", 8192, HIDDEN, HIDDEN),
                       ("qkv", 8192, HIDDEN, NQ + 2 * NKV), ("gate_up", 8192, HIDDEN, INTER),
                       ("o", 3072, HIDDEN, HIDDEN), ("o", 2048, HIDDEN, HIDDEN),
                       ("qkv", 2048, HIDDEN, NQ + 2 * NKV), ("gate_up", 2048, HIDDEN, INTER))


def prefill_pass_flops(op, m, k, n):
    return 2 * m * k * (2 * n if op == "gate_up" else n)


def pmc_pass_prefill():
    """Short run for the MFMA-utilisation counter pass: the GEMM-only W8A8
    entries of all four Llama-3-8B operations at M = 8192 (256 x 256 tiles,
    four waves), o at M = 3072 (192 tiles of 256 x 256: the eight-wave form)
    and o, QKV and gate/up at M = 2048 (256 x 128 / eight-wave 256 x 256 /
    four-wave 256 x 256 tiles), 5 launches each after one act-quant."""
    from lunaflux_amd import fp8, synth
    from lunaflux_amd.fp8 import ProjectionRuntime, _region
    rt = ProjectionRuntime(0)
    rng = np.random.default_rng(6)
    for opname, m, k, n in PREFILL_PASS_SHAPES:
        x = rt.context.upload(synth.activations(rng, m, k))
        c = rt.step_counts(m, decode=False)
        xr = _region(x, alignment=256)
        if opname == "qkv":
            ws = [rt.weight_from_region(fp8.pack_weight(*synth.weight(rng, nn, k))) for nn in (NQ, NKV, NKV)]
            y = rt.context.allocate(m * n * 2)
            op = rt.bind_qkv("w8a8", c, xr, *ws, _region(y, alignment=256), m, one_launch=False)
        elif opname == "gate_up":
            ws = [rt.weight_from_region(fp8.pack_weight(*synth.weight(rng, n, k))) for _ in range(2)]
            y = rt.context.allocate(m * n * 2)
            op = rt.bind_gate_up("w8a8", c, xr, *ws, _region(y, alignment=256), m, one_launch=False)
        else:
            w = rt.weight_from_region(fp8.pack_weight(*synth.weight(rng, n, k)))
            y = rt.context.allocate(m * n * 2)
            op = rt.bind_dense("w8a8", c, xr, w, _region(y, alignment=256), m, one_launch=False)
        op.steps[0].launch(rt.stream, synchronous=False)
        for _ in range(5):
            op.steps[-1].launch(rt.stream, synchronous=False)
        rt.stream.synchronize()
        log(f"pmc prefill pass: {op.steps[-1].name} {opname} M={m} K={k} N={n} x5")


def pmc_pass_all():
    """Short run for counter passes over the kernels of config 2 and 4-5:
    the four decode calls at M = 32 and M = 128 (three launches each over two
    weight copies), one MoE operation of each MoE config (two launches of
    every step), then the calibration copy of 512 MiB three times."""
    from lunaflux_amd.device import KernelArguments, KernelLaunchDimensions
    from lunaflux_amd.fp8 import ProjectionRuntime, _region
    rt = ProjectionRuntime(0)
    layer = Layer(rt, rotations=2)
    for mt in (32, 128):
        b = Bench(rt, layer, mt, "w8a16")
        ops = b.bind(mt)
        for c, _, _, _ in call_shapes():
            for r in (0, 1, 0):
                ops[r][c].launch(rt.stream, synchronous=False)
        rt.stream.synchronize()
        log(f"pmc pass: decode M={mt} x3")
    for name, c in MOE_CONFIGS.items():
        moe_bench(rt, c, steps=2, warmup=0)
        log(f"pmc pass: moe {name} x2")
    n = PMC_COPY_BYTES
    src, dst = rt.context.allocate(n), rt.context.allocate(n)
    cnt = rt.context.upload(np.array([n // 16], np.int64))
    copy = rt.function("lf_calibrate_copy")
    args = KernelArguments([_region(cnt, 8, alignment=8), _region(src, alignment=256),
                            _region(dst, alignment=256)])
    for _ in range(3):
        copy.launch_async(KernelLaunchDimensions.new((4096,), (256,)), args, rt.stream)
    rt.stream.synchronize()
    log(f"pmc pass done (copy {n} bytes x3)")


def summarize_counters(paths):
    """Markdown table, one row per (kernel, grid), of rocprofv3 --pmc counter
    CSVs (any of the passes of --pmc-pass-all; kernel-trace CSVs add the
    duration): FETCH_SIZE and WRITE_SIZE scaled to bytes by what they read for
    lf_calibrate_copy moving a known number of bytes, and the MFMA busy
    fraction SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024
    SIMDs) with the clock GRBM_GUI_ACTIVE / 8 / duration."""
    import csv
    vals, dur = {}, {}
    for path in paths:
        rows = list(csv.DictReader(open(path)))
        # Decode kernels are launched three times back to back per call, and
        # at 128 rows o and down run one kernel on one grid: their rows are
        # told apart by the run of consecutive dispatches they belong to
        # (run 2 = the second call of that kernel and grid). MoE kernels
        # recur in every step of an operation and are pooled.
        run_of, last, runs = {}, None, {}
        order = sorted({int(r.get("Dispatch_Id") or 0) for r in rows})
        first = {}
        for r in rows:
            first.setdefault(int(r.get("Dispatch_Id") or 0), r)
        for d in order:
            r = first[d]
            blocks = int(r.get("Grid_Size_X") or r.get("Grid_Size") or 0) // max(
                int(r.get("Workgroup_Size_X") or r.get("Workgroup_Size") or 1), 1)
            k = (r["Kernel_Name"], blocks)
            if k != last:
                runs[k] = runs.get(k, 0) + 1
            last = k
            run_of[d] = runs[k] if r["Kernel_Name"].startswith("lf_fp8_w8a16") else 1
        for r in rows:
            blocks = int(r.get("Grid_Size_X") or r.get("Grid_Size") or 0) // max(
                int(r.get("Workgroup_Size_X") or r.get("Workgroup_Size") or 1), 1)
            run = run_of[int(r.get("Dispatch_Id") or 0)]
            key = (r["Kernel_Name"], blocks if run == 1 else f"{blocks} (call {run})")
            if "Counter_Name" in r:
                vals.setdefault(key, {}).setdefault(r["Counter_Name"], []).append(
                    float(r["Counter_Value"]))
            elif "Start_Timestamp" in r:
                dur.setdefault(key, []).append(
                    (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)

    def mean(key, counter):
        v = vals.get(key, {}).get(counter)
        return float(np.mean(v)) if v else None

    cal = [k for k in vals if k[0] == "lf_calibrate_copy"]
    f_factor = w_factor = None
    if cal:
        f_cal, w_cal = mean(cal[0], "FETCH_SIZE"), mean(cal[0], "WRITE_SIZE")
        f_factor = PMC_COPY_BYTES / (f_cal * 1024) if f_cal else None
        w_factor = PMC_COPY_BYTES / (w_cal * 1024) if w_cal else None
    out = [f"Calibration (lf_calibrate_copy, {PMC_COPY_BYTES} B read and written): FETCH_SIZE "
           f"factor {f_factor and round(f_factor, 4)}, WRITE_SIZE factor {w_factor and round(w_factor, 4)}",
           "",
           "| Kernel | Blocks | Duration us | HBM read MB | HBM write MB | MFMA busy | Clock GHz |",
           "|---|---|---|---|---|---|---|"]
    for key in sorted(set(vals) | set(dur), key=lambda kk: (kk[0], str(kk[1]))):
        if key[0] == "lf_calibrate_copy":
            continue
        f, w = mean(key, "FETCH_SIZE"), mean(key, "WRITE_SIZE")
        busy, gui = mean(key, "SQ_VALU_MFMA_BUSY_CYCLES"), mean(key, "GRBM_GUI_ACTIVE")
        d = float(np.mean(dur[key])) if key in dur else None
        read_mb = f"{f * 1024 * f_factor / 1e6:.1f}" if f is not None and f_factor else "-"
        write_mb = f"{w * 1024 * w_factor / 1e6:.1f}" if w is not None and w_factor else "-"
        frac = f"{busy / (gui / 8 * 1024) * 100:.0f} %" if busy is not None and gui else "-"
        clock = f"{gui / 8 / (d * 1e-6) / 1e9:.2f}" if gui and d else "-"
        out.append(f"| {key[0]} | {key[1]} | {d and round(d, 1) or '-'} | {read_mb} | {write_mb} | "
                   f"{frac} | {clock} |")
    return "\n".join(out)


def measured_traffic(kernel):
    """HBM bytes per launch of the roofline kernel from its committed counter
    summary (profiles/<kernel>.traffic.json, written by --summarize-traffic),
    or None when there is none for this kernel."""
    path = os.path.join(ROOT, "profiles", f"{kernel}.traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    return data.get("bytes_per_launch") if data.get("kernel") == kernel else None


def summarize_traffic(fetch_csv, write_csv, kernel):
    """Counter summary of one kernel's HBM traffic from two rocprofv3 --pmc
    runs of --pmc-pass (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each
    scaled by what the same counter reads for lf_calibrate_copy moving a
    known number of bytes. Prints the JSON stored under profiles/."""
    import csv

    def per_dispatch(path, counter):
        vals = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter:
                vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return vals

    fetch, write = per_dispatch(fetch_csv, "FETCH_SIZE"), per_dispatch(write_csv, "WRITE_SIZE")
    copy_bytes = PMC_COPY_BYTES
    f_cal = np.mean(fetch["lf_calibrate_copy"])
    w_cal = np.mean(write["lf_calibrate_copy"])
    f_factor = copy_bytes / (f_cal * 1024)
    w_factor = copy_bytes / (w_cal * 1024)
    f_k = np.mean(fetch[kernel])
    w_k = np.mean(write[kernel])
    read_b = int(round(f_k * 1024 * f_factor))
    write_b = int(round(w_k * 1024 * w_factor))
    algo = call_bytes(32, HIDDEN, 2 * INTER, INTER)
    return {
        "kernel": kernel,
        "workload": "Llama-3-8B gate/up (4096 -> 2 x 14336, SwiGLU), M=32, one launch",
        "commands": [
            "cd /tmp && export TMPDIR=/tmp && timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE "
            "--output-format csv -d $GRAFT_REPO_ROOT/gpurun_out/prof_fetch -o fetch -- python3 "
            "$GRAFT_REPO_ROOT/bench.py --pmc-pass",
            "cd /tmp && export TMPDIR=/tmp && timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE "
            "--output-format csv -d $GRAFT_REPO_ROOT/gpurun_out/prof_write -o write -- python3 "
            "$GRAFT_REPO_ROOT/bench.py --pmc-pass",
            "python3 bench.py --summarize-traffic <fetch_counter_collection.csv> "
            "<write_counter_collection.csv>",
        ],
        "fetch_size_kib_per_dispatch": round(f_k, 2),
        "fetch_dispatches": len(fetch[kernel]),
        "write_size_kib_per_dispatch": round(w_k, 2),
        "write_dispatches": len(write[kernel]),
        "calibration": {"kernel": "lf_calibrate_copy", "bytes_read": copy_bytes,
                        "bytes_written": copy_bytes, "fetch_size_kib": round(f_cal, 2),
                        "write_size_kib": round(w_cal, 2), "fetch_factor": round(f_factor, 5),
                        "write_factor": round(w_factor, 5)},
        "read_bytes_per_launch": read_b,
        "write_bytes_per_launch": write_b,
        "bytes_per_launch": read_b + write_b,
        "algorithmic_bytes_per_launch": algo,
        "traffic_over_algorithmic": round((read_b + write_b) / algo, 4),
    }


def summarize_mfma(counter_csv, trace_csv):
    """Markdown table of the --pmc-pass-prefill MFMA counter pass (counter CSV
    of SQ_VALU_MFMA_BUSY_CYCLES, SQ_INSTS_VALU_MFMA_MOPS_F8, SQ_INSTS_VALU_MFMA_F8,
    SQ_INSTS_VALU_MFMA_F6F4, GRBM_GUI_ACTIVE) with durations from a kernel
    trace of the same pass: per shape the mean over its 5 GEMM launches. MFMA
    busy = busy cycles / (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs); clock =
    GRBM_GUI_ACTIVE / 8 / duration."""
    import csv
    gemm = lambda name: name.startswith("lf_fp8_w8a8_") and not name.endswith("_aq")
    disp = {}
    for r in csv.DictReader(open(counter_csv)):
        if gemm(r["Kernel_Name"]):
            d = disp.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"], "wg": int(r["Workgroup_Size"])})
            d[r["Counter_Name"]] = float(r["Counter_Value"])
    ids = sorted(disp)
    trace = [r for r in csv.DictReader(open(trace_csv)) if gemm(r["Kernel_Name"])]
    shapes = PREFILL_PASS_SHAPES
    if len(ids) != 5 * len(shapes) or len(trace) != 5 * len(shapes):
        raise SystemExit(f"expected {5 * len(shapes)} GEMM dispatches, got {len(ids)} / {len(trace)}")
    lines = ["| Kernel | Shape | Threads | MFMA instructions | MFMA flops (MOPS_F8 x 512) | MFMA busy cycles "
             "| GRBM_GUI_ACTIVE | Duration (trace) | Clock | MFMA busy | Achieved |",
             "|---|---|---|---|---|---|---|---|---|---|---|"]
    for s, (opname, m, k, n) in enumerate(shapes):
        ds = [disp[i] for i in ids[5 * s:5 * s + 5]]
        ts = trace[5 * s:5 * s + 5]
        name = ds[0]["name"]
        if any(d["name"] != name for d in ds) or any(t["Kernel_Name"] != name for t in ts):
            raise SystemExit(f"dispatch order does not match the pass at shape {s}")
        mean = lambda c: sum(d[c] for d in ds) / len(ds)
        dur = sum(int(t["End_Timestamp"]) - int(t["Start_Timestamp"]) for t in ts) / len(ts) / 1e3
        ins = mean("SQ_INSTS_VALU_MFMA_F8") + mean("SQ_INSTS_VALU_MFMA_F6F4")
        mops = mean("SQ_INSTS_VALU_MFMA_MOPS_F8") * 512
        busy, gui = mean("SQ_VALU_MFMA_BUSY_CYCLES"), mean("GRBM_GUI_ACTIVE")
        flops = prefill_pass_flops(opname, m, k, n)
        shape = f"N={n}" if opname != "gate_up" else f"N=2x{n}"
        lines.append(f"| {name} | {opname}, M={m}, K={k}, {shape} | {ds[0]['wg']} | {ins:.0f} | {mops:.4g} "
                     f"(= 2MNK {flops:.4g}) | {busy:.4g} | {gui:.4g} | {dur:.1f} us | "
                     f"{gui / 8 / (dur * 1e-6) / 1e9:.2f} GHz | {100 * busy / (gui / 8 * 1024):.0f} % | "
                     f"{flops / dur / 1e6:.0f} TFLOP/s |")
    return "\n".join(lines)


def summarize_trace(trace_csv, gap=32):
    """Markdown table of a rocprofv3 kernel-trace CSV: one row per (kernel,
    blocks, threads) with launches and average / min / max duration in us,
    plus the average of each segment (dispatches of that key with at most
    `gap` other dispatches between consecutive ones), which separates the
    shapes the bench times one after another under the same kernel and grid."""
    import csv
    rows = list(csv.DictReader(open(trace_csv)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    groups, last_seen = {}, {}
    for i, r in enumerate(rows):
        threads = int(r["Workgroup_Size_X"])
        key = (r["Kernel_Name"], int(r["Grid_Size_X"]) // threads, threads)
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        segs = groups.setdefault(key, [])
        if not segs or i - last_seen[key] > gap + 1:
            segs.append([])
        segs[-1].append(us)
        last_seen[key] = i
    out = ["| Kernel | Blocks | Threads | Launches | Average us | Min us | Max us | Segment averages us |",
           "|---|---|---|---|---|---|---|---|"]
    for key in sorted(groups):
        segs = groups[key]
        allv = [v for seg in segs for v in seg]
        seg_avg = ", ".join(f"{sum(seg) / len(seg):.1f} ({len(seg)})" for seg in segs)
        out.append(f"| {key[0]} | {key[1]} | {key[2]} | {len(allv)} | {sum(allv) / len(allv):.2f} | "
                   f"{min(allv):.2f} | {max(allv):.2f} | {seg_avg} |")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only, no detail sweep")
    ap.add_argument("--pmc-pass", action="store_true", help="short run for counter passes")
    ap.add_argument("--pmc-pass-prefill", action="store_true",
                    help="short run for the prefill MFMA counter pass")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the traffic summary of the roofline kernel from the two "
                         "--pmc-pass counter CSVs (no GPU needed)")
    ap.add_argument("--pmc-pass-all", action="store_true",
                    help="short run of the decode and MoE kernels for counter passes")
    ap.add_argument("--summarize-counters", nargs="+", metavar="CSV",
                    help="per-kernel markdown table of --pmc-pass-all counter (and kernel-trace) "
                         "CSVs (no GPU needed)")
    ap.add_argument("--summarize-mfma", nargs=2, metavar=("COUNTER_CSV", "KERNEL_TRACE_CSV"),
                    help="markdown table of the --pmc-pass-prefill MFMA counter pass (no GPU needed)")
    ap.add_argument("--summarize-trace", metavar="KERNEL_TRACE_CSV",
                    help="print a per-kernel markdown summary of a rocprofv3 kernel-trace CSV "
                         "(no GPU needed)")
    args = ap.parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace))
        return
    if args.summarize_mfma:
        print(summarize_mfma(*args.summarize_mfma))
        return
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters))
        return
    if args.summarize_traffic:
        print(json.dumps(summarize_traffic(*args.summarize_traffic, roofline_kernel()), indent=1))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path; one GPU runs each kernel at a shard's shape)", file=sys.stderr)
        sys.exit(2)
    if args.pmc_pass:
        pmc_pass()
        return
    if args.pmc_pass_prefill:
        pmc_pass_prefill()
        return
    if args.pmc_pass_all:
        pmc_pass_all()
        return

    from lunaflux_amd.fp8 import ProjectionRuntime
    from lunaflux_amd import device

    cap = device.device_info(0)
    log(f"device: {cap.name} gfx{cap.major}{cap.minor}{0} mem={cap.total_memory / 2**30:.0f} GiB")
    rt = ProjectionRuntime(0)
    layer = Layer(rt)

    m = 32
    decode = Bench(rt, layer, 32, "w8a16")
    total, _, step_ms = decode.run(m, args.steps, args.warmup, probe=None)
    value = layer_bytes(m) / (step_ms * 1e-3) / 1e9
    gu_bytes = call_bytes(m, HIDDEN, 2 * INTER, INTER)
    kernel = decode.ops[m][1][0]["gate_up"].steps[-1].name
    assert kernel == roofline_kernel(), kernel
    probe_ms = decode.time_kernel(m, "gate_up", args.steps)
    achieved = gu_bytes / (probe_ms * 1e-3) / 1e9
    log(f"decode M={m}: {step_ms * 1e3:.1f} us/layer, {value:.0f} GB/s; gate_up {probe_ms * 1e3:.1f} us "
        f"= {achieved:.0f} GB/s")

    detail = {"decode_w8a16": {}, "prefill_w8a8": {}}
    if not args.quick:
        mlp_bytes = lambda mm: (call_bytes(mm, HIDDEN, 2 * INTER, INTER) +
                                call_bytes(mm, INTER, HIDDEN, HIDDEN) - 4 * mm * INTER)
        for mm, mt in [(1, 16), (8, 16), (32, 32), (128, 128)]:
            b = Bench(rt, layer, mt, "w8a16") if mt != 32 else decode
            # Untimed layer steps first, three weight rotations: at 128 rows
            # (the first MFMA-heavy row) successive 25-step passes of a newly
            # bound layer read 116.6, 110.2, 104.9, 103.4, 101.8 us and then
            # settle at 98-101 us, so a short warm-up times the chip's
            # ramp, not the kernels
            b.run(mm, 3 * ROTATIONS, 0, probe=None)
            row = {}
            for c, k, n, no in call_shapes():
                p = b.time_kernel(mm, c, 20)
                row[c] = {"us": round(p * 1e3, 2), "GB/s": round(call_bytes(mm, k, n, no) / (p * 1e-3) / 1e9, 1)}
            t, _, s_ms = b.run(mm, 20, 5, probe=None)
            row["layer_us"] = round(s_ms * 1e3, 2)
            row["layer_GB/s"] = round(layer_bytes(mm) / (s_ms * 1e-3) / 1e9, 1)
            row["layer_hbm_frac"] = round(row["layer_GB/s"] / HBM_PEAK_GBS, 4)
            # GatedMlp as the plan binds it (one launch where an entry is
            # built) against its two launches; bytes without h's round trip
            one = b.bind_mlp(mm, True)
            two = b.bind_mlp(mm, False)
            t1, t2 = b.time_ops(one, 20), b.time_ops(two, 20)
            row["gated_mlp"] = {"launches": len(one[0].steps), "us": round(t1 * 1e3, 2),
                                "GB/s": round(mlp_bytes(mm) / (t1 * 1e-3) / 1e9, 1),
                                "two_launch_us": round(t2 * 1e3, 2)}
            # the drop-in layer: qkv, o and the GatedMlp operation, one launch each
            row["layer_one_launch_us"] = round((row["qkv"]["us"] + row["o"]["us"]) + t1 * 1e3, 2)
            detail["decode_w8a16"][f"M={mm}"] = row
            log(f"decode M={mm}: {row}")
        detail["lm_head_w8a16"] = lm_head_bench(rt)
        log(f"lm head: {detail['lm_head_w8a16']}")
        for mm in (2048, 8192):
            b = Bench(rt, layer, mm, "w8a8", one_launch=False)
            b1 = Bench(rt, layer, mm, "w8a8", one_launch=True, share=b)
            row = {}
            for c, k, n, no in call_shapes():
                p = b.time_kernel(mm, c, 5, warmup=2)
                q = b.time_kernel(mm, c, 5, warmup=2, step=0)
                p1 = b1.time_kernel(mm, c, 5, warmup=2)
                tf = call_flops(mm, k, n) / (p * 1e-3) / 1e12
                op_tf = call_flops(mm, k, n) / ((p + q) * 1e-3) / 1e12
                one_tf = call_flops(mm, k, n) / (p1 * 1e-3) / 1e12
                row[c] = {"gemm_us": round(p * 1e3, 1), "TFLOP/s": round(tf, 1),
                          "fp8_frac": round(tf / FP8_PEAK_TFLOPS, 4),
                          "act_quant_us": round(q * 1e3, 1),
                          "act_quant_GB/s": round(mm * k * 3 / (q * 1e-3) / 1e9, 1),
                          "op_us": round((p + q) * 1e3, 1), "op_TFLOP/s": round(op_tf, 1),
                          "op_fp8_frac": round(op_tf / FP8_PEAK_TFLOPS, 4),
                          # the plan's binding: one launch, act-quant inside
                          "one_launch_us": round(p1 * 1e3, 1), "one_launch_TFLOP/s": round(one_tf, 1),
                          "one_launch_fp8_frac": round(one_tf / FP8_PEAK_TFLOPS, 4)}
            mlp_flops = call_flops(mm, HIDDEN, 2 * INTER) + call_flops(mm, INTER, HIDDEN)
            t1, t4 = b1.time_ops(b1.bind_mlp(mm, True), 5), b.time_ops(b.bind_mlp(mm, False), 5)
            row["gated_mlp"] = {"launches": 1, "us": round(t1 * 1e3, 1),
                                "TFLOP/s": round(mlp_flops / (t1 * 1e-3) / 1e12, 1),
                                "fp8_frac": round(mlp_flops / (t1 * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
                                "four_launch_us": round(t4 * 1e3, 1)}
            row["rms_norm_quant_k4096"] = rms_norm_quant_bench(rt, b, mm)
            detail["prefill_w8a8"][f"M={mm}"] = row
            log(f"prefill M={mm}: {row}")
            del b, b1
        detail["block_scaled"] = block_scaled_bench(rt)
        detail["moe"] = {}
        for name, c in MOE_CONFIGS.items():
            detail["moe"][name] = moe_bench(rt, c)
            log(f"moe {name}: {detail['moe'][name]}")

    cpu = None
    if not args.no_cpu:
        log("timing the CPU oracle baseline ...")
        cpu = cpu_baseline(32)
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 weights x bf16 activations, fp32 accumulate (W8A16)",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantized to e4m3)",
        "config": {"workload": "llama3-8b decode layer: qkv+o+gate_up(SwiGLU)+down, M=32, W8A16",
                   "global_batch": m, "seq_len": 1, "parallelism": "single GPU",
                   "weight_rotations": ROTATIONS},
        "roofline": {"bound": "hbm", "kernel": kernel,
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(kernel),
                     "algorithmic_bytes_per_launch": gu_bytes,
                     "avg_launch_us": round(probe_ms * 1e3, 2)},
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

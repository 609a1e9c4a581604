"""GPU parity of the MoE expert MLP at BASELINE configs 4 and 5's own shapes.

Config 4 (Mixtral): 8 experts, top-2 (softmax over the two picked logits),
hidden 4096, intermediate 14336, 1024 tokens, router logits N(0, 1) plus a
per-expert bias N(0, 1.5), e4m3 weights with per-channel scales. Config 5:
64 experts, top-6 (softmax over all experts), hidden 2048, intermediate
1408, 128 x 128 block scales with per-token-per-128-group activations,
Zipf(1.1) expert popularity, at 4096 and 32 tokens. These run the kernels the
benchmark times at those shapes (the 256 x 256 grouped GEMMs, the K = 14336
down loop, the grouped GEMV form at 32 tokens).

At full size the oracle cannot recompute every GEMM in seconds, so:
* bit-exact at full size: routing ids, the stable sort, inverse positions,
  expert row / tile offsets and the list of experts with rows, the token
  quantizer and the hidden quantizer (on the GPU's h);
* each GEMM stage on its actual inputs, on a row sample holding the first
  and last row of every expert and of every 128- and 256-row tile (so every
  expert with rows and every partial last tile is covered) plus random rows,
  and a column sample holding the edges of every 64-, 128- and 256-column
  block plus random columns: gate/up + SwiGLU from the GPU's quantized
  tokens, down from the GPU's quantized h, at the BASELINE bar;
* the combine at full size from the GPU's y and routing weights;
* end to end from the original inputs for 64 sampled tokens (all 32 at
  T = 32): the oracle's own h codes against the GPU's, every difference a
  move across an e4m3 rounding boundary (the two bf16 h values within one
  ulp); the output at the BASELINE bar against the oracle's down and
  combine (y rounded to bf16, as the device stores it) over the GPU's
  codes; and at the documented looser bound against lfo_moe_mlp with its
  own codes.
"""
import numpy as np
import pytest

import oracle_lib as o
from lunaflux_amd import synth
from parity import (abs_sum, combine, combine_tol, moved_codes_explained, parity,
                    swiglu_midpoint_tol)
from test_gpu_moe import check_routing

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from lunaflux_amd.fp8 import ProjectionRuntime
    return ProjectionRuntime(0)


def expert_stack(rng, experts, rows, cols, block):
    """E distinct expert weights: one N(0, 0.02) [rows, cols] draw quantized
    by the oracle's quantizer, then permuted per expert (rows, or 128-row
    blocks with block scales). Each expert's codes and scales are exactly the
    quantization of its own permuted matrix, and E full-size draws (1.4 G
    values for Mixtral) are not needed."""
    w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
    if block:
        q, s = o.quantize_blocks(w, 128)
        qb = q.reshape(rows // 128, 128, cols)
        perms = [rng.permutation(rows // 128) for _ in range(experts)]
        return (np.stack([qb[p].reshape(rows, cols) for p in perms]),
                np.stack([s[p] for p in perms]))
    q, s = o.quantize_rows(w)
    perms = [rng.permutation(rows) for _ in range(experts)]
    return np.stack([q[p] for p in perms]), np.stack([s[p] for p in perms])


def dequant_rows(q, s, rows, block):
    """fp32(code) * scale of rows `rows` of one expert weight (the oracle's
    dequantization, applied to just those rows)."""
    if not block:
        return o.dequantize(q[rows], s[rows])
    out = np.empty((len(rows), q.shape[1]), np.float32)
    for i, r in enumerate(rows):
        out[i] = o.dequantize(q[r:r + 1], s[r // 128:r // 128 + 1], mode=2, group=128)[0]
    return out


def dequant_expert(q, s, block):
    return o.dequantize(q, s, mode=2 if block else 0, group=128 if block else 0)


def sample_positions(offsets, rng, extra=48):
    """Positions (rows in expert order): first and last of every expert and
    of every 128- and 256-row tile (tiles start at each expert's first row),
    plus random ones."""
    picks = []
    for e in range(len(offsets) - 1):
        a, b = int(offsets[e]), int(offsets[e + 1])
        for tile in (128, 256):
            for start in range(a, b, tile):
                picks += [start, min(start + tile, b) - 1]
    total = int(offsets[-1])
    picks += list(rng.choice(total, min(extra, total), replace=False))
    return np.unique(np.asarray(picks, np.int64))


def sample_columns(n, rng, extra=160):
    picks = [0, n - 1]
    for block in (64, 128, 256):
        for start in range(0, n, block):
            if rng.random() < 0.15:
                picks += [start, min(start + block, n) - 1]
    picks += list(rng.choice(n, min(extra, n), replace=False))
    return np.unique(np.asarray(picks, np.int64))


def run_full(rt, rng, t, e, k, hidden, inter, route_mode, block, logits):
    from lunaflux_amd import fp8, moe
    x = synth.activations(rng, t, hidden)
    weights = (expert_stack(rng, e, inter, hidden, block) + expert_stack(rng, e, inter, hidden, block)
               + expert_stack(rng, e, hidden, inter, block))
    mode = fp8.BLOCK128 if block else fp8.PER_CHANNEL
    wg, wu, wd = (rt.upload_weight(weights[i], weights[i + 1], mode) for i in (0, 2, 4))
    out, st = moe.moe_expert_mlp(rt, x, logits, wg, wu, wd, k, route_mode, 128 if block else 0,
                                 max_tokens=t, return_workspace=True)
    return x, weights, out, st


def check_full(x, weights, out, st, logits, k, route_mode, block, rng, label, e2e_tokens=64):
    qg, sg, qu, su, qd, sd = weights
    e = logits.shape[1]
    grp, dmode = (128, 1) if block else (None, 0)
    ex, w = check_routing(logits, k, route_mode, st)
    # token and hidden quantizers: bit-exact over every row
    xq, xs = o.quantize_rows(o.bf16_decode(x), group=grp)
    np.testing.assert_array_equal(st["xq"], xq)
    np.testing.assert_array_equal(st["xs"].reshape(xs.shape[0], -1), xs.reshape(xs.shape[0], -1))
    hq, hs = o.quantize_rows(o.bf16_decode(st["h"]), group=grp)
    np.testing.assert_array_equal(st["hq"], hq)
    np.testing.assert_array_equal(st["hs"].reshape(hs.shape[0], -1), hs.reshape(hs.shape[0], -1))
    xr = o.dequantize(xq, xs, mode=dmode, group=grp or 0)
    sorted_a = st["sorted"]
    experts = ex.reshape(-1)[sorted_a]
    tokens = sorted_a // k
    offsets = st["offsets"]
    pos = sample_positions(offsets, rng)
    ch = sample_columns(qg.shape[1], rng)
    cy = sample_columns(qd.shape[1], rng)
    inter, hidden = qg.shape[1], qd.shape[1]
    h_ref = np.zeros((len(pos), len(ch)), np.float32)
    h_tol = np.zeros_like(h_ref)
    y_ref = np.zeros((len(pos), len(cy)), np.float32)
    y_abs = np.zeros_like(y_ref)
    hr = o.dequantize(hq[pos], hs[pos], mode=dmode, group=grp or 0)
    for ee in np.unique(experts[pos]):
        i = np.flatnonzero(experts[pos] == ee)
        xe = xr[tokens[pos[i]]]
        wgr = dequant_rows(qg[ee], sg[ee], ch, block)
        wur = dequant_rows(qu[ee], su[ee], ch, block)
        g = o.dense_projection(xe, wgr)
        u = o.dense_projection(xe, wur)
        h_ref[i] = o.silu_mul_array(g, u)
        h_tol[i] = swiglu_midpoint_tol(g, u, abs_sum(xe, wgr), abs_sum(xe, wur), hidden)
        wdr = dequant_rows(qd[ee], sd[ee], cy, block)
        y_ref[i] = o.dense_projection(hr[i], wdr)
        y_abs[i] = abs_sum(hr[i], wdr)
    print(f"{label}: {len(pos)} sampled rows over {len(np.unique(experts[pos]))} experts, "
          f"{len(ch)} h columns, {len(cy)} y columns", flush=True)
    parity(st["h"][pos][:, ch], h_ref, label=label + " gate_up", midpoint_tol=h_tol)
    parity(o.bf16_round(st["y"][pos][:, cy]), y_ref, k=inter, s_abs=y_abs, label=label + " down")
    # combine at full size, from the GPU's y and routing weights
    comb = np.zeros(out.shape, np.float32)
    for j in range(k):
        comb = (comb + (st["topk_w"][:, j:j + 1]
                        * st["y"][st["pos"].reshape(-1, k)[:, j]]).astype(np.float32)).astype(np.float32)
    # the combine's arithmetic is defined exactly (products and sums each
    # rounded, ascending j, from 0): bit-identical on the GPU's own y
    np.testing.assert_array_equal(out, o.bf16_round(comb))
    # End to end from the original inputs, for e2e_tokens sampled tokens
    # (the lightest experts' tokens first, then random ones). h is
    # re-quantized to e4m3 between the GEMMs, and one bf16 ulp of h can move
    # an e4m3 code across its rounding boundary, so: (a) the oracle's own h
    # codes (its sequential fp32 gate/up, SiLU, bf16 rounding and quantizer:
    # lfo_moe_mlp's arithmetic) are formed for every sampled assignment, and
    # every code that differs from the GPU's must be such a move; (b) the
    # output must meet the BASELINE bar against the oracle's down and combine
    # (y rounded to bf16, as the device stores it) over the GPU's codes,
    # which are the oracle's except the moved ones; (c) the pure oracle (its
    # own codes, lfo_moe_mlp) at the looser bound.
    counts = np.diff(offsets)
    light = [int(tokens[offsets[ee]]) for ee in np.argsort(counts) if counts[ee] > 0][:2]
    n_tok = min(e2e_tokens, ex.shape[0])
    toks = np.unique(np.concatenate([light, rng.choice(ex.shape[0], n_tok - len(light), replace=False)]))
    used = np.unique(ex[toks])
    remap = np.full(e, -1, np.int32)
    remap[used] = np.arange(len(used))
    wgf = np.stack([dequant_expert(qg[u_], sg[u_], block) for u_ in used])
    wuf = np.stack([dequant_expert(qu[u_], su[u_], block) for u_ in used])
    wdf = np.stack([dequant_expert(qd[u_], sd[u_], block) for u_ in used])
    pos_of = st["pos"].reshape(-1, k)
    y_gpu_codes = np.zeros((len(toks), k, hidden), np.float32)
    y_abs = np.zeros((len(toks), k, hidden), np.float64)
    moved = codes = 0
    for ui, ue in enumerate(used):
        sel = np.argwhere(ex[toks] == ue)          # (index in toks, pick j)
        xe = xr[toks[sel[:, 0]]]
        g = o.project_values_mt(xe, wgf[ui], 16)
        u = o.project_values_mt(xe, wuf[ui], 16)
        h_o = o.silu_mul_array(g, u)
        h_tol = swiglu_midpoint_tol(g, u, abs_sum(xe, wgf[ui]), abs_sum(xe, wuf[ui]), hidden)
        hq_o, hs_o = o.quantize_rows(o.bf16_decode(o.bf16_round(h_o)), group=grp)
        p = pos_of[toks[sel[:, 0]], sel[:, 1]]
        moved += moved_codes_explained(h_o, st["h"][p], h_tol, hq_o, st["hq"][p], hs_o, st["hs"][p],
                                       f"{label} expert {ue}")
        codes += hq_o.size
        hr_g = o.dequantize(st["hq"][p], st["hs"][p], mode=dmode, group=grp or 0)
        y_gpu_codes[sel[:, 0], sel[:, 1]] = o.project_values_mt(hr_g, wdf[ui], 16)
        y_abs[sel[:, 0], sel[:, 1]] = abs_sum(hr_g, wdf[ui])
    print(f"{label} end-to-end: {len(toks)} tokens; {moved} of {codes} h codes moved across a "
          f"rounding boundary", flush=True)
    # (routing weights: the GPU's, which check_routing holds within 2e-6 of
    # the oracle's softmax; a one-ulp weight can flip an output rounding)
    wg_ = st["topk_w"][toks]
    parity(out[toks], combine(wg_, y_gpu_codes), label=label + " end-to-end (GPU h codes)",
           value_tol=combine_tol(wg_, y_gpu_codes, y_abs, inter))
    ref = o.moe_mlp(xr[toks], wgf, wuf, wdf, remap[ex[toks]], w[toks],
                    hidden_transform=(5 if block else 3) | 8, threads=16)
    parity(out[toks], ref, rel_l2=1e-2, max_abs=0.25, label=label + " end-to-end (oracle h codes)")
    return ex


def test_moe_config4_mixtral_full_shape(rt):
    from lunaflux_amd import _abi, moe
    t, e, k, hidden, inter = 1024, 8, 2, 4096, 14336
    desc = moe.moe_descriptor(e, k, 0, hidden, inter, 0)
    assert moe.launch_geometry(_abi.MOE_GATE_UP, desc, t)[1] == "lf_moe_gate_up_t256"
    assert moe.launch_geometry(_abi.MOE_DOWN, desc, t)[1] == "lf_moe_down_t256_aq"
    assert moe.launch_geometry(_abi.MOE_QUANT_HIDDEN, desc, t)[1] == ""
    rng = np.random.default_rng(40)
    logits = (rng.standard_normal((t, e)) + rng.normal(0, 1.5, e)).astype(np.float32)
    x, weights, out, st = run_full(rt, rng, t, e, k, hidden, inter, 0, False, logits)
    ex = check_full(x, weights, out, st, logits, k, 0, False, rng, "moe config4 mixtral")
    assert st["offsets"][-1] == t * k


def zipf_logits(rng, t, e):
    """Router logits N(0, 1) plus a Zipf(1.1) log-popularity by expert rank
    (the benchmark's config 5 input)."""
    logits = rng.standard_normal((t, e)).astype(np.float32)
    return logits + np.log(1.0 / np.arange(1, e + 1) ** 1.1).astype(np.float32)[rng.permutation(e)]


@pytest.mark.parametrize("t,gemm", [(4096, "t256_b128"), (32, "gemv")])
def test_moe_config5_fine_grained_full_shape(rt, t, gemm):
    from lunaflux_amd import _abi, moe
    e, k, hidden, inter = 64, 6, 2048, 1408
    desc = moe.moe_descriptor(e, k, 1, hidden, inter, 128)
    # (t256 with block scales: the gate/up epilogue quantizes h)
    fused = "_q" if gemm == "t256_b128" else ""
    assert moe.launch_geometry(_abi.MOE_GATE_UP, desc, t)[1] == f"lf_moe_gate_up_{gemm}{fused}"
    assert moe.launch_geometry(_abi.MOE_DOWN, desc, t)[1] == f"lf_moe_down_{gemm}"
    rng = np.random.default_rng(50 + t)
    logits = zipf_logits(rng, t, e)
    x, weights, out, st = run_full(rt, rng, t, e, k, hidden, inter, 1, True, logits)
    check_full(x, weights, out, st, logits, k, 1, True, rng, f"moe config5 t={t}")
    assert st["offsets"][-1] == t * k

"""Host side of the grouped (MoE expert MLP) form of the FP8 path.

The reference has no MoE operation; this module binds the launch sequence
documented in include/lunaflux_fp8.h (route -> stable sort -> token
quantization -> grouped gate/up + SwiGLU -> hidden quantization -> grouped
down -> top-k combine) to device regions, and offers a numpy-level call,
`moe_expert_mlp`, for tests and tools.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _abi
from .device import DeviceError, KernelArgument, KernelArguments, KernelLaunchDimensions
from .fp8 import COUNTS_BYTES, BoundOperation, Fp8Weight, LaunchStep, ProjectionRuntime, _region

ROUTE_TOPK_SOFTMAX = 0   # Mixtral: softmax over the k picked logits
ROUTE_SOFTMAX_TOPK = 1   # softmax over all experts, keep the k picked


class MoeDescriptor(ctypes.Structure):
    _fields_ = [("magic", ctypes.c_uint32), ("experts", ctypes.c_int32), ("top_k", ctypes.c_int32),
                ("route_mode", ctypes.c_int32), ("hidden", ctypes.c_int32), ("inter", ctypes.c_int32),
                ("group", ctypes.c_int32), ("reserved", ctypes.c_int32)]

    def as_bytes(self) -> np.ndarray:
        return np.frombuffer(bytes(self), np.uint8).copy()


def _check(operation, status):
    if status != _abi.LF_OK:
        raise DeviceError(operation, status)


def moe_descriptor(experts: int, top_k: int, route_mode: int, hidden: int, inter: int,
                   group: int = 0) -> MoeDescriptor:
    d = MoeDescriptor()
    _check("moe_descriptor", _abi.lib().lunaflux_fp8_moe_descriptor(
        experts, top_k, route_mode, hidden, inter, group, ctypes.byref(d)))
    return d


def workspace_bytes(desc: MoeDescriptor, max_tokens: int) -> int:
    n = _abi.lib().lunaflux_fp8_moe_workspace_bytes(ctypes.byref(desc), max_tokens)
    if n < 0:
        raise DeviceError("moe_workspace_bytes", _abi.LF_INVALID_ARGUMENT)
    return n


def sync_offset(desc: MoeDescriptor, max_tokens: int):
    """Offset of the down launch's counter area in the workspace, or None
    where the profile's down entry takes none (lunaflux_fp8_moe_sync_offset).
    Its first int32 is the error word of the counted waits."""
    n = _abi.lib().lunaflux_fp8_moe_sync_offset(ctypes.byref(desc), max_tokens)
    return None if n < 0 else n


LAYOUT_FIELDS = ("topk_ids", "topk_w", "sorted", "pos", "offsets", "tiles", "xq", "xs", "h", "hq",
                 "hs", "y", "end")


def workspace_layout(desc: MoeDescriptor, tokens: int) -> dict:
    out = (ctypes.c_int64 * 13)()
    _check("moe_workspace_layout", _abi.lib().lunaflux_fp8_moe_workspace_layout(
        ctypes.byref(desc), tokens, out))
    return dict(zip(LAYOUT_FIELDS, (int(v) for v in out)))


def launch_geometry(entry: int, desc: MoeDescriptor, max_tokens: int):
    dims = (ctypes.c_int32 * 7)()
    symbol = ctypes.create_string_buffer(128)
    _check("moe_launch_geometry", _abi.lib().lunaflux_fp8_moe_launch_geometry(
        entry, ctypes.byref(desc), max_tokens, dims, symbol))
    return (KernelLaunchDimensions.new(tuple(dims[0:3]), tuple(dims[3:6]), dims[6]),
            symbol.value.decode("ascii"))


@dataclass
class BoundMoe(BoundOperation):
    desc: MoeDescriptor = None


def bind_moe(rt: ProjectionRuntime, counts, desc: MoeDescriptor, desc_region: KernelArgument,
             logits: KernelArgument, x: KernelArgument, wg: Fp8Weight, wu: Fp8Weight,
             wd: Fp8Weight, out: KernelArgument, max_tokens: int) -> BoundMoe:
    """Binds one MoE expert-MLP operation to its regions: 8 launch steps,
    fewer where the geometry gives a step an empty symbol (no launch): the
    hidden quantizer when the gate/up epilogue (block scales) or the down
    launch (lf_moe_down_t256_aq: per-token scales on 256-row tiles, with
    the workspace's counter area as a fifth operand and its error word read
    after a synchronous launch) runs it, and the two sort steps and the
    token quantizer when the route step's kernel (lf_moe_route_sort,
    profiles of at most 1024 assignments) does their work."""
    e, h, i = desc.experts, desc.hidden, desc.inter
    mode = _abi.LF_FP8_SCALE_BLOCK128 if desc.group == 128 else _abi.LF_FP8_SCALE_PER_CHANNEL
    for w, rows, cols in ((wg, i, h), (wu, i, h), (wd, h, i)):
        if (w.experts, w.rows, w.columns, w.scale_mode) != (e, rows, cols, mode):
            raise DeviceError("moe weight shape", _abi.LF_INVALID_ARGUMENT)
        w.admit(_abi.ENTRY_GROUPED)
    nbytes = workspace_bytes(desc, max_tokens)
    ws = rt.context.allocate(nbytes)
    # the counter area of a down launch with the hidden quantizer inside:
    # zero-filled once here, back at zero after every launch
    sync_at = sync_offset(desc, max_tokens)
    if sync_at is not None:
        ws.copy_from_host(np.zeros(nbytes, np.uint8))
    wsr = _region(ws, alignment=256)
    c = _region(counts, COUNTS_BYTES, alignment=4)

    def step(entry, operands):
        dims, symbol = launch_geometry(entry, desc, max_tokens)
        if not symbol:
            return None
        return LaunchStep(rt.function(symbol), dims, KernelArguments(operands), symbol)

    steps = [
        step(_abi.MOE_ROUTE, [c, desc_region, logits, x, wsr]),
        step(_abi.MOE_SORT_COUNT, [c, desc_region, wsr]),
        step(_abi.MOE_SORT, [c, desc_region, wsr]),
        step(_abi.MOE_QUANT_TOKENS, [c, desc_region, x, wsr]),
        step(_abi.MOE_GATE_UP, [c, desc_region, wg.region, wu.region, wsr]),
        step(_abi.MOE_QUANT_HIDDEN, [c, desc_region, wsr]),
        step(_abi.MOE_DOWN, [c, desc_region, wd.region, wsr]
             + ([_region(ws, nbytes - sync_at, sync_at, alignment=256)] if sync_at is not None else [])),
        step(_abi.MOE_COMBINE, [c, desc_region, wsr, out]),
    ]
    return BoundMoe(steps=[s for s in steps if s is not None], workspace=ws, desc=desc,
                    error_offset=sync_at)


def moe_expert_mlp(rt: ProjectionRuntime, x: np.ndarray, logits: np.ndarray, wg: Fp8Weight,
                   wu: Fp8Weight, wd: Fp8Weight, top_k: int, route_mode: int, group: int = 0,
                   max_tokens: int | None = None, return_workspace: bool = False):
    """x bf16 bits [T, H], logits fp32 [T, E] -> out bf16 bits [T, H]. With
    return_workspace, also returns the routing intermediates read back from
    the device (top-k ids and weights, sorted assignments, positions, expert
    row offsets and 128- and 256-row tile offsets)."""
    x = np.ascontiguousarray(x, np.uint16)
    logits = np.ascontiguousarray(logits, np.float32)
    t, hdim = x.shape
    e = logits.shape[1]
    desc = moe_descriptor(e, top_k, route_mode, hdim, wg.rows, group)
    max_tokens = max(t, 1) if max_tokens is None else max_tokens
    if t > max_tokens:
        raise DeviceError("tokens exceed max_tokens", _abi.LF_INVALID_ARGUMENT)
    ctx = rt.context
    xa = ctx.allocate(max_tokens * hdim * 2)
    xa.copy_from_host(x)
    la = ctx.allocate(max_tokens * e * 4)
    la.copy_from_host(logits)
    da = ctx.upload(desc.as_bytes())
    oa = ctx.allocate(max_tokens * hdim * 2)
    counts = rt.step_counts(t, decode=False)
    op = bind_moe(rt, counts, desc, _region(da, 32, alignment=4), _region(la, alignment=256),
                  _region(xa, alignment=256), wg, wu, wd, _region(oa, alignment=256), max_tokens)
    op.launch(rt.stream, synchronous=True)
    out = oa.read(np.uint16, (t, hdim)) if t else np.zeros((0, hdim), np.uint16)
    if not return_workspace:
        return out
    gate_up = next(s for s in op.steps if s.name.startswith("lf_moe_gate_up"))
    if gate_up.name.endswith("_q"):
        # The plan quantized h in the gate/up epilogue and never stored it;
        # for inspection the unfused kernel writes the bf16 h (and nothing
        # else the intermediates below hold).
        plain = gate_up.name[:-2]
        LaunchStep(rt.function(plain), gate_up.dims, gate_up.args, plain).launch(
            rt.stream, synchronous=True)
    lay = workspace_layout(desc, t)
    a = t * top_k
    ws = op.workspace
    i = wg.rows
    gx = hdim // group if group else 1
    gh = i // group if group else 1
    inter = dict(
        topk_ids=ws.read(np.int32, (t, top_k), lay["topk_ids"]),
        topk_w=ws.read(np.float32, (t, top_k), lay["topk_w"]),
        sorted=ws.read(np.int32, (a,), lay["sorted"]),
        pos=ws.read(np.int32, (a,), lay["pos"]),
        offsets=ws.read(np.int32, (e + 1,), lay["offsets"]),
        tiles=ws.read(np.int32, (e + 1,), lay["tiles"]),
        tiles256=ws.read(np.int32, (e + 1,), lay["tiles"] + 4 * (e + 1)),
        live_experts=ws.read(np.int32, (e + 1,), lay["tiles"] + 8 * (e + 1)),
        xq=ws.read(np.uint8, (t, hdim), lay["xq"]),
        xs=ws.read(np.float32, (t, gx), lay["xs"]),
        h=ws.read(np.uint16, (a, i), lay["h"]),
        hq=ws.read(np.uint8, (a, i), lay["hq"]),
        hs=ws.read(np.float32, (a, gh), lay["hs"]),
        y=(ws.read(np.uint16, (a, hdim), lay["y"]).astype(np.uint32) << 16).view(np.float32),
    )
    return out, inter

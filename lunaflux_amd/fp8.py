"""Host side of the FP8 projection path.

The reference executes each plan operation as one AOT entry point with a
prebuilt operand list (kernels/launch_contract/paged_admit.mbt:76-107,
engine/device_step/paged_executor_run.mbt:112-143). This module builds those
launch steps for the FP8 families and offers numpy-level calls named after
the reference kernels they replace (kernels/reference/basic.mbt:102-153,
mlp.mbt:4-39), so parity tests read like the reference's own tests:

  dense_projection(x, w)          output / down projection
  language_model_head(x, w)       vocabulary logits (the dense entry)
  qkv_projection(x, wq, wk, wv)   packed Q|K|V
  gate_up_swiglu(x, wg, wu)       silu(x Wg^T) * (x Wu^T), the first half of
                                  silu_gated_mlp
  silu_gated_mlp(x, wg, wu, wd)   the whole GatedMlp operation
  rms_norm_quant(x, g, w, eps)    RmsNorm (kernels/reference/basic.mbt:32-68)
                                  written as the per-token e4m3 rows the W8A8
                                  projection with first weight w reads

Two families (include/lunaflux_fp8.h): "w8a16" (bf16 activations, decode)
and "w8a8" (per-token e4m3 activations, prefill). Activations and outputs
are bf16 carried as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _abi
from .device import (Allocation, DeviceError, Function, KernelArgument, KernelArguments,
                     KernelLaunchDimensions, Stream, open_context)

FAMILIES = ("w8a16", "w8a8")
# The entry of (family, operation) for weights with 128 x 128 block scales.
_BLOCK_ENTRIES = {
    ("w8a16", "dense"): _abi.ENTRY_W8A16_DENSE_B128,
    ("w8a16", "qkv"): _abi.ENTRY_W8A16_QKV_B128,
    ("w8a16", "gate_up"): _abi.ENTRY_W8A16_GATE_UP_B128,
    ("w8a8", "dense"): _abi.ENTRY_W8A8_DENSE_B128,
    ("w8a8", "qkv"): _abi.ENTRY_W8A8_QKV_B128,
    ("w8a8", "gate_up"): _abi.ENTRY_W8A8_GATE_UP_B128,
}
PER_CHANNEL = _abi.LF_FP8_SCALE_PER_CHANNEL
BLOCK128 = _abi.LF_FP8_SCALE_BLOCK128
W8A16_MAX_TOKENS = 128
COUNTS_BYTES = 20


def _check(operation, status):
    if status != _abi.LF_OK:
        raise DeviceError(operation, status)


def weight_region_bytes(rows: int, columns: int, experts: int = 1,
                        scale_mode: int = PER_CHANNEL) -> int:
    out = ctypes.c_int64(0)
    _check("weight_region_bytes", _abi.lib().lunaflux_fp8_weight_region_bytes(
        scale_mode, rows, columns, experts, ctypes.byref(out)))
    return out.value


def scale_count(rows: int, columns: int, experts: int = 1, scale_mode: int = PER_CHANNEL) -> int:
    """fp32 scales of a weight: N per expert per channel, (N/128)(K/128) per
    expert for 128 x 128 blocks."""
    per = rows if scale_mode == PER_CHANNEL else (rows // 128) * (columns // 128)
    return experts * per


def pack_weight(q: np.ndarray, scales: np.ndarray, scale_mode: int = PER_CHANNEL) -> np.ndarray:
    """Pre-swizzles e4m3 codes [N, K] (or [E, N, K]) and their fp32 scales
    into one weight region (header + MFMA-order tiles + scales). The scale
    array must hold exactly the scale block's count (DeviceError
    INVALID_ARGUMENT otherwise: the library checks both counts before it
    reads either array)."""
    q = np.ascontiguousarray(q, np.uint8)
    if q.ndim == 2:
        q = q[None]
    experts, rows, columns = q.shape
    scales = np.ascontiguousarray(scales, np.float32)
    size = weight_region_bytes(rows, columns, experts, scale_mode)
    region = np.empty(size, np.uint8)
    _check("pack_weight", _abi.lib().lunaflux_fp8_pack_weight(
        scale_mode, rows, columns, experts,
        q.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), q.size,
        scales.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), scales.size,
        region.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), size))
    return region


def admit_weight(entry: int, head: np.ndarray, region_bytes: int, rows: int, columns: int,
                 experts: int = 1):
    """lunaflux_fp8_admit_weight: raises DeviceError (UNSUPPORTED for a
    block-scaled region on a dense entry, INVALID_ARGUMENT for a region that
    is not the format's for this shape)."""
    head = np.ascontiguousarray(head, np.uint8)
    _check("admit_weight", _abi.lib().lunaflux_fp8_admit_weight(
        entry, head.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), head.size, region_bytes,
        rows, columns, experts))


def unpack_weight(region: np.ndarray):
    """Inverse of pack_weight: (q [E, N, K], scales, header fields)."""
    region = np.ascontiguousarray(region, np.uint8)
    head = region[:32].view(np.uint32)
    scale_mode, rows, columns, experts = int(head[3]), int(head[4]), int(head[5]), int(head[6])
    per = rows if scale_mode == PER_CHANNEL else (rows // 128) * (columns // 128)
    q = np.empty((experts, rows, columns), np.uint8)
    s = np.empty(experts * per, np.float32)
    _check("unpack_weight", _abi.lib().lunaflux_fp8_unpack_weight(
        region.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), region.size,
        q.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), q.size,
        s.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), s.size))
    return q, s.reshape(experts, -1), dict(scale_mode=scale_mode, rows=rows, columns=columns,
                                           experts=experts)


def act_quant_bytes(max_rows: int, columns: int) -> int:
    n = _abi.lib().lunaflux_fp8_act_quant_bytes(max_rows, columns)
    if n < 0:
        raise DeviceError("act_quant_bytes", _abi.LF_INVALID_ARGUMENT)
    return n


def w8a16_workspace_bytes(entry: int, n: int, k: int, max_tokens: int,
                          qkv_split: tuple[int, int] | None = None) -> int:
    """Split-K workspace bytes; qkv_split = (Nq, Nkv) lets a QKV operation
    select its shape-specialized entry."""
    if qkv_split is not None:
        nbytes = _abi.lib().lunaflux_fp8_qkv_w8a16_workspace_bytes(*qkv_split, k, max_tokens)
    else:
        nbytes = _abi.lib().lunaflux_fp8_w8a16_workspace_bytes(entry, n, k, max_tokens)
    if nbytes < 0:
        raise DeviceError("w8a16_workspace_bytes", _abi.LF_INVALID_ARGUMENT)
    return nbytes


def w8a8_workspace_bytes(entry: int, n: int, k: int, max_tokens: int) -> int:
    """Workspace of a one-launch W8A8 entry (_AQ): the sync area, then the
    quantized rows for the profile."""
    nbytes = _abi.lib().lunaflux_fp8_w8a8_workspace_bytes(entry, n, k, max_tokens)
    if nbytes < 0:
        raise DeviceError("w8a8_workspace_bytes", _abi.LF_INVALID_ARGUMENT)
    return nbytes


def launch_geometry(entry: int, n: int, k: int, max_tokens: int,
                    qkv_split: tuple[int, int] | None = None):
    dims = (ctypes.c_int32 * 7)()
    symbol = ctypes.create_string_buffer(128)
    if qkv_split is not None:
        _check("launch_geometry", _abi.lib().lunaflux_fp8_qkv_launch_geometry(
            entry, *qkv_split, k, max_tokens, dims, symbol))
    else:
        _check("launch_geometry", _abi.lib().lunaflux_fp8_launch_geometry(
            entry, n, k, max_tokens, dims, symbol))
    return (KernelLaunchDimensions.new(tuple(dims[0:3]), tuple(dims[3:6]), dims[6]),
            symbol.value.decode("ascii"))


def gated_mlp_geometry(hidden: int, inter: int, max_tokens: int,
                       entry: int = _abi.ENTRY_W8A16_GATED_MLP):
    """(dims, symbol) of the one-launch GatedMlp entry (W8A16 or W8A8) for the
    shape and profile, or None where none is built."""
    dims = (ctypes.c_int32 * 7)()
    symbol = ctypes.create_string_buffer(128)
    status = _abi.lib().lunaflux_fp8_gated_mlp_geometry(entry, hidden, inter, max_tokens, dims, symbol)
    if status == _abi.LF_UNSUPPORTED:
        return None
    _check("gated_mlp_geometry", status)
    return (KernelLaunchDimensions.new(tuple(dims[0:3]), tuple(dims[3:6]), dims[6]),
            symbol.value.decode("ascii"))


def rms_norm_quant_geometry(epsilon: float, k: int, max_rows: int):
    """(dims, symbol) of the fused RmsNorm + quantizer entry for an epsilon
    (fp32), input width K and profile; DeviceError(UNSUPPORTED) for an
    epsilon with no built entry."""
    dims = (ctypes.c_int32 * 7)()
    symbol = ctypes.create_string_buffer(128)
    _check("rms_norm_quant_geometry", _abi.lib().lunaflux_fp8_rms_norm_quant_geometry(
        float(np.float32(epsilon)), k, max_rows, dims, symbol))
    return (KernelLaunchDimensions.new(tuple(dims[0:3]), tuple(dims[3:6]), dims[6]),
            symbol.value.decode("ascii"))


@dataclass
class Fp8Weight:
    """One device-resident weight region (a TensorRef's region) and the
    host copy of its header, which admission checks."""

    allocation: Allocation
    rows: int
    columns: int
    experts: int
    scale_mode: int
    header: np.ndarray = None

    @property
    def region(self) -> KernelArgument:
        return KernelArgument.device_region(self.allocation, 0, self.allocation.byte_count, 256)

    def admit(self, entry: int):
        """Admission for an operand of `entry` (lunaflux_fp8_admit_weight)."""
        admit_weight(entry, self.header, self.allocation.byte_count, self.rows, self.columns,
                     self.experts)


@dataclass
class LaunchStep:
    """One kernel launch of a plan operation: function, geometry, operands."""

    function: Function
    dims: KernelLaunchDimensions
    args: KernelArguments
    name: str = ""

    def launch(self, stream: Stream, synchronous: bool = True):
        if synchronous:
            self.function.launch_synchronous(self.dims, self.args, stream)
        else:
            self.function.launch_async(self.dims, self.args, stream)


@dataclass
class BoundOperation:
    """A plan operation bound to its regions: one or more launch steps run
    in order on one stream.

    error_offset: byte offset in the workspace of the int32 error word of an
    entry with counted waits (kernels/phases.h), or None. A synchronous
    launch reads it back; a set word (a wait ran out: never on a correct
    launch) zero-fills the workspace, which puts its counters back at rest,
    and raises DeviceError(LF_DRIVER_FAILURE). check() does the same after
    asynchronous launches."""

    steps: list
    workspace: Allocation | None = None
    keep: list = field(default_factory=list)
    error_offset: int | None = None

    def launch(self, stream: Stream, synchronous: bool = True):
        for i, step in enumerate(self.steps):
            step.launch(stream, synchronous and i == len(self.steps) - 1)
        if synchronous:
            self.check()

    def check(self):
        """Raises DeviceError if a counted wait of an earlier launch ran out
        (the caller synchronizes the stream first)."""
        if self.error_offset is None:
            return
        word = self.workspace.read(np.int32, (1,), self.error_offset)[0]
        if word != 0:
            self.workspace.copy_from_host(np.zeros(self.workspace.byte_count, np.uint8))
            raise DeviceError("a counted wait of a one-launch entry ran out", _abi.LF_DRIVER_FAILURE)


@dataclass
class _Chain(BoundOperation):
    """An operation bound as the steps of several bound operations in order
    (their workspaces kept alive); check() checks each part's error word."""

    parts: list = field(default_factory=list)

    def check(self):
        for part in self.parts:
            part.check()


def _region(alloc: Allocation, byte_count: int | None = None, offset: int = 0,
            alignment: int = 16) -> KernelArgument:
    n = alloc.byte_count - offset if byte_count is None else byte_count
    return KernelArgument.device_region(alloc, offset, n, alignment)


class ProjectionRuntime:
    """A device context with the FP8 code object loaded."""

    def __init__(self, ordinal: int = 0):
        self.context = open_context(ordinal)
        self.stream = self.context.create_stream()
        self.module = self.context.load_module(_abi.code_object_bytes())
        self._functions = {}

    # -- resources ---------------------------------------------------------
    def function(self, symbol: str) -> Function:
        fn = self._functions.get(symbol)
        if fn is None:
            fn = self.module.load_function(symbol)
            self._functions[symbol] = fn
        return fn

    def upload_weight(self, q: np.ndarray, scales: np.ndarray,
                      scale_mode: int = PER_CHANNEL) -> Fp8Weight:
        return self.weight_from_region(pack_weight(q, scales, scale_mode))

    def weight_from_region(self, region: np.ndarray) -> Fp8Weight:
        head = np.ascontiguousarray(region[:32]).view(np.uint32)
        return Fp8Weight(self.context.upload(region), int(head[4]), int(head[5]), int(head[6]),
                         int(head[3]), np.array(region[:_abi.LF_FP8_HEADER_BYTES], np.uint8))

    def step_counts(self, query_tokens: int, decode: bool = True) -> Allocation:
        """StepCounts int32[5] = {prefill_rows, decode_rows, total_rows,
        query_tokens, page_entries} (engine/device_step/stage.mbt:59-68)."""
        rows = query_tokens
        counts = np.array([0 if decode else 1, rows if decode else 0, rows if decode else 1,
                           query_tokens, 0], np.int32)
        return self.context.upload(counts)

    def _step(self, entry: int, n: int, k: int, max_tokens: int, operands,
              qkv_split=None) -> LaunchStep:
        dims, symbol = launch_geometry(entry, n, k, max_tokens, qkv_split)
        return LaunchStep(self.function(symbol), dims, KernelArguments(operands), symbol)

    def _w8a16(self, entry: int, n: int, k: int, max_tokens: int, operands,
               qkv_split=None) -> BoundOperation:
        """A W8A16 launch with its split-K workspace (zero-filled once here;
        the kernels leave its arrival counters at zero after every launch)."""
        # (the Q / K-V split selects a shape-specialized per-channel entry;
        # the block-scaled QKV entry is sized by its packed width)
        nbytes = w8a16_workspace_bytes(entry, n, k, max_tokens,
                                       qkv_split if entry == _abi.ENTRY_W8A16_QKV else None)
        ws = self.context.allocate(nbytes)
        ws.copy_from_host(np.zeros(nbytes, np.uint8))
        step = self._step(entry, n, k, max_tokens, operands + [_region(ws, alignment=256)],
                          qkv_split)
        return BoundOperation([step], workspace=ws)

    def _w8a8_one_launch(self, entry: int, n: int, k: int, max_tokens: int, operands,
                         qkv_split=None) -> BoundOperation:
        """A one-launch W8A8 operation (_AQ entry): bf16 x in, the quantizer
        and the GEMM as counted steps of one grid; its workspace (sync area,
        quantized rows) zero-filled once here."""
        nbytes = w8a8_workspace_bytes(entry, n, k, max_tokens)
        ws = self.context.allocate(nbytes)
        ws.copy_from_host(np.zeros(nbytes, np.uint8))
        step = self._step(entry, n, k, max_tokens, operands + [_region(ws, alignment=256)], qkv_split)
        return BoundOperation([step], workspace=ws, error_offset=_abi.LF_FP8_AQ_ERROR_OFFSET)

    # -- binding plan operations to launch steps ---------------------------
    def bind_act_quant(self, counts: Allocation, x: KernelArgument, w: Fp8Weight,
                       xq: KernelArgument, max_tokens: int) -> LaunchStep:
        return self._step(_abi.ENTRY_ACT_QUANT_ROWS, w.rows, w.columns, max_tokens,
                          [_region(counts, COUNTS_BYTES, alignment=4), x, w.region, xq])

    def bind_rms_norm_quant(self, counts: Allocation, x: KernelArgument, gamma: KernelArgument,
                            w: Fp8Weight, xq: KernelArgument, max_tokens: int,
                            epsilon: float) -> LaunchStep:
        """The RmsNorm operation (kernels/reference/basic.mbt:32-68) writing
        per-token e4m3 rows for the W8A8 projection whose first weight is w
        (xq: lunaflux_fp8_act_quant_bytes(max_tokens, K) bytes)."""
        dims, symbol = rms_norm_quant_geometry(epsilon, w.columns, max_tokens)
        return LaunchStep(self.function(symbol), dims, KernelArguments(
            [_region(counts, COUNTS_BYTES, alignment=4), x, gamma, w.region, xq]), symbol)

    def bind_dense_quantized(self, counts: Allocation, xq: KernelArgument, w: Fp8Weight,
                             y: KernelArgument, max_tokens: int) -> LaunchStep:
        """The W8A8 dense GEMM alone, over rows already quantized (by
        bind_rms_norm_quant or bind_act_quant)."""
        w.admit(_abi.ENTRY_W8A8_DENSE)
        return self._step(_abi.ENTRY_W8A8_DENSE, w.rows, w.columns, max_tokens,
                          [_region(counts, COUNTS_BYTES, alignment=4), xq, w.region, y])

    def _block(self, family: str, op: str, counts: Allocation, weights, operands, n: int, k: int,
               max_tokens: int, qkv_split=None) -> BoundOperation:
        """A projection over weights with 128 x 128 block scales: the _B128
        entry of the family (W8A16: the column-group form with its split-K
        workspace; W8A8: one launch, the per-128-column-group quantizer
        inside it)."""
        entry = _BLOCK_ENTRIES[(family, op)]
        for w in weights:
            w.admit(entry)
        c = _region(counts, COUNTS_BYTES, alignment=4)
        if family == "w8a16":
            return self._w8a16(entry, n, k, max_tokens, [c, *operands], qkv_split)
        return self._w8a8_one_launch(entry, n, k, max_tokens, [c, *operands], qkv_split)

    def bind_dense(self, family: str, counts: Allocation, x: KernelArgument, w: Fp8Weight,
                   y: KernelArgument, max_tokens: int, one_launch: bool = True) -> BoundOperation:
        """OutputProjection / down / the vocabulary head. W8A8: one launch
        (the _aq entry quantizes x inside it); one_launch=False binds the
        act-quant launch and the GEMM-only launch instead (same outputs).
        A weight with 128 x 128 block scales binds the family's _B128 entry
        (one launch in both families, whatever one_launch says)."""
        _family(family, max_tokens)
        if w.scale_mode == BLOCK128:
            return self._block(family, "dense", counts, [w], [x, w.region, y], w.rows, w.columns,
                               max_tokens)
        w.admit(_abi.ENTRY_W8A16_DENSE if family == "w8a16" else _abi.ENTRY_W8A8_DENSE)
        c = _region(counts, COUNTS_BYTES, alignment=4)
        if family == "w8a16":
            return self._w8a16(_abi.ENTRY_W8A16_DENSE, w.rows, w.columns, max_tokens,
                               [c, x, w.region, y])
        if one_launch:
            w.admit(_abi.ENTRY_W8A8_DENSE_AQ)
            return self._w8a8_one_launch(_abi.ENTRY_W8A8_DENSE_AQ, w.rows, w.columns, max_tokens,
                                         [c, x, w.region, y])
        ws = self.context.allocate(act_quant_bytes(max_tokens, w.columns))
        xq = _region(ws, alignment=256)
        return BoundOperation([
            self.bind_act_quant(counts, x, w, xq, max_tokens),
            self._step(_abi.ENTRY_W8A8_DENSE, w.rows, w.columns, max_tokens, [c, xq, w.region, y]),
        ], workspace=ws)

    def bind_qkv(self, family: str, counts: Allocation, x: KernelArgument, wq: Fp8Weight,
                 wk: Fp8Weight, wv: Fp8Weight, y: KernelArgument, max_tokens: int,
                 one_launch: bool = True) -> BoundOperation:
        _family(family, max_tokens)
        if not (wq.columns == wk.columns == wv.columns) or wk.rows != wv.rows:
            raise DeviceError("qkv shapes", _abi.LF_INVALID_ARGUMENT)
        n = wq.rows + wk.rows + wv.rows
        if wq.scale_mode == BLOCK128 or wk.scale_mode == BLOCK128 or wv.scale_mode == BLOCK128:
            return self._block(family, "qkv", counts, [wq, wk, wv],
                               [x, wq.region, wk.region, wv.region, y], n, wq.columns, max_tokens,
                               qkv_split=(wq.rows, wk.rows))
        for w in (wq, wk, wv):
            w.admit(_abi.ENTRY_W8A16_QKV if family == "w8a16" else _abi.ENTRY_W8A8_QKV)
        c = _region(counts, COUNTS_BYTES, alignment=4)
        if family == "w8a16":
            return self._w8a16(_abi.ENTRY_W8A16_QKV, n, wq.columns, max_tokens,
                               [c, x, wq.region, wk.region, wv.region, y],
                               qkv_split=(wq.rows, wk.rows))
        if one_launch:
            return self._w8a8_one_launch(_abi.ENTRY_W8A8_QKV_AQ, n, wq.columns, max_tokens,
                                         [c, x, wq.region, wk.region, wv.region, y],
                                         qkv_split=(wq.rows, wk.rows))
        ws = self.context.allocate(act_quant_bytes(max_tokens, wq.columns))
        xq = _region(ws, alignment=256)
        return BoundOperation([
            self.bind_act_quant(counts, x, wq, xq, max_tokens),
            self._step(_abi.ENTRY_W8A8_QKV, n, wq.columns, max_tokens,
                       [c, xq, wq.region, wk.region, wv.region, y]),
        ], workspace=ws)

    def bind_gate_up(self, family: str, counts: Allocation, x: KernelArgument, wg: Fp8Weight,
                     wu: Fp8Weight, h: KernelArgument, max_tokens: int,
                     one_launch: bool = True) -> BoundOperation:
        _family(family, max_tokens)
        if wg.rows != wu.rows or wg.columns != wu.columns:
            raise DeviceError("gate/up shapes", _abi.LF_INVALID_ARGUMENT)
        if wg.scale_mode == BLOCK128 or wu.scale_mode == BLOCK128:
            return self._block(family, "gate_up", counts, [wg, wu], [x, wg.region, wu.region, h],
                               wg.rows, wg.columns, max_tokens)
        for w in (wg, wu):
            w.admit(_abi.ENTRY_W8A16_GATE_UP if family == "w8a16" else _abi.ENTRY_W8A8_GATE_UP)
        c = _region(counts, COUNTS_BYTES, alignment=4)
        if family == "w8a16":
            return self._w8a16(_abi.ENTRY_W8A16_GATE_UP, wg.rows, wg.columns, max_tokens,
                               [c, x, wg.region, wu.region, h])
        if one_launch:
            return self._w8a8_one_launch(_abi.ENTRY_W8A8_GATE_UP_AQ, wg.rows, wg.columns, max_tokens,
                                         [c, x, wg.region, wu.region, h])
        ws = self.context.allocate(act_quant_bytes(max_tokens, wg.columns))
        xq = _region(ws, alignment=256)
        return BoundOperation([
            self.bind_act_quant(counts, x, wg, xq, max_tokens),
            self._step(_abi.ENTRY_W8A8_GATE_UP, wg.rows, wg.columns, max_tokens,
                       [c, xq, wg.region, wu.region, h]),
        ], workspace=ws)

    def bind_gated_mlp(self, family: str, counts: Allocation, x: KernelArgument, wg: Fp8Weight,
                       wu: Fp8Weight, wd: Fp8Weight, y: KernelArgument,
                       max_tokens: int, one_launch: bool = True) -> BoundOperation:
        """GatedMlp (model/plan/plan.mbt:47-59) as one launch, the plan's one
        AOT entry point for the operation (lunaflux_fp8_gated_mlp_geometry):
        W8A8 for any width (x quantizer, gate/up + SwiGLU, h quantizer and
        down as counted steps of one grid), W8A16 where a one-launch entry is
        built for the shape and profile. Elsewhere, or with one_launch=False,
        two launch steps: gate/up + SwiGLU into a bf16 intermediate, then the
        down projection from it (each W8A8 step then quantizes its input
        inside its own launch, or, with one_launch=False, in a launch of its
        own). Every form computes the same values. Weights with 128 x 128
        block scales: the _B128 GatedMlp entry of the family (W8A8 any width,
        W8A16 where its one-launch forms are built), else, or with
        one_launch=False, the two block-scaled launches."""
        if wd.columns != wg.rows or wd.rows != wg.columns:
            raise DeviceError("mlp shapes", _abi.LF_INVALID_ARGUMENT)
        if wg.rows != wu.rows or wg.columns != wu.columns:
            raise DeviceError("gate/up shapes", _abi.LF_INVALID_ARGUMENT)
        _family(family, max_tokens)
        modes = {wg.scale_mode, wu.scale_mode, wd.scale_mode}
        if modes == {BLOCK128}:
            entry = _abi.ENTRY_W8A8_GATED_MLP_B128 if family == "w8a8" else _abi.ENTRY_W8A16_GATED_MLP_B128
        elif BLOCK128 in modes:
            entry = None
        else:
            entry = _abi.ENTRY_W8A16_GATED_MLP if family == "w8a16" else _abi.ENTRY_W8A8_GATED_MLP
        geometry = (gated_mlp_geometry(wg.columns, wg.rows, max_tokens, entry)
                    if one_launch and entry is not None else None)
        if geometry is not None:
            for w in (wg, wu, wd):
                w.admit(entry)
            dims, symbol = geometry
            nbytes = _abi.lib().lunaflux_fp8_gated_mlp_workspace_bytes(entry, wg.columns, wg.rows,
                                                                        max_tokens)
            if nbytes < 0:
                raise DeviceError("gated_mlp_workspace_bytes", _abi.LF_INVALID_ARGUMENT)
            ws = self.context.allocate(nbytes)
            ws.copy_from_host(np.zeros(nbytes, np.uint8))
            c = _region(counts, COUNTS_BYTES, alignment=4)
            step = LaunchStep(self.function(symbol), dims,
                              KernelArguments([c, x, wg.region, wu.region, wd.region, y,
                                               _region(ws, alignment=256)]), symbol)
            error_offset = (nbytes - _abi.LF_FP8_GATED_MLP_ERROR_OFFSET_FROM_END if family == "w8a16"
                            else _abi.LF_FP8_AQ_ERROR_OFFSET)
            return BoundOperation([step], workspace=ws, error_offset=error_offset)
        h_bytes = max_tokens * wg.rows * 2
        h_alloc = self.context.allocate(h_bytes)
        h = _region(h_alloc, h_bytes, alignment=256)
        first = self.bind_gate_up(family, counts, x, wg, wu, h, max_tokens, one_launch=one_launch)
        second = self.bind_dense(family, counts, h, wd, y, max_tokens, one_launch=one_launch)
        return _Chain(first.steps + second.steps, workspace=h_alloc, parts=[first, second])

    # -- numpy convenience (tests, smoke) -----------------------------------
    def _run(self, bind, x: np.ndarray, out_shape, max_tokens):
        x = np.ascontiguousarray(x, np.uint16)
        m = x.shape[0]
        max_tokens = max(m, 1) if max_tokens is None else max_tokens
        if m > max_tokens:
            raise DeviceError("rows exceed the profile's max_query_tokens", _abi.LF_INVALID_ARGUMENT)
        # Inputs and outputs are sized for the profile (max_tokens rows), as
        # the engine's activation regions are.
        xa = self.context.allocate(max(max_tokens * x.shape[1] * 2, 16))
        xa.copy_from_host(x)
        out_bytes = max_tokens * out_shape[1] * 2
        ya = self.context.allocate(out_bytes)
        counts = self.step_counts(m)
        op = bind(counts, _region(xa, alignment=256), _region(ya, alignment=256), max_tokens)
        op.launch(self.stream, synchronous=True)
        return ya.read(np.uint16, out_shape) if m else np.zeros(out_shape, np.uint16)

    def dense_projection(self, x, w: Fp8Weight, family="w8a16", max_tokens=None):
        return self._run(lambda c, xr, yr, mt: self.bind_dense(family, c, xr, w, yr, mt),
                         x, (x.shape[0], w.rows), max_tokens)

    def language_model_head(self, x, w: Fp8Weight, family="w8a16", max_tokens=None):
        """Vocabulary logits [M, vocab] in bf16: the dense projection entry
        over the head weight [vocab, hidden], as the reference's
        `language_model_head` is `dense_projection`
        (kernels/reference/basic.mbt:175-181) and the catalog binds
        LanguageModelHead to the dense-projection capability
        (kernels/catalog/entry.mbt:92-93)."""
        return self.dense_projection(x, w, family, max_tokens)

    def qkv_projection(self, x, wq, wk, wv, family="w8a16", max_tokens=None):
        n = wq.rows + wk.rows + wv.rows
        return self._run(lambda c, xr, yr, mt: self.bind_qkv(family, c, xr, wq, wk, wv, yr, mt),
                         x, (x.shape[0], n), max_tokens)

    def gate_up_swiglu(self, x, wg, wu, family="w8a16", max_tokens=None):
        return self._run(lambda c, xr, yr, mt: self.bind_gate_up(family, c, xr, wg, wu, yr, mt),
                         x, (x.shape[0], wg.rows), max_tokens)

    def silu_gated_mlp(self, x, wg, wu, wd, family="w8a16", max_tokens=None):
        return self._run(lambda c, xr, yr, mt: self.bind_gated_mlp(family, c, xr, wg, wu, wd, yr, mt),
                         x, (x.shape[0], wd.rows), max_tokens)

    def rms_norm_quant(self, x, gamma, w: Fp8Weight, epsilon: float, max_tokens=None):
        """Runs only the fused RmsNorm + quantizer on bf16 rows x [M, K] with
        the bf16 norm weight gamma [K]: (codes [M, K], scales [M])."""
        x = np.ascontiguousarray(x, np.uint16)
        m, k = x.shape
        max_tokens = max(m, 1) if max_tokens is None else max_tokens
        xa = self.context.allocate(max_tokens * k * 2)
        if m:
            xa.copy_from_host(x)
        ga = self.context.upload(np.ascontiguousarray(gamma, np.uint16))
        ws = self.context.allocate(act_quant_bytes(max_tokens, k))
        counts = self.step_counts(m)
        step = self.bind_rms_norm_quant(counts, _region(xa, alignment=256),
                                        _region(ga, alignment=16), w,
                                        _region(ws, alignment=256), max_tokens, epsilon)
        step.launch(self.stream, synchronous=True)
        if m == 0:
            return np.zeros((0, k), np.uint8), np.zeros(0, np.float32)
        codes = ws.read(np.uint8, (m, k))
        off = (m * k + 255) // 256 * 256
        return codes, ws.read(np.float32, (m,), offset=off)

    def act_quant(self, x, w: Fp8Weight, max_tokens=None):
        """Runs only the per-token quantizer: (codes [M, K], scales [M])."""
        x = np.ascontiguousarray(x, np.uint16)
        m, k = x.shape
        max_tokens = max(m, 1) if max_tokens is None else max_tokens
        xa = self.context.allocate(max_tokens * k * 2)
        xa.copy_from_host(x)
        ws = self.context.allocate(act_quant_bytes(max_tokens, k))
        counts = self.step_counts(m)
        step = self.bind_act_quant(counts, _region(xa, alignment=256), w,
                                   _region(ws, alignment=256), max_tokens)
        step.launch(self.stream, synchronous=True)
        codes = ws.read(np.uint8, (m, k))
        off = (m * k + 255) // 256 * 256
        return codes, ws.read(np.float32, (m,), offset=off)


def _family(family: str, max_tokens: int):
    if family not in FAMILIES:
        raise ValueError(f"unknown family {family!r}; expected one of {FAMILIES}")
    if max_tokens <= 0:
        raise DeviceError("max_tokens", _abi.LF_INVALID_ARGUMENT)
    if family == "w8a16" and max_tokens > W8A16_MAX_TOKENS:
        raise DeviceError("w8a16 supports at most 128 rows", _abi.LF_INVALID_ARGUMENT)

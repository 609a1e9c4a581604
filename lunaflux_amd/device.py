"""Python mirror of LunaFlux's public `device` package over the HIP C-ABI.

Names follow the reference API so host code reads the same:
  open_context            device/execution.mbt:4-12
  Context.create_stream / create_event / allocate / load_module
                          device/execution.mbt:44-232
  Module.load_function    device/execution.mbt:238-250
  KernelLaunchDimensions  device/kernel_launch_types.mbt:45-76
  KernelArgument.device_region
                          device/kernel_launch_types.mbt:89-103
  KernelArguments         device/kernel_launch_types.mbt:117-140
  Function.launch_synchronous
                          device/kernel_launch.mbt:5-27
Errors are raised as DeviceError carrying the C status (the reference maps
the same codes to DeviceError variants, device/execution_types.mbt:4-50).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _abi


class DeviceError(RuntimeError):
    def __init__(self, operation: str, status: int):
        super().__init__(f"{operation}: {_abi.STATUS_NAMES.get(status, status)}")
        self.operation = operation
        self.status = status


def _check(operation: str, status: int):
    if status != _abi.LF_OK:
        raise DeviceError(operation, status)


def probe():
    """(availability, driver_version, device_count)."""
    out = (ctypes.c_int64 * 3)()
    availability = _abi.lib().lunaflux_hip_probe(out)
    return availability, int(out[0]), int(out[1])


@dataclass(frozen=True)
class DeviceCapability:
    total_memory: int
    major: int
    minor: int
    supports_bf16: bool
    supports_vendor_gemm: bool
    name: str


def device_info(ordinal: int = 0) -> DeviceCapability:
    numeric = (ctypes.c_int64 * 5)()
    name = (ctypes.c_uint8 * 96)()
    _check("device_info", _abi.lib().lunaflux_hip_device_info(ordinal, numeric, name))
    raw = bytes(name).split(b"\0", 1)[0].decode("ascii", "replace")
    return DeviceCapability(int(numeric[0]), int(numeric[1]), int(numeric[2]),
                            bool(numeric[3]), bool(numeric[4]), raw)


class _Handle:
    _close_fn = ""

    def __init__(self, ptr):
        self._ptr = ptr

    @property
    def ptr(self):
        return self._ptr

    def close(self):
        if self._ptr:
            _check(self._close_fn, getattr(_abi.lib(), self._close_fn)(self._ptr))

    def __del__(self):
        ptr = getattr(self, "_ptr", None)
        if ptr:
            self._ptr = None
            try:
                _abi.lib().lunaflux_hip_release(ptr)
            except Exception:  # interpreter shutdown
                pass


def _create(fn, *args, operation: str):
    status = ctypes.c_int32(0)
    ptr = fn(*args, ctypes.byref(status))
    if status.value != _abi.LF_OK:
        if ptr:
            _abi.lib().lunaflux_hip_release(ptr)
        raise DeviceError(operation, status.value)
    return ptr


class Stream(_Handle):
    _close_fn = "lunaflux_hip_stream_close"

    def synchronize(self):
        _check("stream_synchronize", _abi.lib().lunaflux_hip_stream_synchronize(self._ptr))


class Event(_Handle):
    _close_fn = "lunaflux_hip_event_close"

    def record(self, stream: Stream):
        _check("event_record", _abi.lib().lunaflux_hip_event_record(self._ptr, stream.ptr))

    def synchronize(self):
        _check("event_synchronize", _abi.lib().lunaflux_hip_event_synchronize(self._ptr))

    def elapsed_milliseconds(self, finish: "Event") -> float:
        status = ctypes.c_int32(0)
        ms = _abi.lib().lunaflux_hip_event_elapsed(self._ptr, finish.ptr, ctypes.byref(status))
        _check("event_elapsed", status.value)
        return float(ms)


class Allocation(_Handle):
    _close_fn = "lunaflux_hip_allocation_close"

    def __init__(self, ptr, byte_count: int, context: "Context"):
        super().__init__(ptr)
        self.byte_count = byte_count
        self.context = context

    def copy_from_host(self, data, offset: int = 0):
        buf = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        if buf.size == 0:
            return
        _check("copy_to_device", _abi.lib().lunaflux_hip_copy_to_device(
            self._ptr, buf.ctypes.data, buf.size, 0, offset, buf.size))

    def copy_to_host(self, byte_count: int | None = None, offset: int = 0) -> np.ndarray:
        n = self.byte_count - offset if byte_count is None else byte_count
        out = np.empty(n, np.uint8)
        if n:
            _check("copy_to_host", _abi.lib().lunaflux_hip_copy_to_host(
                self._ptr, offset, n, out.ctypes.data, n))
        return out

    def read(self, dtype, shape, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = int(np.prod(shape)) * dtype.itemsize
        return self.copy_to_host(count, offset).view(dtype).reshape(shape)

    def region(self, offset: int = 0, byte_count: int | None = None, alignment: int = 16):
        n = self.byte_count - offset if byte_count is None else byte_count
        return KernelArgument.device_region(self, offset, n, alignment)


class Function(_Handle):
    _close_fn = "lunaflux_hip_function_close"

    def __init__(self, ptr, name: str):
        super().__init__(ptr)
        self.name = name

    def launch_synchronous(self, dims: "KernelLaunchDimensions", args: "KernelArguments",
                           stream: Stream):
        _check(f"launch {self.name}", args._launch(self, dims, stream, True))

    def launch_async(self, dims: "KernelLaunchDimensions", args: "KernelArguments",
                     stream: Stream):
        _check(f"launch {self.name}", args._launch(self, dims, stream, False))

    def launch_scratch(self, dims: "KernelLaunchDimensions", args: "KernelArguments",
                       stream: Stream, scratch_bytes: int, clear: bool = True):
        """lunaflux_hip_function_launch_scratch: synchronous, allocates
        nothing; the kernel's last argument is the library's scratch array on
        this device (the first scratch_bytes of it, zeroed first when clear)."""
        _check(f"launch_scratch {self.name}", _abi.lib().lunaflux_hip_function_launch_scratch(
            self._ptr, stream.ptr, *dims.grid, *dims.block, dims.shared_memory_bytes,
            len(args.arguments), args._allocs, args._offsets, args._bytes, args._aligns,
            int(scratch_bytes), int(bool(clear))))


class Module(_Handle):
    _close_fn = "lunaflux_hip_module_close"

    def load_function(self, name: str) -> Function:
        raw = name.encode("ascii")
        buf = ctypes.create_string_buffer(raw, len(raw))
        ptr = _create(_abi.lib().lunaflux_hip_function_load, self._ptr, buf, len(raw),
                      operation=f"function_load {name}")
        return Function(ptr, name)


class Context(_Handle):
    _close_fn = "lunaflux_hip_context_close"

    def __init__(self, ptr, ordinal: int):
        super().__init__(ptr)
        self.ordinal = ordinal

    def create_stream(self) -> Stream:
        return Stream(_create(_abi.lib().lunaflux_hip_stream_create, self._ptr,
                              operation="stream_create"))

    def create_event(self) -> Event:
        return Event(_create(_abi.lib().lunaflux_hip_event_create, self._ptr,
                             operation="event_create"))

    def allocate(self, byte_count: int) -> Allocation:
        ptr = _create(_abi.lib().lunaflux_hip_allocation_create, self._ptr, int(byte_count),
                      operation="allocation_create")
        return Allocation(ptr, int(byte_count), self)

    def upload(self, data) -> Allocation:
        buf = np.ascontiguousarray(data)
        alloc = self.allocate(max(buf.nbytes, 1))
        alloc.copy_from_host(buf)
        return alloc

    def load_module(self, image: bytes) -> Module:
        buf = ctypes.create_string_buffer(image, len(image))
        return Module(_create(_abi.lib().lunaflux_hip_module_load, self._ptr, buf, len(image),
                              operation="module_load"))

    def validate_region(self, allocation: Allocation, offset: int, byte_count: int,
                        alignment: int) -> int:
        return _abi.lib().lunaflux_hip_context_validate_allocation_region(
            self._ptr, allocation.ptr, offset, byte_count, alignment)


def open_context(ordinal: int = 0) -> Context:
    return Context(_create(_abi.lib().lunaflux_hip_context_create, ordinal,
                           operation="context_create"), ordinal)


@dataclass(frozen=True)
class KernelLaunchDimensions:
    grid: tuple
    block: tuple
    shared_memory_bytes: int = 0

    @staticmethod
    def new(grid, block, shared_memory_bytes: int = 0) -> "KernelLaunchDimensions":
        grid = tuple(grid) + (1,) * (3 - len(grid))
        block = tuple(block) + (1,) * (3 - len(block))
        return KernelLaunchDimensions(grid, block, shared_memory_bytes)


@dataclass(frozen=True)
class KernelArgument:
    allocation: Allocation
    offset: int
    byte_count: int
    alignment: int

    @staticmethod
    def device_region(allocation: Allocation, offset: int, byte_count: int,
                      alignment: int) -> "KernelArgument":
        return KernelArgument(allocation, int(offset), int(byte_count), int(alignment))


class KernelArguments:
    """Prebuilt argument arrays (the reference builds them once per step,
    engine/device_step/paged_executor_prepare.mbt:184-232)."""

    def __init__(self, arguments):
        self.arguments = list(arguments)
        n = len(self.arguments)
        self._allocs = (ctypes.c_void_p * n)(*[a.allocation.ptr for a in self.arguments])
        self._offsets = (ctypes.c_int64 * n)(*[a.offset for a in self.arguments])
        self._bytes = (ctypes.c_int64 * n)(*[a.byte_count for a in self.arguments])
        self._aligns = (ctypes.c_int64 * n)(*[a.alignment for a in self.arguments])

    def _launch(self, fn: Function, dims: KernelLaunchDimensions, stream: Stream, sync: bool):
        call = (_abi.lib().lunaflux_hip_function_launch if sync
                else _abi.lib().lunaflux_hip_function_launch_async)
        return call(fn.ptr, stream.ptr, *dims.grid, *dims.block, dims.shared_memory_bytes,
                    len(self.arguments), self._allocs, self._offsets, self._bytes, self._aligns)

"""ctypes binding of liblunaflux_hip.so (include/lunaflux_hip.h and
include/lunaflux_fp8.h). This is the Python counterpart of the MoonBit
externs in /root/reference/internal/cuda/ffi.mbt:29-240: one declaration per
exported symbol, no logic.

The library must have been built (``python -m lunaflux_amd.build``); a
missing library is an error, never a fallback.
"""
from __future__ import annotations

import ctypes
import os

PACKAGE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(PACKAGE, "liblunaflux_hip.so")
CODE_OBJECT_PATH = os.path.join(PACKAGE, "lunaflux_fp8.hsaco")

# internal/cuda/cuda_abi.h:44-54
LF_OK = 0
LF_UNAVAILABLE = -1
LF_INVALID_ARGUMENT = -2
LF_CLOSED = -3
LF_BUSY = -4
LF_DRIVER_FAILURE = -5
LF_HOST_ALLOCATION_FAILED = -6
LF_SIZE_OVERFLOW = -7
LF_UNSUPPORTED = -8

STATUS_NAMES = {
    LF_OK: "OK", LF_UNAVAILABLE: "UNAVAILABLE", LF_INVALID_ARGUMENT: "INVALID_ARGUMENT",
    LF_CLOSED: "CLOSED", LF_BUSY: "BUSY", LF_DRIVER_FAILURE: "DRIVER_FAILURE",
    LF_HOST_ALLOCATION_FAILED: "HOST_ALLOCATION_FAILED", LF_SIZE_OVERFLOW: "SIZE_OVERFLOW",
    LF_UNSUPPORTED: "UNSUPPORTED",
}

LF_AVAILABLE = 0
LF_NO_DEVICES = 5

# include/lunaflux_hip.h
LF_SCRATCH_MAX_BYTES = 16 << 20

# include/lunaflux_fp8.h
LF_FP8_SCALE_PER_CHANNEL = 1
LF_FP8_SCALE_BLOCK128 = 2
LF_FP8_HEADER_BYTES = 256
ENTRY_ACT_QUANT_ROWS = 1
ENTRY_W8A16_DENSE = 2
ENTRY_W8A16_QKV = 3
ENTRY_W8A16_GATE_UP = 4
ENTRY_W8A8_DENSE = 5
ENTRY_W8A8_QKV = 6
ENTRY_W8A8_GATE_UP = 7
ENTRY_RMS_NORM_QUANT_ROWS = 8
ENTRY_GROUPED = 9
ENTRY_W8A16_GATED_MLP = 10
ENTRY_W8A8_DENSE_AQ = 11
ENTRY_W8A8_QKV_AQ = 12
ENTRY_W8A8_GATE_UP_AQ = 13
ENTRY_W8A8_GATED_MLP = 14
ENTRY_W8A16_DENSE_B128 = 15
ENTRY_W8A16_QKV_B128 = 16
ENTRY_W8A16_GATE_UP_B128 = 17
ENTRY_W8A8_DENSE_B128 = 18
ENTRY_W8A8_QKV_B128 = 19
ENTRY_W8A8_GATE_UP_B128 = 20
ENTRY_W8A8_GATED_MLP_B128 = 21
ENTRY_W8A16_GATED_MLP_B128 = 22
LF_FP8_GATED_MLP_ERROR_OFFSET_FROM_END = 128
LF_FP8_AQ_ERROR_OFFSET = 0

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)

SIGNATURES = {
    "lunaflux_hip_probe": (_i32, [_i64p]),
    "lunaflux_hip_device_info": (_i32, [_i32, _i64p, _u8p]),
    "lunaflux_hip_release": (None, [_vp]),
    "lunaflux_hip_context_create": (_vp, [_i32, _i32p]),
    "lunaflux_hip_context_close": (_i32, [_vp]),
    "lunaflux_hip_stream_create": (_vp, [_vp, _i32p]),
    "lunaflux_hip_stream_close": (_i32, [_vp]),
    "lunaflux_hip_stream_synchronize": (_i32, [_vp]),
    "lunaflux_hip_event_create": (_vp, [_vp, _i32p]),
    "lunaflux_hip_event_close": (_i32, [_vp]),
    "lunaflux_hip_event_record": (_i32, [_vp, _vp]),
    "lunaflux_hip_event_synchronize": (_i32, [_vp]),
    "lunaflux_hip_event_elapsed": (ctypes.c_double, [_vp, _vp, _i32p]),
    "lunaflux_hip_allocation_create": (_vp, [_vp, _i64, _i32p]),
    "lunaflux_hip_allocation_close": (_i32, [_vp]),
    "lunaflux_hip_allocation_lease_create": (_vp, [_vp, _vp, _i32p]),
    "lunaflux_hip_allocation_lease_close": (_i32, [_vp]),
    "lunaflux_hip_context_validate_allocation_region": (_i32, [_vp, _vp, _i64, _i64, _i64]),
    "lunaflux_hip_copy_to_device": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64]),
    "lunaflux_hip_context_copy_fixed_to_device": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64]),
    "lunaflux_hip_context_copy_device_to_fixed": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64]),
    "lunaflux_hip_copy_to_host": (_i32, [_vp, _i64, _i64, _vp, _i64]),
    "lunaflux_hip_module_load": (_vp, [_vp, _vp, _i64, _i32p]),
    "lunaflux_hip_module_close": (_i32, [_vp]),
    "lunaflux_hip_function_load": (_vp, [_vp, _vp, _i64, _i32p]),
    "lunaflux_hip_function_close": (_i32, [_vp]),
    "lunaflux_hip_function_launch": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                            _vp, _i64p, _i64p, _i64p]),
    "lunaflux_hip_function_launch_async": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                                  _i32, _vp, _i64p, _i64p, _i64p]),
    "lunaflux_hip_function_launch_scratch": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32,
                                                    _i32, _i32, _vp, _i64p, _i64p, _i64p, _i64,
                                                    _i32]),
    "lunaflux_hip_blas_create": (_vp, [_vp, _i32p]),
    "lunaflux_hip_blas_close": (_i32, [_vp]),
    "lunaflux_hip_bf16_gemm_plan_create": (_vp, [_vp, _i64, _i64, _i64, _i64, _i32p]),
    "lunaflux_hip_bf16_gemm_plan_close": (_i32, [_vp]),
    "lunaflux_hip_bf16_gemm_plan_run": (_i32, [_vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp]),
    "lunaflux_fp8_weight_region_bytes": (_i32, [_i32, _i64, _i64, _i32, _i64p]),
    "lunaflux_fp8_pack_weight": (_i32, [_i32, _i64, _i64, _i32, _u8p, _i64, _f32p, _i64, _u8p,
                                        _i64]),
    "lunaflux_fp8_admit_weight": (_i32, [_i32, _u8p, _i64, _i64, _i64, _i64, _i32]),
    "lunaflux_fp8_unpack_weight": (_i32, [_u8p, _i64, _u8p, _i64, _f32p, _i64]),
    "lunaflux_fp8_act_quant_bytes": (_i64, [_i64, _i64]),
    "lunaflux_fp8_w8a16_workspace_bytes": (_i64, [_i32, _i64, _i64, _i32]),
    "lunaflux_fp8_w8a8_workspace_bytes": (_i64, [_i32, _i64, _i64, _i32]),
    "lunaflux_fp8_launch_geometry": (_i32, [_i32, _i64, _i64, _i32, _i32p, ctypes.c_char_p]),
    "lunaflux_fp8_gated_mlp_geometry": (_i32, [_i32, _i64, _i64, _i32, _i32p, ctypes.c_char_p]),
    "lunaflux_fp8_gated_mlp_workspace_bytes": (_i64, [_i32, _i64, _i64, _i32]),
    "lunaflux_fp8_qkv_launch_geometry": (_i32, [_i32, _i64, _i64, _i64, _i32, _i32p,
                                                ctypes.c_char_p]),
    "lunaflux_fp8_qkv_w8a16_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32]),
    "lunaflux_fp8_rms_norm_quant_geometry": (_i32, [ctypes.c_float, _i64, _i32, _i32p,
                                                    ctypes.c_char_p]),
    "lunaflux_fp8_moe_descriptor": (_i32, [_i32, _i32, _i32, _i64, _i64, _i32, _vp]),
    "lunaflux_fp8_moe_workspace_bytes": (_i64, [_vp, _i32]),
    "lunaflux_fp8_moe_sync_offset": (_i64, [_vp, _i32]),
    "lunaflux_fp8_moe_workspace_layout": (_i32, [_vp, _i32, _i64p]),
    "lunaflux_fp8_moe_launch_geometry": (_i32, [_i32, _vp, _i32, _i32p, ctypes.c_char_p]),
}

MOE_ROUTE, MOE_SORT, MOE_QUANT_TOKENS, MOE_GATE_UP, MOE_QUANT_HIDDEN, MOE_DOWN, MOE_COMBINE = range(1, 8)
MOE_SORT_COUNT = 8


class NativeLibraryMissing(RuntimeError):
    pass


_LIB = None


def lib():
    """The loaded C-ABI library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIBRARY_PATH):
            raise NativeLibraryMissing(
                f"{LIBRARY_PATH} is missing: run `python -m lunaflux_amd.build` first")
        handle = ctypes.CDLL(LIBRARY_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = handle
    return _LIB


def code_object_bytes() -> bytes:
    if not os.path.exists(CODE_OBJECT_PATH):
        raise NativeLibraryMissing(
            f"{CODE_OBJECT_PATH} is missing: run `python -m lunaflux_amd.build` first")
    with open(CODE_OBJECT_PATH, "rb") as f:
        return f.read()

"""ctypes binding of the CPU oracle (oracle/liblf_oracle.so).

Test infrastructure: the oracle is the checker for the HIP path. Only tests,
``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg load it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB_PATH = os.path.join(ORACLE_DIR, "liblf_oracle.so")

OK, INVALID_LIMIT, LIMIT_EXCEEDED, INVALID_SHAPE, INVALID_SCALAR, OVERFLOW, NON_FINITE = range(7)
ROUTE_TOPK_SOFTMAX, ROUTE_SOFTMAX_TOPK = 0, 1

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class Limits(ctypes.Structure):
    _fields_ = [("max_rows", _i32), ("max_columns", _i32), ("max_elements", _i32)]


def _load():
    sources = [os.path.join(ORACLE_DIR, f) for f in ("lf_oracle.c", "lf_oracle.h")]
    if not os.path.exists(LIB_PATH) or any(
            os.path.getmtime(f) > os.path.getmtime(LIB_PATH) for f in sources if os.path.exists(f)):
        subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)
    lib = ctypes.CDLL(LIB_PATH)
    sig = {
        "lfo_limits_new": (_i32, [_i32, _i32, _i32, ctypes.POINTER(Limits)]),
        "lfo_checked_element_count": (_i32, [_i32, _i32, ctypes.POINTER(Limits), _i32p]),
        "lfo_decode_bfloat16_le": (_i32, [_u8p, _i64, _i32, _i32, ctypes.POINTER(Limits), _f32p]),
        "lfo_project_values": (_i32, [_f32p, _i32, _i32, _f32p, _i32, _i32, ctypes.POINTER(Limits), _f32p]),
        "lfo_dense_projection": (_i32, [_f32p, _i32, _i32, _f32p, _i32, _i32, ctypes.POINTER(Limits), _f32p]),
        "lfo_qkv_projection": (_i32, [_f32p, _i32, _i32, _f32p, _i32, _f32p, _i32, _f32p, _i32,
                                      ctypes.POINTER(Limits), _f32p]),
        "lfo_silu_gated_mlp": (_i32, [_f32p, _i32, _i32, _f32p, _f32p, _i32, _f32p, _i32,
                                      ctypes.POINTER(Limits), _f32p, _f32p]),
        "lfo_rms_norm": (_i32, [_f32p, _i32, _i32, _f32p, _i32, _i32, ctypes.c_float,
                                ctypes.POINTER(Limits), _f32p]),
        "lfo_silu_mul": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
        "lfo_silu_mul_array": (None, [_f32p, _f32p, _i64, _f32p]),
        "lfo_bf16_rne": (ctypes.c_uint16, [ctypes.c_float]),
        "lfo_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "lfo_bf16_round_array": (None, [_f32p, _i64, _u16p]),
        "lfo_bf16_decode_array": (None, [_u16p, _i64, _f32p]),
        "lfo_e4m3_decode": (ctypes.c_float, [ctypes.c_uint8]),
        "lfo_e4m3_encode": (ctypes.c_uint8, [ctypes.c_float]),
        "lfo_e4m3_encode_array": (None, [_f32p, _i64, _u8p]),
        "lfo_e4m3_decode_array": (None, [_u8p, _i64, _f32p]),
        "lfo_quantize_rows": (_i32, [_f32p, _i32, _i32, _i32, _u8p, _f32p]),
        "lfo_quantize_blocks": (_i32, [_f32p, _i32, _i32, _i32, _u8p, _f32p]),
        "lfo_dequantize": (_i32, [_u8p, _f32p, _i32, _i32, _i32, _i32, _f32p]),
        "lfo_route_topk": (_i32, [_f32p, _i32, _i32, _i32, _i32, _i32p, _f32p]),
        "lfo_moe_sort": (_i32, [_i32p, _i32, _i32, _i32, _i32p, _i32p]),
        "lfo_moe_mlp": (_i32, [_f32p, _i32, _i32, _f32p, _f32p, _f32p, _i32, _i32, _i32p, _f32p,
                               _i32, _i32, _i32, _f32p]),
        "lfo_project_values_mt": (_i32, [_f32p, _i32, _i32, _f32p, _i32, _i32, _f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


LIB = _load()


class OracleError(RuntimeError):
    def __init__(self, status: int):
        super().__init__(f"oracle status {status}")
        self.status = status


def _p(a: np.ndarray, ptype):
    return a.ctypes.data_as(ptype)


def _check(status: int):
    if status != OK:
        raise OracleError(status)


def limits(max_rows=1 << 30, max_columns=1 << 30, max_elements=2147483647):
    lim = Limits()
    _check(LIB.lfo_limits_new(max_rows, max_columns, max_elements, ctypes.byref(lim)))
    return lim


def _lim(lim):
    return ctypes.byref(lim) if lim is not None else None


def decode_bfloat16_le(data: bytes, rows: int, columns: int, lim=None) -> np.ndarray:
    buf = np.frombuffer(bytes(data), dtype=np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    out = np.zeros(max(rows * columns, 1), np.float32)
    _check(LIB.lfo_decode_bfloat16_le(_p(buf, _u8p), len(data), rows, columns, _lim(lim), _p(out, _f32p)))
    return out[: rows * columns].reshape(rows, columns)


def project_values(x: np.ndarray, w: np.ndarray, lim=None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros((x.shape[0], w.shape[0]), np.float32)
    _check(LIB.lfo_project_values(_p(x, _f32p), x.shape[0], x.shape[1], _p(w, _f32p), w.shape[0],
                                  w.shape[1], _lim(lim), _p(out, _f32p)))
    return out


dense_projection = project_values


def project_values_mt(x: np.ndarray, w: np.ndarray, threads: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    assert x.shape[1] == w.shape[1]
    out = np.zeros((x.shape[0], w.shape[0]), np.float32)
    _check(LIB.lfo_project_values_mt(_p(x, _f32p), x.shape[0], x.shape[1], _p(w, _f32p), w.shape[0],
                                     threads, _p(out, _f32p)))
    return out


def qkv_projection(x, wq, wk, wv, lim=None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    wq, wk, wv = (np.ascontiguousarray(a, np.float32) for a in (wq, wk, wv))
    for wt in (wq, wk, wv):
        if wt.shape[1] != x.shape[1]:
            raise OracleError(INVALID_SHAPE)
    out = np.zeros((x.shape[0], wq.shape[0] + wk.shape[0] + wv.shape[0]), np.float32)
    _check(LIB.lfo_qkv_projection(_p(x, _f32p), x.shape[0], x.shape[1], _p(wq, _f32p), wq.shape[0],
                                  _p(wk, _f32p), wk.shape[0], _p(wv, _f32p), wv.shape[0], _lim(lim),
                                  _p(out, _f32p)))
    return out


def silu_gated_mlp(x, wg, wu, wd, round_hidden_bf16=False, lim=None, return_hidden=False):
    x = np.ascontiguousarray(x, np.float32)
    wg, wu, wd = (np.ascontiguousarray(a, np.float32) for a in (wg, wu, wd))
    inter = wg.shape[0]
    assert wg.shape[1] == x.shape[1] and wu.shape == wg.shape and wd.shape == (x.shape[1], inter)
    hidden = np.zeros((x.shape[0], inter), np.float32)
    out = np.zeros((x.shape[0], x.shape[1]), np.float32)
    _check(LIB.lfo_silu_gated_mlp(_p(x, _f32p), x.shape[0], x.shape[1], _p(wg, _f32p), _p(wu, _f32p),
                                  inter, _p(wd, _f32p), int(bool(round_hidden_bf16)), _lim(lim),
                                  _p(hidden, _f32p), _p(out, _f32p)))
    return (out, hidden) if return_hidden else out


def rms_norm(x: np.ndarray, w: np.ndarray, epsilon: float, lim=None) -> np.ndarray:
    """x [rows, K] fp32, w the norm weight ([K] or [1, K]) -> fp32 [rows, K]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    w2 = w.reshape(1, -1) if w.ndim == 1 else w
    out = np.empty_like(x)
    _check(LIB.lfo_rms_norm(_p(x, _f32p), x.shape[0], x.shape[1], _p(w2, _f32p), w2.shape[0],
                            w2.shape[1], float(np.float32(epsilon)), _lim(lim), _p(out, _f32p)))
    return out


def silu_mul(g: float, u: float) -> float:
    return LIB.lfo_silu_mul(g, u)


def silu_mul_array(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    assert g.shape == u.shape
    out = np.zeros(g.shape, np.float32)
    LIB.lfo_silu_mul_array(_p(g, _f32p), _p(u, _f32p), g.size, _p(out, _f32p))
    return out


def bf16_round(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits (uint16), round to nearest even."""
    a = np.ascontiguousarray(a, np.float32)
    out = np.zeros(a.shape, np.uint16)
    LIB.lfo_bf16_round_array(_p(a, _f32p), a.size, _p(out, _u16p))
    return out


def bf16_decode(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, np.uint16)
    out = np.zeros(bits.shape, np.float32)
    LIB.lfo_bf16_decode_array(_p(bits, _u16p), bits.size, _p(out, _f32p))
    return out


def e4m3_encode(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    out = np.zeros(a.shape, np.uint8)
    LIB.lfo_e4m3_encode_array(_p(a, _f32p), a.size, _p(out, _u8p))
    return out


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.uint8)
    out = np.zeros(codes.shape, np.float32)
    LIB.lfo_e4m3_decode_array(_p(codes, _u8p), codes.size, _p(out, _f32p))
    return out


def quantize_rows(x: np.ndarray, group: int | None = None):
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    group = cols if group is None else group
    q = np.zeros((rows, cols), np.uint8)
    s = np.zeros((rows, cols // group), np.float32)
    _check(LIB.lfo_quantize_rows(_p(x, _f32p), rows, cols, group, _p(q, _u8p), _p(s, _f32p)))
    return q, (s[:, 0].copy() if group == cols else s)


def quantize_blocks(w: np.ndarray, block: int = 128):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    q = np.zeros((rows, cols), np.uint8)
    s = np.zeros(((rows + block - 1) // block, (cols + block - 1) // block), np.float32)
    _check(LIB.lfo_quantize_blocks(_p(w, _f32p), rows, cols, block, _p(q, _u8p), _p(s, _f32p)))
    return q, s


def dequantize(q: np.ndarray, s: np.ndarray, mode: int = 0, group: int = 0) -> np.ndarray:
    """mode 0: per-row scales; 1: per-row-per-group; 2: group x group blocks."""
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.float32)
    out = np.zeros(q.shape, np.float32)
    _check(LIB.lfo_dequantize(_p(q, _u8p), _p(s, _f32p), q.shape[0], q.shape[1], mode, group,
                              _p(out, _f32p)))
    return out


def route_topk(logits: np.ndarray, k: int, mode: int):
    logits = np.ascontiguousarray(logits, np.float32)
    t, e = logits.shape
    ex = np.zeros((t, k), np.int32)
    w = np.zeros((t, k), np.float32)
    _check(LIB.lfo_route_topk(_p(logits, _f32p), t, e, k, mode, _p(ex, _i32p), _p(w, _f32p)))
    return ex, w


def moe_sort(topk_experts: np.ndarray, experts: int):
    te = np.ascontiguousarray(topk_experts, np.int32)
    t, k = te.shape
    sorted_a = np.zeros(t * k, np.int32)
    offsets = np.zeros(experts + 1, np.int32)
    _check(LIB.lfo_moe_sort(_p(te, _i32p), t, k, experts, _p(sorted_a, _i32p), _p(offsets, _i32p)))
    return sorted_a, offsets


def moe_mlp(x, wg, wu, wd, topk_experts, topk_weights, hidden_transform=0, threads=8):
    x = np.ascontiguousarray(x, np.float32)
    wg, wu, wd = (np.ascontiguousarray(a, np.float32) for a in (wg, wu, wd))
    te = np.ascontiguousarray(topk_experts, np.int32)
    tw = np.ascontiguousarray(topk_weights, np.float32)
    e, inter, hidden = wg.shape
    t, k = te.shape
    out = np.zeros((t, hidden), np.float32)
    _check(LIB.lfo_moe_mlp(_p(x, _f32p), t, hidden, _p(wg, _f32p), _p(wu, _f32p), _p(wd, _f32p), e,
                           inter, _p(te, _i32p), _p(tw, _f32p), k, hidden_transform, threads,
                           _p(out, _f32p)))
    return out

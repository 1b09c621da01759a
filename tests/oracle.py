"""ctypes binding of oracle/liboracle.so — the CPU checker (test infrastructure).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product path never does.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_double, c_float, c_int, c_int64, c_uint64, c_void_p
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = ROOT / "oracle" / "liboracle.so"

_lib = None
_F = POINTER(c_float)

_SIGS = {
    "orc_set_threads": (None, [c_int]),
    "orc_get_threads": (c_int, []),
    "orc_stream_key": (c_uint64, [c_uint64, c_uint64]),
    "orc_fill_uniform": (None, [_F, c_int64, c_uint64, c_uint64, c_float, c_float]),
    "orc_fill_normal": (None, [_F, c_int64, c_uint64, c_uint64, c_float, c_float]),
    "orc_fill_uniform_mt": (None, [_F, c_int64, c_uint64, c_uint64, c_float, c_float]),
    "orc_fill_normal_mt": (None, [_F, c_int64, c_uint64, c_uint64, c_float, c_float]),
    "orc_map_scale_add": (None, [_F, _F, _F, c_int64, c_float]),
    "orc_map_scale_add_mt": (None, [_F, _F, _F, c_int64, c_float]),
    "orc_block_reduce": (c_float, [_F, c_int, c_int]),
    "orc_reduce": (c_float, [_F, c_int, c_int]),
    "orc_sum_f64": (c_double, [_F, c_int64]),
    "orc_sum_abs_f64": (c_double, [_F, c_int64]),
    "orc_softmax_rows": (None, [_F, _F, c_int, c_int]),
    "orc_layer_norm_rows": (None, [_F, _F, _F, _F, c_int, c_int, c_float]),
    "orc_rms_norm_rows": (None, [_F, _F, _F, c_int, c_int, c_float]),
    "orc_mat_mul_rows": (None, [_F, _F, _F, _F, POINTER(c_double), c_int, c_int, c_int, POINTER(c_int), c_int,
                                c_int, c_int]),
    "orc_gemv": (None, [_F, _F, _F, c_int, c_int]),
    "orc_round_bf16": (None, [_F, _F, c_void_p, c_int64]),
    "orc_attention_explicit": (None, [_F, _F, _F, _F, POINTER(c_double), c_int, c_int, c_int, c_int, c_int, c_int,
                                      POINTER(c_int), c_int]),
    "orc_attention_decode": (None, [_F, _F, _F, _F, c_int, c_int, c_int, c_int, c_int]),
}


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m opworks_amd.build oracle`")
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def declare(name, restype, argtypes):
    _SIGS[name] = (restype, argtypes)
    if _lib is not None:
        fn = getattr(_lib, name)
        fn.restype, fn.argtypes = restype, argtypes


def fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_F)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


def fill_uniform(n: int, seed: int, stream: int, lo: float, hi: float, mt: bool = False) -> np.ndarray:
    out = np.empty(n, np.float32)
    (lib().orc_fill_uniform_mt if mt else lib().orc_fill_uniform)(fp(out), n, seed, stream, lo, hi)
    return out


def fill_normal(n: int, seed: int, stream: int, mean: float, sd: float, mt: bool = False) -> np.ndarray:
    out = np.empty(n, np.float32)
    (lib().orc_fill_normal_mt if mt else lib().orc_fill_normal)(fp(out), n, seed, stream, mean, sd)
    return out


def map_scale_add(a, b, alpha: float, mt: bool = False) -> np.ndarray:
    a, b = f32(a), f32(b)
    out = np.empty_like(a)
    (lib().orc_map_scale_add_mt if mt else lib().orc_map_scale_add)(fp(a), fp(b), fp(out), a.size, alpha)
    return out


REDUCE_OPS = {"sum": 0, "max": 1, "product": 2}


def block_reduce(vals, op: str = "sum") -> float:
    v = f32(vals)
    return lib().orc_block_reduce(fp(v), v.size, REDUCE_OPS[op])


def reduce(x, op: str = "sum") -> float:
    x = f32(x)
    return lib().orc_reduce(fp(x), x.size, REDUCE_OPS[op])


def sum_f64(x) -> float:
    x = f32(x)
    return lib().orc_sum_f64(fp(x), x.size)


def sum_abs_f64(x) -> float:
    x = f32(x)
    return lib().orc_sum_abs_f64(fp(x), x.size)


def softmax_rows(x, rows: int, cols: int) -> np.ndarray:
    x = f32(x)
    out = np.empty(rows * cols, np.float32)
    lib().orc_softmax_rows(fp(x), fp(out), rows, cols)
    return out


def layer_norm_rows(x, gamma, beta, rows: int, cols: int, eps: float) -> np.ndarray:
    x, g, b = f32(x), f32(gamma), f32(beta)
    out = np.empty(rows * cols, np.float32)
    lib().orc_layer_norm_rows(fp(x), fp(out), fp(g), fp(b), rows, cols, eps)
    return out


def rms_norm_rows(x, w, rows: int, cols: int, eps: float) -> np.ndarray:
    x, w = f32(x), f32(w)
    out = np.empty(rows * cols, np.float32)
    lib().orc_rms_norm_rows(fp(x), fp(w), fp(out), rows, cols, eps)
    return out


ACTS = {"none": 0, "relu": 1, "gelu": 2}


def mat_mul_rows(A, B, M, N, K, rows=None, bias=None, b_transposed=False, act="none"):
    """Reference names: A is M x N, B is N x K (K x N when b_transposed).
    Returns (out[len(rows) or M, K], absdot float64 of the same shape)."""
    A, B = f32(A), f32(B)
    nrows = M if rows is None else len(rows)
    out = np.empty(nrows * K, np.float32)
    absdot = np.empty(nrows * K, np.float64)
    rp = None
    if rows is not None:
        rows = np.ascontiguousarray(rows, np.int32)
        rp = rows.ctypes.data_as(POINTER(c_int))
    bp = fp(f32(bias)) if bias is not None else None
    lib().orc_mat_mul_rows(fp(A), fp(B), bp, fp(out), absdot.ctypes.data_as(POINTER(c_double)), M, N, K, rp,
                           nrows, int(b_transposed), ACTS[act])
    return out.reshape(nrows, K), absdot.reshape(nrows, K)


def gemv(x, W, in_features, out_features):
    x, W = f32(x), f32(W)
    y = np.empty(out_features, np.float32)
    lib().orc_gemv(fp(x), fp(W), fp(y), in_features, out_features)
    return y


def round_bf16(x):
    """Returns (rounded float32 array, uint16 bf16 bits)."""
    x = f32(x)
    out = np.empty_like(x)
    bits = np.empty(x.size, np.uint16)
    lib().orc_round_bf16(fp(x), fp(out), bits.ctypes.data, x.size)
    return out, bits


def attention_explicit(q, k, v, T, S, qh, kv_rep, D, cap, rows=None):
    """Returns (out [qh][nrows][D], bound float64 of the same shape)."""
    q, k, v = f32(q), f32(k), f32(v)
    nrows = T if rows is None else len(rows)
    out = np.empty(qh * nrows * D, np.float32)
    bound = np.empty(qh * nrows * D, np.float64)
    rp = None
    if rows is not None:
        rows = np.ascontiguousarray(rows, np.int32)
        rp = rows.ctypes.data_as(POINTER(c_int))
    lib().orc_attention_explicit(fp(q), fp(k), fp(v), fp(out), bound.ctypes.data_as(POINTER(c_double)), T, S, qh,
                                 kv_rep, D, cap, rp, nrows)
    return out.reshape(qh, nrows, D), bound.reshape(qh, nrows, D)


def attention_decode(q, k, v, qh, kv_rep, D, length, max_seq):
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty(qh * D, np.float32)
    lib().orc_attention_decode(fp(q), fp(k), fp(v), fp(out), qh, kv_rep, D, length, max_seq)
    return out.reshape(qh, D)

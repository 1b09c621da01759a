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
    "orc_linear": (None, [_F, _F, _F, c_int, c_int, c_int]),
    "orc_linear_exact": (None, [_F, _F, _F, c_int, c_int, c_int]),
    "orc_rope_inv_freq": (None, [c_int, c_float, c_int, c_float, c_float, c_float, c_int, _F]),
    "orc_rope": (None, [_F, _F, c_int, c_int, c_int, c_int]),
    "orc_argmax": (c_int, [_F, c_int]),
    "orc_swiglu": (None, [_F, _F, _F, ctypes.c_int64]),
    "orc_llama_set_bf16": (None, [c_void_p]),
    "orc_causal_scale": (None, [_F, c_int, c_int, ctypes.c_float]),
    "orc_llama_create": (c_void_p, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_float, c_int,
                                    c_float, c_float, c_float, c_int, c_uint64, c_float, c_int]),
    "orc_llama_destroy": (None, [c_void_p]),
    "orc_llama_weight": (c_void_p, [c_void_p, c_int, c_int]),
    "orc_llama_reset": (None, [c_void_p, c_int]),
    "orc_llama_prefill": (c_int, [c_void_p, POINTER(c_int), c_int, _F, _F]),
    "orc_llama_decode": (c_int, [c_void_p, c_int, _F]),
    "orc_scan": (None, [_F, _F, POINTER(c_double), c_int64, c_int, c_int]),
    "orc_transpose": (None, [_F, _F, c_int, c_int]),
    "orc_gather": (None, [_F, c_int64, POINTER(c_int), _F, c_int64]),
    "orc_scatter": (None, [_F, POINTER(c_int), _F, c_int64, c_int64]),
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


def linear(X, W, rows, in_f, out_f):
    X, W = f32(X), f32(W)
    Y = np.empty(rows * out_f, np.float32)
    lib().orc_linear(fp(X), fp(W), fp(Y), rows, in_f, out_f)
    return Y.reshape(rows, out_f)


def linear_exact(X, W, rows, in_f, out_f):
    X, W = f32(X), f32(W)
    Y = np.empty(rows * out_f, np.float32)
    lib().orc_linear_exact(fp(X), fp(W), fp(Y), rows, in_f, out_f)
    return Y.reshape(rows, out_f)


def rope_inv_freq(head_dim, theta, llama3=False, factor=0.0, low=0.0, high=0.0, orig=0):
    out = np.empty(head_dim // 2, np.float32)
    lib().orc_rope_inv_freq(head_dim, theta, int(llama3), factor, low, high, orig, fp(out))
    return out


def rope(x, inv_freq, rows, heads, head_dim, pos_start):
    x = f32(x).copy()
    lib().orc_rope(fp(x), fp(f32(inv_freq)), rows, heads, head_dim, pos_start)
    return x


def argmax(x):
    x = f32(x)
    return lib().orc_argmax(fp(x), x.size)


def _ip(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(POINTER(c_int))


def scan(x, maximum=False, inclusive=True):
    """Returns (out, abs_prefix): the exact prefix sum (or running fmaxf) and the
    float64 running sum of |x| over the same range."""
    x = f32(x)
    out = np.empty_like(x)
    absp = np.empty(x.size, np.float64)
    lib().orc_scan(fp(x), fp(out), absp.ctypes.data_as(POINTER(c_double)), x.size, int(maximum), int(inclusive))
    return out, absp


def transpose(x, rows, cols):
    x = f32(x)
    out = np.empty(rows * cols, np.float32)
    lib().orc_transpose(fp(x), fp(out), rows, cols)
    return out


def gather(x, idx):
    x, idx = f32(x), np.ascontiguousarray(idx, np.int32)
    out = np.empty(idx.size, np.float32)
    lib().orc_gather(fp(x), x.size, _ip(idx), fp(out), idx.size)
    return out


def scatter(x, idx, out):
    x, idx, out = f32(x), np.ascontiguousarray(idx, np.int32), f32(out).copy()
    lib().orc_scatter(fp(x), _ip(idx), fp(out), out.size, idx.size)
    return out


class Llama:
    """The oracle's Llama forward on seeded weights (one session)."""

    def __init__(self, cfg: dict, seed: int, sd: float = 0.02, norm_init: str = "ones", bf16: bool = False) -> None:
        rs = cfg.get("rope_scaling") or {}
        self.cfg = cfg
        self.V = cfg["vocab_size"]
        self.L = cfg["num_hidden_layers"]
        self.H = cfg["hidden_size"]
        self.h = lib().orc_llama_create(
            self.L, self.H, cfg["intermediate_size"], cfg["num_attention_heads"], cfg["num_key_value_heads"],
            cfg.get("head_dim", self.H // cfg["num_attention_heads"]), self.V, cfg["rms_norm_eps"], cfg["rope_theta"],
            int(bool(rs)), rs.get("factor", 0.0), rs.get("low_freq_factor", 0.0), rs.get("high_freq_factor", 0.0),
            rs.get("original_max_position_embeddings", 0), seed, sd, 1 if norm_init == "uniform" else 0)
        if bf16 or cfg.get("torch_dtype") == "bfloat16":
            lib().orc_llama_set_bf16(self.h)

    def weight(self, kind: int, layer: int, numel: int) -> np.ndarray:
        p = lib().orc_llama_weight(self.h, kind, layer)
        return np.ctypeslib.as_array(ctypes.cast(p, POINTER(c_float)), shape=(numel,)).copy()

    def reset(self, cap: int) -> None:
        lib().orc_llama_reset(self.h, cap)

    def prefill(self, ids, capture: bool = False):
        ids = np.ascontiguousarray(ids, np.int32)
        logits = np.empty(self.V, np.float32)
        caps = np.empty((self.L + 1) * ids.size * self.H, np.float32) if capture else None
        tok = lib().orc_llama_prefill(self.h, ids.ctypes.data_as(POINTER(c_int)), ids.size, fp(logits),
                                      fp(caps) if capture else None)
        if capture:
            return tok, logits, caps.reshape(self.L + 1, ids.size, self.H)
        return tok, logits

    def decode(self, token: int):
        logits = np.empty(self.V, np.float32)
        tok = lib().orc_llama_decode(self.h, token, fp(logits))
        return tok, logits

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.orc_llama_destroy(self.h)
            self.h = None


def swiglu(gate, up) -> np.ndarray:
    g, u = f32(gate), f32(up)
    out = np.empty_like(g)
    lib().orc_swiglu(fp(g), fp(u), fp(out), g.size)
    return out


def causal_scale(scores, rows: int, cols: int, scale: float) -> np.ndarray:
    s = f32(scores).copy()
    lib().orc_causal_scale(fp(s), rows, cols, scale)
    return s

"""Python host binding of libopworks_amd.so (the C ABI declared in include/*.h).

This is the ctypes side a reference user would bind (the reference drives its
C ABI the same way, examples/llama/generate.py:23-61). Device memory, streams
and events come from the library itself, so no other GPU runtime is loaded.
The native library is mandatory: every entry point raises if it is missing.

Errors: an entry point returning -1 raises OpworksError (a ValueError, the
Python face of the reference's std::invalid_argument) carrying the library's
message.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint64, c_void_p
from pathlib import Path
from typing import Optional, Union

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "lib" / "libopworks_amd.so"

__all__ = [
    "OpworksError", "lib", "DeviceBuffer", "DeviceView", "Stream", "Event", "Graph", "ops", "fill_uniform", "fill_normal",
    "device_name", "device_count", "synchronize", "cu_count",
]


class OpworksError(ValueError):
    """A contract violation reported by the native library."""


_lib: Optional[ctypes.CDLL] = None

# name -> (restype, argtypes)
_SIGNATURES = {
    "opw_last_error": (c_char_p, []),
    "opw_device_count": (c_int, [POINTER(c_int)]),
    "opw_set_device": (c_int, [c_int]),
    "opw_device_name": (c_int, [c_char_p, c_int]),
    "opw_device_cu_count": (c_int, [POINTER(c_int)]),
    "opw_malloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "opw_free": (c_int, [c_void_p]),
    "opw_memcpy_htod": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "opw_memcpy_dtoh": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "opw_memcpy_dtod": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "opw_memset": (c_int, [c_void_p, c_int, c_size_t, c_void_p]),
    "opw_stream_create": (c_int, [POINTER(c_void_p)]),
    "opw_stream_destroy": (c_int, [c_void_p]),
    "opw_stream_synchronize": (c_int, [c_void_p]),
    "opw_device_synchronize": (c_int, []),
    "opw_event_create": (c_int, [POINTER(c_void_p)]),
    "opw_event_destroy": (c_int, [c_void_p]),
    "opw_event_record": (c_int, [c_void_p, c_void_p]),
    "opw_event_synchronize": (c_int, [c_void_p]),
    "opw_event_elapsed_ms": (c_int, [c_void_p, c_void_p, POINTER(c_float)]),
    "opw_graph_capture_begin": (c_int, [c_void_p]),
    "opw_graph_capture_end": (c_int, [c_void_p, POINTER(c_void_p)]),
    "opw_graph_launch": (c_int, [c_void_p, c_void_p]),
    "opw_graph_destroy": (c_int, [c_void_p]),
    "opw_fill_uniform_f32": (c_int, [c_void_p, c_int64, c_uint64, c_uint64, c_float, c_float, c_void_p]),
    "opw_fill_normal_f32": (c_int, [c_void_p, c_int64, c_uint64, c_uint64, c_float, c_float, c_void_p]),
    "opw_map_scale_add_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_float, c_void_p]),
    "opw_map_add_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "opw_map_scale_f32": (c_int, [c_void_p, c_void_p, c_int, c_float, c_void_p]),
    "opw_map_relu_f32": (c_int, [c_void_p, c_void_p, c_int, c_void_p]),
    "opw_reduction_workspace_size": (c_int, [c_int]),
    "opw_reduce_f32_noalloc": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "opw_reduce_f32": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_int, c_void_p]),
    "opw_softmax_f32": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "opw_layer_norm_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_float, c_void_p]),
    "opw_rms_norm_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_float, c_void_p]),
    "opw_mat_mul_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "opw_mat_mul_fused_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                      c_void_p]),
    "opw_linear_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "opw_mat_mul_fused_ex_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                         c_int, c_void_p]),
    "opw_linear_wbf16": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "opw_linear_bf16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "opw_linear_bf16_bf16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "opw_convert_f32_to_bf16": (c_int, [c_void_p, c_void_p, c_int64, c_void_p]),
    "opw_attention_prefill_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                          c_int, c_int, c_void_p]),
    "opw_attention_prefill_workspace_size": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                                     ctypes.POINTER(c_int64), ctypes.POINTER(c_int64)]),
    "opw_attention_prefill_ws_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                             c_int, c_int, c_int, c_void_p, c_int64, c_void_p, c_int64, c_int,
                                             c_void_p]),
    "opw_attention_decode_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                         c_void_p]),
    "opw_attention_decode_workspace_size": (c_int, [c_int, c_int, c_int]),
    "opw_attention_decode_counters_size": (c_int, [c_int, c_int]),
    "opw_attention_decode_fused_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                               c_int, c_void_p, c_int, c_void_p, c_int, c_void_p]),
    "opw_attention_decode_ws_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                            c_void_p, c_int, c_void_p]),
    "opw_add_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "opw_swiglu_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "opw_causal_scale_f32": (c_int, [c_void_p, c_int, c_int, c_float, c_void_p]),
    "opw_embedding_f32": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "opw_embedding_bf16": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "opw_split_heads_f32": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "opw_merge_heads_f32": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "opw_rope_f32": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "opw_argmax_f32": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "opw_scan_workspace_size": (c_int, [c_int]),
    "opw_scan_f32": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_int, c_void_p]),
    "opw_transpose_f32": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "opw_copy_f32": (c_int, [c_void_p, c_void_p, c_int, c_void_p]),
    "opw_gather_f32": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int, c_void_p]),
    "opw_scatter_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p]),
}


def lib() -> ctypes.CDLL:
    """Loads libopworks_amd.so (once) and declares the ABI signatures."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m opworks_amd.build` first")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def declare(name: str, restype, argtypes) -> None:
    """Registers the signature of an additional ABI symbol (used by submodules)."""
    _SIGNATURES[name] = (restype, argtypes)
    if _lib is not None:
        fn = getattr(_lib, name)
        fn.restype = restype
        fn.argtypes = argtypes


def last_error() -> str:
    msg = lib().opw_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> int:
    if rc < 0:
        raise OpworksError(last_error())
    return rc


# ------------------------------------------------------------------ plumbing
def device_count() -> int:
    n = c_int(0)
    check(lib().opw_device_count(ctypes.byref(n)))
    return n.value


def device_name() -> str:
    buf = ctypes.create_string_buffer(256)
    check(lib().opw_device_name(buf, 256))
    return buf.value.decode()


def cu_count() -> int:
    n = c_int(0)
    check(lib().opw_device_cu_count(ctypes.byref(n)))
    return n.value


def synchronize(stream: "Optional[Stream]" = None) -> None:
    check(lib().opw_stream_synchronize(_stream(stream)))


class Stream:
    """A non-blocking HIP stream owned by the library."""

    def __init__(self) -> None:
        h = c_void_p()
        check(lib().opw_stream_create(ctypes.byref(h)))
        self.handle = h.value

    def synchronize(self) -> None:
        check(lib().opw_stream_synchronize(self.handle))

    def __del__(self) -> None:
        if getattr(self, "handle", None) and _lib is not None:
            _lib.opw_stream_destroy(self.handle)
            self.handle = None


class Event:
    def __init__(self) -> None:
        h = c_void_p()
        check(lib().opw_event_create(ctypes.byref(h)))
        self.handle = h.value

    def record(self, stream: "Optional[Stream]" = None) -> "Event":
        check(lib().opw_event_record(self.handle, _stream(stream)))
        return self

    def synchronize(self) -> None:
        check(lib().opw_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float(0)
        check(lib().opw_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)))
        return ms.value

    def __del__(self) -> None:
        if getattr(self, "handle", None) and _lib is not None:
            _lib.opw_event_destroy(self.handle)
            self.handle = None


class Graph:
    """A HIP graph captured from the library calls enqueued on one Stream:

        g = Graph.capture(stream, lambda: ops.attention_decode(..., stream=stream))
        g.launch(stream)

    Capture runs in global mode, so a call that allocates or synchronizes while it is open
    makes capture fail with OpworksError."""

    def __init__(self, handle: int) -> None:
        self.handle = handle

    @classmethod
    def capture(cls, stream: "Stream", body) -> "Graph":
        check(lib().opw_graph_capture_begin(stream.handle))
        try:
            body()
        finally:
            h = c_void_p()
            rc = lib().opw_graph_capture_end(stream.handle, ctypes.byref(h))
        check(rc)
        return cls(h.value)

    def launch(self, stream: "Stream") -> None:
        check(lib().opw_graph_launch(self.handle, stream.handle))

    def __del__(self) -> None:
        if getattr(self, "handle", None) and _lib is not None:
            _lib.opw_graph_destroy(self.handle)
            self.handle = None


def _stream(s) -> Optional[int]:
    if s is None:
        return None
    if isinstance(s, Stream):
        return s.handle
    return int(s)


class DeviceView:
    """A non-owning typed pointer into device memory."""

    def __init__(self, ptr: int, n: int, dtype=np.float32, owner=None) -> None:
        self.ptr = ptr
        self.n = n
        self.dtype = np.dtype(dtype)
        self._owner = owner

    @property
    def nbytes(self) -> int:
        return self.n * self.dtype.itemsize

    def offset(self, elems: int, n: Optional[int] = None) -> "DeviceView":
        rest = self.n - elems if n is None else n
        return DeviceView(self.ptr + elems * self.dtype.itemsize, rest, self.dtype, self)

    def to_host(self, stream=None) -> np.ndarray:
        out = np.empty(self.n, dtype=self.dtype)
        if self.n:
            check(lib().opw_memcpy_dtoh(out.ctypes.data, self.ptr, self.nbytes, _stream(stream)))
        return out

    def copy_from_host(self, arr: np.ndarray, stream=None) -> None:
        arr = np.ascontiguousarray(arr, dtype=self.dtype).reshape(-1)
        if arr.size > self.n:
            raise OpworksError("host array larger than the device view")
        if arr.size:
            check(lib().opw_memcpy_htod(self.ptr, arr.ctypes.data, arr.nbytes, _stream(stream)))

    def fill_bytes(self, value: int = 0, stream=None) -> None:
        check(lib().opw_memset(self.ptr, value, self.nbytes, _stream(stream)))


class DeviceBuffer(DeviceView):
    """Owning device allocation (the reference's DeviceBuffer / TypedDeviceBuffer).

    Freeing waits for the device (as the reference's cudaFree-based destructor
    does), but a buffer must still be alive when work that uses it is
    enqueued: keep a reference, do not pass `DeviceBuffer(...).ptr` of a
    temporary to an entry point."""

    def __init__(self, n: int, dtype=np.float32) -> None:
        if n < 0:
            raise OpworksError("size must be nonnegative")
        p = c_void_p()
        check(lib().opw_malloc(ctypes.byref(p), int(n) * np.dtype(dtype).itemsize))
        super().__init__(p.value or 0, int(n), dtype)

    @classmethod
    def empty(cls, n: int, dtype=np.float32) -> "DeviceBuffer":
        return cls(n, dtype)

    @classmethod
    def from_host(cls, arr: np.ndarray, dtype=None, stream=None) -> "DeviceBuffer":
        arr = np.asarray(arr)
        buf = cls(arr.size, dtype or arr.dtype)
        buf.copy_from_host(arr, stream)
        return buf

    def free(self) -> None:
        if self.ptr and _lib is not None:
            _lib.opw_free(self.ptr)
        self.ptr = 0

    def __del__(self) -> None:
        try:
            self.free()
        except Exception:
            pass


Ptr = Union[DeviceView, int, None]


def _p(x: Ptr) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, DeviceView):
        return x.ptr or None
    return int(x) or None


def fill_uniform(buf: DeviceView, seed: int, stream_id: int, lo: float, hi: float, n: Optional[int] = None,
                 stream=None) -> None:
    check(lib().opw_fill_uniform_f32(_p(buf), buf.n if n is None else n, seed, stream_id, lo, hi, _stream(stream)))


def fill_normal(buf: DeviceView, seed: int, stream_id: int, mean: float, stddev: float, n: Optional[int] = None,
                stream=None) -> None:
    check(lib().opw_fill_normal_f32(_p(buf), buf.n if n is None else n, seed, stream_id, mean, stddev,
                                    _stream(stream)))


class _Ops:
    """Mirrors the reference's opworks::ops entry points on the C ABI."""

    REDUCE_OPS = {"sum": 0, "max": 1, "product": 2}

    def map_scale_add(self, a: Ptr, b: Ptr, out: Ptr, n: int, alpha: float, stream=None) -> None:
        check(lib().opw_map_scale_add_f32(_p(a), _p(b), _p(out), n, alpha, _stream(stream)))

    def map_add(self, a: Ptr, b: Ptr, out: Ptr, n: int, stream=None) -> None:
        check(lib().opw_map_add_f32(_p(a), _p(b), _p(out), n, _stream(stream)))

    def map_scale(self, x: Ptr, out: Ptr, n: int, factor: float, stream=None) -> None:
        check(lib().opw_map_scale_f32(_p(x), _p(out), n, factor, _stream(stream)))

    def map_relu(self, x: Ptr, out: Ptr, n: int, stream=None) -> None:
        check(lib().opw_map_relu_f32(_p(x), _p(out), n, _stream(stream)))

    def reduction_workspace_size(self, n: int) -> int:
        return check(lib().opw_reduction_workspace_size(n))

    def reduce(self, x: Ptr, out: Ptr, n: int, op: str = "sum", workspace: Ptr = None, workspace_size: int = 0,
               stream=None) -> None:
        if isinstance(workspace, DeviceView) and workspace_size == 0:
            workspace_size = workspace.n
        check(lib().opw_reduce_f32(_p(x), _p(out), n, self.REDUCE_OPS[op], _p(workspace), workspace_size,
                                   _stream(stream)))

    def softmax(self, x: Ptr, out: Ptr, rows: int, cols: int, stream=None) -> None:
        check(lib().opw_softmax_f32(_p(x), _p(out), rows, cols, _stream(stream)))

    def layer_norm(self, x: Ptr, out: Ptr, gamma: Ptr, beta: Ptr, rows: int, cols: int, eps: float = 1e-5,
                   stream=None) -> None:
        check(lib().opw_layer_norm_f32(_p(x), _p(out), _p(gamma), _p(beta), rows, cols, eps, _stream(stream)))

    def rms_norm(self, x: Ptr, weight: Ptr, out: Ptr, rows: int, cols: int, eps: float, stream=None) -> None:
        check(lib().opw_rms_norm_f32(_p(x), _p(weight), _p(out), rows, cols, eps, _stream(stream)))

    ACTIVATIONS = {"none": 0, "relu": 1, "gelu": 2}

    # Reference names: A is M x N, B is N x K (K x N when b_transposed), C is M x K.
    def mat_mul(self, A: Ptr, B: Ptr, C: Ptr, M: int, N: int, K: int, stream=None) -> None:
        check(lib().opw_mat_mul_f32(_p(A), _p(B), _p(C), M, N, K, _stream(stream)))

    def mat_mul_fused(self, A: Ptr, B: Ptr, bias: Ptr, C: Ptr, M: int, N: int, K: int, b_transposed: bool = False,
                      activation: str = "none", stream=None) -> None:
        check(lib().opw_mat_mul_fused_f32(_p(A), _p(B), _p(bias), _p(C), M, N, K, int(b_transposed),
                                          self.ACTIVATIONS[activation], _stream(stream)))

    def mat_mul_fused_ex(self, A: Ptr, B: Ptr, bias: Ptr, C: Ptr, M: int, N: int, K: int, a_transposed: bool,
                         b_transposed: bool, activation: str = "none", stream=None) -> None:
        check(lib().opw_mat_mul_fused_ex_f32(_p(A), _p(B), _p(bias), _p(C), M, N, K, int(a_transposed),
                                             int(b_transposed), self.ACTIVATIONS[activation], _stream(stream)))

    def linear(self, X: Ptr, W: Ptr, Y: Ptr, rows: int, in_features: int, out_features: int, stream=None) -> None:
        check(lib().opw_linear_f32(_p(X), _p(W), _p(Y), rows, in_features, out_features, _stream(stream)))

    # ops::linear<bf16>: fp32 X against bf16 weights (uint16 bits) widened exactly, fp32 accumulation.
    def linear_wbf16(self, X: Ptr, W: Ptr, Y: Ptr, rows: int, in_features: int, out_features: int,
                     stream=None) -> None:
        check(lib().opw_linear_wbf16(_p(X), _p(W), _p(Y), rows, in_features, out_features, _stream(stream)))

    def linear_bf16(self, X: Ptr, W: Ptr, bias: Ptr, Y: Ptr, rows: int, in_features: int, out_features: int,
                    activation: str = "none", x_bf16: bool = False, stream=None) -> None:
        fn = lib().opw_linear_bf16_bf16 if x_bf16 else lib().opw_linear_bf16
        check(fn(_p(X), _p(W), _p(bias), _p(Y), rows, in_features, out_features, self.ACTIVATIONS[activation],
                 _stream(stream)))

    def attention_prefill(self, q: Ptr, k: Ptr, v: Ptr, out: Ptr, T: int, S: int, q_offset: int, num_q_heads: int,
                          kv_rep: int, head_dim: int, cap: int, stream=None) -> None:
        check(lib().opw_attention_prefill_f32(_p(q), _p(k), _p(v), _p(out), T, S, q_offset, num_q_heads, kv_rep,
                                              head_dim, cap, _stream(stream)))

    # Workspace form: the heaviest query-tile groups split their K/V range over two workgroups.
    def attention_prefill_workspace_size(self, T: int, S: int, q_offset: int, num_q_heads: int, kv_rep: int,
                                         head_dim: int, split_threshold: int = -1) -> tuple:
        rec, ctr = c_int64(0), c_int64(0)
        check(lib().opw_attention_prefill_workspace_size(T, S, q_offset, num_q_heads, kv_rep, head_dim,
                                                         split_threshold, ctypes.byref(rec), ctypes.byref(ctr)))
        return rec.value, ctr.value

    def attention_prefill_ws(self, q: Ptr, k: Ptr, v: Ptr, out: Ptr, T: int, S: int, q_offset: int, num_q_heads: int,
                             kv_rep: int, head_dim: int, cap: int, rec: Ptr, rec_floats: int, counters: Ptr,
                             counter_ints: int, split_threshold: int = -1, stream=None) -> None:
        check(lib().opw_attention_prefill_ws_f32(_p(q), _p(k), _p(v), _p(out), T, S, q_offset, num_q_heads, kv_rep,
                                                 head_dim, cap, _p(rec), rec_floats, _p(counters), counter_ints,
                                                 split_threshold, _stream(stream)))

    def attention_decode(self, q: Ptr, k: Ptr, v: Ptr, out: Ptr, num_q_heads: int, kv_rep: int, head_dim: int,
                         length: int, max_seq: int, workspace: Ptr = None, workspace_size: int = 0,
                         stream=None) -> None:
        if workspace is None:
            check(lib().opw_attention_decode_f32(_p(q), _p(k), _p(v), _p(out), num_q_heads, kv_rep, head_dim, length,
                                                 max_seq, _stream(stream)))
        else:
            if isinstance(workspace, DeviceView) and workspace_size == 0:
                workspace_size = workspace.n
            check(lib().opw_attention_decode_ws_f32(_p(q), _p(k), _p(v), _p(out), num_q_heads, kv_rep, head_dim,
                                                    length, max_seq, _p(workspace), workspace_size,
                                                    _stream(stream)))

    # One launch: the last chunk workgroup of each kv head merges; counters (int32,
    # attention_decode_counters_size of them) are zero before and after the call.
    def attention_decode_fused(self, q: Ptr, k: Ptr, v: Ptr, out: Ptr, num_q_heads: int, kv_rep: int,
                               head_dim: int, length: int, max_seq: int, workspace: Ptr, workspace_size: int,
                               counters: Ptr, counters_size: int = 0, stream=None) -> None:
        if isinstance(counters, DeviceView) and counters_size == 0:
            counters_size = counters.n
        check(lib().opw_attention_decode_fused_f32(_p(q), _p(k), _p(v), _p(out), num_q_heads, kv_rep, head_dim,
                                                   length, max_seq, _p(workspace), workspace_size, _p(counters),
                                                   counters_size, _stream(stream)))

    def attention_decode_counters_size(self, num_q_heads: int, kv_rep: int) -> int:
        return check(lib().opw_attention_decode_counters_size(num_q_heads, kv_rep))

    def attention_decode_workspace_size(self, num_q_heads: int, max_len: int, head_dim: int) -> int:
        return check(lib().opw_attention_decode_workspace_size(num_q_heads, max_len, head_dim))

    def convert_f32_to_bf16(self, src: Ptr, dst: Ptr, n: int, stream=None) -> None:
        check(lib().opw_convert_f32_to_bf16(_p(src), _p(dst), n, _stream(stream)))

    # ---- decoder-block steps
    def add(self, a: Ptr, b: Ptr, out: Ptr, n: int, stream=None) -> None:
        check(lib().opw_add_f32(_p(a), _p(b), _p(out), n, _stream(stream)))

    def swiglu(self, gate: Ptr, up: Ptr, out: Ptr, n: int, stream=None) -> None:
        check(lib().opw_swiglu_f32(_p(gate), _p(up), _p(out), n, _stream(stream)))

    def causal_scale(self, scores: Ptr, rows: int, cols: int, scale: float, stream=None) -> None:
        check(lib().opw_causal_scale_f32(_p(scores), rows, cols, scale, _stream(stream)))

    def embedding(self, table: Ptr, vocab: int, ids: Ptr, out: Ptr, n: int, hidden: int, bf16: bool = False,
                  stream=None) -> None:
        fn = lib().opw_embedding_bf16 if bf16 else lib().opw_embedding_f32
        check(fn(_p(table), vocab, _p(ids), _p(out), n, hidden, _stream(stream)))

    def split_heads(self, x: Ptr, out: Ptr, rows: int, heads: int, head_dim: int, out_row_stride: int,
                    out_row_offset: int = 0, stream=None) -> None:
        check(lib().opw_split_heads_f32(_p(x), _p(out), rows, heads, head_dim, out_row_stride, out_row_offset,
                                        _stream(stream)))

    def merge_heads(self, x: Ptr, out: Ptr, rows: int, heads: int, head_dim: int, in_row_stride: int,
                    in_row_offset: int = 0, stream=None) -> None:
        check(lib().opw_merge_heads_f32(_p(x), _p(out), rows, heads, head_dim, in_row_stride, in_row_offset,
                                        _stream(stream)))

    def rope(self, x: Ptr, inv_freq: Ptr, rows: int, heads: int, head_dim: int, pos_start: int, stream=None) -> None:
        check(lib().opw_rope_f32(_p(x), _p(inv_freq), rows, heads, head_dim, pos_start, _stream(stream)))

    def argmax(self, x: Ptr, n: int, out: Ptr, stream=None) -> None:
        check(lib().opw_argmax_f32(_p(x), n, _p(out), _stream(stream)))

    SCAN_OPS = {"sum": 0, "maximum": 1}

    def scan_workspace_size(self, n: int) -> int:
        return check(lib().opw_scan_workspace_size(n))

    def scan(self, x: Ptr, out: Ptr, n: int, op: str = "sum", inclusive: bool = True, workspace: Ptr = None,
             workspace_size: int = 0, stream=None) -> None:
        check(lib().opw_scan_f32(_p(x), _p(out), n, self.SCAN_OPS[op], int(inclusive), _p(workspace),
                                 workspace_size, _stream(stream)))

    def transpose(self, x: Ptr, out: Ptr, rows: int, cols: int, stream=None) -> None:
        check(lib().opw_transpose_f32(_p(x), _p(out), rows, cols, _stream(stream)))

    def copy(self, x: Ptr, out: Ptr, n: int, stream=None) -> None:
        check(lib().opw_copy_f32(_p(x), _p(out), n, _stream(stream)))

    def gather(self, x: Ptr, in_size: int, idx: Ptr, out: Ptr, count: int, stream=None) -> None:
        check(lib().opw_gather_f32(_p(x), in_size, _p(idx), _p(out), count, _stream(stream)))

    def scatter(self, x: Ptr, idx: Ptr, out: Ptr, out_size: int, count: int, stream=None) -> None:
        check(lib().opw_scatter_f32(_p(x), _p(idx), _p(out), out_size, count, _stream(stream)))


ops = _Ops()

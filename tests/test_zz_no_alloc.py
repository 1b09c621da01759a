"""GPU: opw_reduce_f32_noalloc — the reduction for callers that cannot allocate
(graph capture, serving loops, harnesses that forbid hipMalloc). Its partials
live in a static device array of the library instead of a workspace.

Checked against opw_reduce_f32 with a caller workspace (the same kernels and
summation order, so bit-identical) for every op, on two calls in a row, the
second with a smaller input, so a result cannot come from the previous call's
scratch contents; the 2^29-element limit is rejected before any launch."""
import ctypes
from ctypes import c_float, c_int, c_void_p

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
SEED = 8080
LIMIT = 1 << 29


def noalloc(lib):
    fn = lib.opw_reduce_f32_noalloc
    fn.argtypes = [c_void_p, c_void_p, c_int, c_int, c_void_p]
    fn.restype = c_int
    return fn


def with_workspace(ow, d_in, n, op):
    out = ow.DeviceBuffer.empty(1)
    ws_n = ow.lib().opw_reduction_workspace_size(n)
    ws = ow.DeviceBuffer.empty(max(ws_n, 1))
    ow.check(ow.lib().opw_reduce_f32(d_in.ptr, out.ptr, n, op, ws.ptr, max(ws_n, 1), None))
    return out.to_host()[0]


@pytest.mark.parametrize("op", [0, 1, 2])
def test_noalloc_reduce_matches_workspace_form(ow, orc, op):
    fn = noalloc(ow.lib())
    sizes = [(1 << 24) + 77, 100_003, 8192, 1, 0]  # shrinking: each call reuses the scratch of the last
    for i, n in enumerate(sizes):
        print(f"[noalloc] op={op} n={n}", flush=True)
        if op == 2:  # product of values near 1 stays finite
            host = (1.0 + orc.fill_uniform(max(n, 1), SEED, 10 + i, -1e-6, 1e-6))[:n].astype(np.float32)
        else:
            host = orc.fill_normal(max(n, 1), SEED, 20 + i, 0.0, 1.0)[:n]
        d_in = ow.DeviceBuffer.from_host(host) if n else ow.DeviceBuffer.empty(1)
        out = ow.DeviceBuffer.empty(1)
        assert fn(d_in.ptr, out.ptr, n, op, None) == 0, ow.lib().opw_last_error()
        got = np.float32(out.to_host()[0])
        want = np.float32(with_workspace(ow, d_in, n, op))
        assert got.view(np.uint32) == want.view(np.uint32), (op, n, got, want)
        if n and op == 0:
            assert abs(float(got) - float(host.astype(np.float64).sum())) <= 1e-5 * float(np.abs(host).sum())


def test_noalloc_reduce_on_a_stream_and_limits(ow, orc):
    fn = noalloc(ow.lib())
    n = 3 * 8192 + 5
    host = orc.fill_normal(n, SEED, 40, 0.0, 1.0)
    d_in = ow.DeviceBuffer.from_host(host)
    out = ow.DeviceBuffer.empty(1)
    stream = ow.Stream()
    assert fn(d_in.ptr, out.ptr, n, 1, stream.handle) == 0
    stream.synchronize()
    assert out.to_host()[0] == np.max(host)
    # beyond the static scratch: rejected before anything is enqueued (no input of that size exists)
    assert fn(d_in.ptr, out.ptr, LIMIT + 1, 0, None) == -1
    assert "536870912" in ow.lib().opw_last_error().decode()
    assert fn(d_in.ptr, out.ptr, 10, 7, None) == -1
    assert fn(d_in.ptr, out.ptr, -1, 0, None) == -1


@pytest.mark.parametrize("op", [0, 1])
def test_noalloc_reduce_in_a_captured_graph(ow, orc, op):
    """Captured into a HIP graph (global mode: an allocation inside the call would fail the capture) after a
    first call outside capture has looked up the device's scratch address, then replayed three times, each
    after new input contents were uploaded into the captured buffer, with eager workspace-form calls between
    the replays: every replay bit-identical to opw_reduce_f32 with a caller workspace."""
    fn = noalloc(ow.lib())
    n = (1 << 20) + 333
    d_in = ow.DeviceBuffer.from_host(orc.fill_normal(n, SEED, 70, 0.0, 1.0))
    out = ow.DeviceBuffer.empty(1)
    assert fn(d_in.ptr, out.ptr, n, op, None) == 0, ow.lib().opw_last_error()
    stream = ow.Stream()
    stream.synchronize()

    def body():
        assert fn(d_in.ptr, out.ptr, n, op, stream.handle) == 0, ow.lib().opw_last_error()

    graph = ow.Graph.capture(stream, body)
    for r in range(3):
        host = orc.fill_normal(n, SEED, 71 + r, 0.0, 1.0)
        d_in.copy_from_host(host)
        graph.launch(stream)
        stream.synchronize()
        got = np.float32(out.to_host()[0])
        want = np.float32(with_workspace(ow, d_in, n, op))
        assert got.view(np.uint32) == want.view(np.uint32), (op, r, got, want)
        if op == 1:
            assert got == np.max(host)

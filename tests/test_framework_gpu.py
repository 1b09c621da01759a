"""GPU: the hipcc-built framework self-test executable (C++ operator API,
builders, graph replay, two translation units) and the six `solve` challenge
adapters, each called through ctypes like the reference's runner
(tests/run.py:48-64) and checked against the CPU oracle.

Bars: vector_add / relu bit-exact; softmax and layer_normalization within
|a-e| <= 1e-5 (1+|e|); reduction |gpu - sum| <= 1e-5 * sum|x|;
matrix_multiplication |gpu - ref| <= 1e-4 * sum_k |a b| per element."""
import ctypes
import subprocess
from ctypes import POINTER, c_float, c_int, c_size_t, c_void_p

import numpy as np
import pytest

from tests.conftest import ROOT, bits, framework_close

pytestmark = pytest.mark.gpu
SEED = 77
ADAPTERS = ROOT / "opworks_amd" / "lib" / "adapters"


def test_framework_executable():
    """The C++ operator API self-test, driven by the reference unit test's known answers
    (tests/golden/framework_kats.json)."""
    exe = ROOT / "opworks_amd" / "lib" / "tests" / "framework"
    assert exe.exists(), "build the C++ tests first (python -m opworks_amd.build tests)"
    kats = ROOT / "tests" / "golden" / "framework_kats.json"
    print("[framework] running", exe, kats, flush=True)
    proc = subprocess.run([str(exe), str(kats)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                          timeout=90)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout
    assert proc.stdout.startswith("PASS"), proc.stdout


_SIGS = {
    "vector_add": [c_void_p, c_void_p, c_void_p, c_size_t],
    "relu": [c_void_p, c_void_p, c_int],
    "reduction": [c_void_p, c_void_p, c_int],
    "softmax": [c_void_p, c_void_p, c_int],
    "layer_normalization": [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_float],
    "matrix_multiplication": [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int],
}


def solve(name):
    lib = ctypes.CDLL(str(ADAPTERS / f"libopw_solve_{name}.so"))
    fn = lib.solve
    fn.argtypes = _SIGS[name]
    fn.restype = None
    lib.opw_solve_last_error.restype = ctypes.c_char_p
    return fn, lib


def up(ow, a):
    return ow.DeviceBuffer.from_host(np.ascontiguousarray(a, np.float32))


@pytest.mark.parametrize("n", [1, 3, 4, 1025, 1 << 20])
def test_vector_add_and_relu(ow, orc, n):
    a = orc.fill_uniform(n, SEED, 0, -1, 1)
    b = orc.fill_uniform(n, SEED, 1, -1, 1)
    da, db, dout = up(ow, a), up(ow, b), ow.DeviceBuffer.empty(n)
    add, _ = solve("vector_add")
    add(da.ptr, db.ptr, dout.ptr, n)
    assert np.array_equal(bits(dout.to_host()), bits(a + b))
    relu, _ = solve("relu")
    relu(da.ptr, dout.ptr, n)
    assert np.array_equal(bits(dout.to_host()), bits(np.maximum(a, np.float32(0))))


@pytest.mark.parametrize("n", [0, 1, 257, 4099, 1 << 22])
def test_reduction(ow, orc, n):
    x = orc.fill_uniform(max(n, 1), SEED, 2, -1, 1)[:n]
    dx, dout = up(ow, x) if n else ow.DeviceBuffer.empty(1), ow.DeviceBuffer.empty(1)
    fn, _ = solve("reduction")
    for _ in range(2):  # the second call reuses the cached workspace
        fn(dx.ptr, dout.ptr, n)
        got = float(dout.to_host()[0])
        assert abs(got - orc.sum_f64(x)) <= 1e-5 * orc.sum_abs_f64(x) + 1e-30


@pytest.mark.parametrize("n", [1, 5, 1000, 4096, 50_000])
def test_softmax(ow, orc, n):
    x = orc.fill_normal(n, SEED, 3, 0, 3)
    dx, dout = up(ow, x), ow.DeviceBuffer.empty(n)
    fn, _ = solve("softmax")
    fn(dx.ptr, dout.ptr, n)
    assert framework_close(dout.to_host(), orc.softmax_rows(x, 1, n))


@pytest.mark.parametrize("rows,cols", [(1, 1), (2, 5), (7, 300), (64, 4096)])
def test_layer_normalization(ow, orc, rows, cols):
    x = orc.fill_normal(rows * cols, SEED, 4, 0.5, 2)
    g = orc.fill_uniform(cols, SEED, 5, 0.5, 1.5)
    b = orc.fill_uniform(cols, SEED, 6, -0.5, 0.5)
    dx, dg, db, dout = up(ow, x), up(ow, g), up(ow, b), ow.DeviceBuffer.empty(rows * cols)
    fn, _ = solve("layer_normalization")
    fn(dx.ptr, dg.ptr, db.ptr, dout.ptr, rows, cols, 1e-5)
    assert framework_close(dout.to_host(), orc.layer_norm_rows(x, g, b, rows, cols, 1e-5))


@pytest.mark.parametrize("m,n,k", [(3, 5, 7), (64, 64, 64), (129, 257, 65), (512, 512, 512)])
def test_matrix_multiplication(ow, orc, m, n, k):
    a = orc.fill_normal(m * n, SEED, 7, 0, 1)
    b = orc.fill_normal(n * k, SEED, 8, 0, 1)
    da, db, dout = up(ow, a), up(ow, b), ow.DeviceBuffer.empty(m * k)
    fn, _ = solve("matrix_multiplication")
    fn(da.ptr, db.ptr, dout.ptr, m, n, k)
    ref, absdot = orc.mat_mul_rows(a, b, m, n, k)
    err = np.abs(dout.to_host().reshape(m, k).astype(np.float64) - ref)
    assert np.all(err <= 1e-4 * absdot + 1e-6)


def test_adapter_contract_violation_is_reported(ow):
    """Null inputs with n > 0 are rejected before any launch; outputs untouched,
    the message kept per thread and cleared by the next good call."""
    out = up(ow, [42.0])
    fn, lib = solve("softmax")
    fn(None, out.ptr, 1)
    assert b"non-null" in lib.opw_solve_last_error()
    assert out.to_host()[0] == 42.0
    x = up(ow, [0.0])
    fn(x.ptr, out.ptr, 1)
    assert lib.opw_solve_last_error() == b""
    assert out.to_host()[0] == 1.0

"""GPU parity: map / reduce / softmax / layer_norm / rms_norm through the C ABI
against the CPU oracle on identical seeded inputs.

Bars: map bit-exact; reduce |gpu - ref| <= 1e-5 * sum|x|; row ops within the
reference's unit-test criterion |a-e| <= 1e-5 (1+|e|) and, elementwise,
relative error <= 1e-5 where |e| is not tiny."""
import math

import numpy as np
import pytest

from tests.conftest import bits, framework_close, max_rel

pytestmark = pytest.mark.gpu

SEED = 1234


def upload(ow, arr):
    return ow.DeviceBuffer.from_host(np.ascontiguousarray(arr, np.float32))


# ----------------------------------------------------------------------- map
def test_fill_generators_bit_identical(ow, orc):
    n = 100_003
    buf = ow.DeviceBuffer.empty(n)
    ow.fill_uniform(buf, SEED, 3, -1.0, 1.0)
    assert np.array_equal(bits(buf.to_host()), bits(orc.fill_uniform(n, SEED, 3, -1.0, 1.0)))
    ow.fill_normal(buf, SEED, 4, 0.0, 0.02)
    assert np.array_equal(bits(buf.to_host()), bits(orc.fill_normal(n, SEED, 4, 0.0, 0.02)))


def test_map_known_answers(ow):
    a = upload(ow, [1, 2, 3])
    b = upload(ow, [4, 5, 6])
    out = ow.DeviceBuffer.empty(3)
    ow.ops.map_add(a, b, out, 3)
    assert np.array_equal(out.to_host(), [5, 7, 9])
    ow.ops.map_scale(a, out, 3, 3.0)
    assert np.array_equal(out.to_host(), [3, 6, 9])


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 31, 32, 33, 255, 256, 257, 1025, 65539])
@pytest.mark.parametrize("offset", [0, 1])
def test_map_boundaries_and_inplace(ow, orc, n, offset):
    # tests/unit/framework.cu:109-129: values i-10, aligned and misaligned starts, exact in-place
    host = (np.arange(n + offset) - 10).astype(np.float32)
    a = upload(ow, host)
    b = upload(ow, host)
    out = ow.DeviceBuffer.empty(n + offset)
    ow.ops.map_add(a.offset(offset), b.offset(offset), out.offset(offset), n)
    assert np.array_equal(out.to_host()[offset:], 2 * host[offset:])
    ow.ops.map_scale(a.offset(offset), a.offset(offset), n, 3.0)
    assert np.array_equal(a.to_host()[offset:], 3 * host[offset:])
    # ScaleAdd is bit-exact against fmaf on random data on both paths
    x = orc.fill_uniform(n + offset, SEED, 10, -1, 1)
    y = orc.fill_uniform(n + offset, SEED, 11, -1, 1)
    dx, dy = upload(ow, x), upload(ow, y)
    ow.ops.map_scale_add(dx.offset(offset), dy.offset(offset), out.offset(offset), n, 2.5)
    assert np.array_equal(bits(out.to_host()[offset:]), bits(orc.map_scale_add(x[offset:], y[offset:], 2.5)))


@pytest.mark.slow
def test_map_scale_add_full_size_bit_exact(ow, orc):
    """Config 2: n = 2^28, a, b ~ U[-1,1] from the seed, alpha = 2.5."""
    n = 1 << 28
    orc.set_threads(16)
    a = ow.DeviceBuffer.empty(n)
    b = ow.DeviceBuffer.empty(n)
    c = ow.DeviceBuffer.empty(n)
    ow.fill_uniform(a, SEED, 0, -1.0, 1.0)
    ow.fill_uniform(b, SEED, 1, -1.0, 1.0)
    ow.ops.map_scale_add(a, b, c, n, 2.5)
    got = c.to_host()
    ha = orc.fill_uniform(n, SEED, 0, -1.0, 1.0, mt=True)
    hb = orc.fill_uniform(n, SEED, 1, -1.0, 1.0, mt=True)
    want = orc.map_scale_add(ha, hb, 2.5, mt=True)
    assert np.array_equal(bits(got), bits(want))
    # reduce of the same c at full size: within 1e-5 of sum|c|, and deterministic
    out = ow.DeviceBuffer.empty(1)
    ws = ow.DeviceBuffer.empty(ow.ops.reduction_workspace_size(n))
    ow.ops.reduce(c, out, n, "sum", ws)
    r1 = out.to_host()[0]
    ow.ops.reduce(c, out, n, "sum", ws)
    assert out.to_host()[0] == r1
    ref = orc.reduce(want, "sum")
    assert abs(r1 - ref) <= 1e-5 * orc.sum_abs_f64(want)


# -------------------------------------------------------------------- reduce
@pytest.mark.parametrize("n", [0, 1, 31, 32, 33, 255, 256, 257, 4097, 4099, 8191, 8192, 8193, 16385, 100_000, 1 << 20, (1 << 20) + 3])
def test_reduce_sum_matches_oracle(ow, orc, n):
    x = orc.fill_normal(max(n, 1), SEED, 20 + n % 97, 0.0, 1.0)[:n]
    dx = upload(ow, x) if n else ow.DeviceBuffer.empty(0)
    out = ow.DeviceBuffer.empty(1)
    ws_n = ow.ops.reduction_workspace_size(n)
    ws = ow.DeviceBuffer.empty(ws_n)
    ow.ops.reduce(dx, out, n, "sum", ws if ws_n else None, ws_n)
    got = float(out.to_host()[0])
    ref = orc.reduce(x, "sum")
    assert abs(got - ref) <= 1e-5 * max(orc.sum_abs_f64(x), 1e-30)
    # convenience overload (stream-ordered allocation)
    ow.ops.reduce(dx, out, n, "sum")
    assert abs(float(out.to_host()[0]) - ref) <= 1e-5 * max(orc.sum_abs_f64(x), 1e-30)


def test_reduce_ones_and_ops(ow, orc):
    ones = upload(ow, np.ones(4099, np.float32))
    out = ow.DeviceBuffer.empty(1)
    ws = ow.DeviceBuffer.empty(ow.ops.reduction_workspace_size(4099))
    for n in (0, 1, 31, 32, 33, 255, 256, 257, 4099):  # framework.cu:144-149
        ow.ops.reduce(ones, out, n, "sum", ws)
        assert out.to_host()[0] == n
    empty = ow.DeviceBuffer.empty(0)
    ow.ops.reduce(empty, out, 0, "product")
    assert out.to_host()[0] == 1.0  # framework.cu:80
    x = orc.fill_normal(12345, SEED, 30, 0.0, 1.0)
    ow.ops.reduce(upload(ow, x), out, x.size, "max")
    assert out.to_host()[0] == x.max()
    # misaligned input takes the scalar kernel
    d = upload(ow, x)
    ow.ops.reduce(d.offset(1), out, x.size - 1, "sum")
    assert abs(out.to_host()[0] - orc.reduce(x[1:], "sum")) <= 1e-5 * orc.sum_abs_f64(x)


# ---------------------------------------------------------------------- rows
ROW_SHAPES = [(2, 5), (3, 64), (7, 256), (5, 300), (9, 512), (4096, 1024), (11, 1028), (3, 2048), (6, 4096),
              (3, 8192), (2, 16384), (2, 32768), (2, 32772), (3, 1001)]


def _rows_input(orc, rows, cols, scale, stream):
    return orc.fill_normal(rows * cols, SEED, stream, 0.0, scale)


@pytest.mark.parametrize("rows,cols", ROW_SHAPES)
def test_softmax_matches_oracle(ow, orc, rows, cols):
    x = _rows_input(orc, rows, cols, 4.0, 40)
    dx = upload(ow, x)
    out = ow.DeviceBuffer.empty(rows * cols)
    ow.ops.softmax(dx, out, rows, cols)
    got = out.to_host()
    ref = orc.softmax_rows(x, rows, cols)
    assert framework_close(got, ref)
    big = ref > 1e-30
    assert max_rel(got[big], ref[big]) <= 1e-5


def test_softmax_known_answer_and_inplace(ow):
    x = np.arange(-2, 8, dtype=np.float32)  # framework.cu:185-195
    d = upload(ow, x)
    ow.ops.softmax(d, d, 2, 5)
    den = sum(math.exp(j - 4) for j in range(5))
    assert framework_close(d.to_host(), [math.exp(i % 5 - 4) / den for i in range(10)])


@pytest.mark.parametrize("rows,cols", ROW_SHAPES)
def test_layer_norm_matches_oracle(ow, orc, rows, cols):
    x = _rows_input(orc, rows, cols, 2.0, 41) + np.float32(0.5)
    g = orc.fill_uniform(cols, SEED, 42, 0.5, 1.5)
    b = orc.fill_uniform(cols, SEED, 43, -0.5, 0.5)
    out = ow.DeviceBuffer.empty(rows * cols)
    ow.ops.layer_norm(upload(ow, x), out, upload(ow, g), upload(ow, b), rows, cols, 1e-5)
    got = out.to_host()
    ref = orc.layer_norm_rows(x, g, b, rows, cols, 1e-5)
    assert framework_close(got, ref)


def test_layer_norm_known_answer(ow):
    x = np.arange(-2, 8, dtype=np.float32)  # framework.cu:196-199
    out = ow.DeviceBuffer.empty(10)
    ow.ops.layer_norm(upload(ow, x), out, upload(ow, np.full(5, 2.0)), upload(ow, np.ones(5)), 2, 5, 1e-5)
    assert framework_close(out.to_host(), [(i % 5 - 2) * 2 / math.sqrt(2 + 1e-5) + 1 for i in range(10)])


# (512, 2048), (1500, 2048): prefill shapes whose rows are spread over 4 and 2 waves
@pytest.mark.parametrize("rows,cols", ROW_SHAPES + [(8192, 2048), (512, 2048), (1500, 2048)])
def test_rms_norm_matches_oracle(ow, orc, rows, cols):
    x = _rows_input(orc, rows, cols, 1.0, 44)
    w = orc.fill_uniform(cols, SEED, 45, 0.5, 1.5)
    out = ow.DeviceBuffer.empty(rows * cols)
    ow.ops.rms_norm(upload(ow, x), upload(ow, w), out, rows, cols, 1e-5)
    got = out.to_host()
    ref = orc.rms_norm_rows(x, w, rows, cols, 1e-5)
    assert framework_close(got, ref)
    nz = np.abs(ref) > 1e-6
    assert max_rel(got[nz], ref[nz]) <= 1e-5


def test_rows_misaligned_take_streaming_kernel(ow, orc):
    rows, cols = 5, 1024
    x = _rows_input(orc, rows, cols + 1, 3.0, 46)
    d = upload(ow, x)
    out = ow.DeviceBuffer.empty(rows * cols + 1)
    ow.ops.softmax(d.offset(1), out.offset(1), rows, cols)
    assert framework_close(out.to_host()[1:], orc.softmax_rows(x[1:], rows, cols))

"""GPU parity of the bf16 matrix-core path (ops::linear_mma_bf16 equivalent).

Bars: against the oracle run on the same bf16-rounded inputs, K-scaled 1e-4
(far tighter than needed); against the unrounded fp32 product, the reference's
bf16 bar NRMSE <= 1e-2 and cosine >= 0.999 (tests/model/ops_test.cu:101-116)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
SEED = 4321


def upload(ow, arr, dtype=np.float32):
    return ow.DeviceBuffer.from_host(np.ascontiguousarray(arr, dtype))


def nrmse_cos(got, ref):
    got = got.astype(np.float64).ravel()
    ref = ref.astype(np.float64).ravel()
    nrmse = np.sqrt(np.mean((got - ref) ** 2)) / max(np.sqrt(np.mean(ref ** 2)), 1e-6)
    cos = float(got @ ref / max(np.linalg.norm(got) * np.linalg.norm(ref), 1e-30))
    return nrmse, cos


def test_convert_bits_match_oracle(ow, orc):
    x = orc.fill_normal(100_001, SEED, 0, 0.0, 3.0)
    dx = upload(ow, x)
    db = ow.DeviceBuffer.empty(x.size, np.uint16)
    ow.ops.convert_f32_to_bf16(dx, db, x.size)
    assert np.array_equal(db.to_host(), orc.round_bf16(x)[1])


SHAPES = [(1, 8, 1), (16, 64, 64), (100, 200, 300), (256, 256, 256), (300, 2048, 520), (512, 1024, 3072),
          (257, 40, 513), (3, 4104, 7),  # a full K tile + an 8-wide tail; tiles one row/column past 256
          # the three-stage 128 x 256 tiles (from 256 rows) with 1, 2 and 3 full K tiles, tails and
          # partial row and column tiles
          (260, 72, 300), (512, 128, 512), (300, 200, 600)]


@pytest.mark.parametrize("rows,in_f,out_f", SHAPES)
@pytest.mark.parametrize("x_bf16", [False, True])
@pytest.mark.parametrize("act", ["none", "relu"])
def test_linear_bf16_matches_oracle(ow, orc, rows, in_f, out_f, x_bf16, act):
    X = orc.fill_normal(rows * in_f, SEED, 1, 0.0, 1.0)
    W = orc.fill_normal(out_f * in_f, SEED, 2, 0.0, 0.05)
    bias = orc.fill_uniform(out_f, SEED, 3, -0.1, 0.1)
    Xr, Xb = orc.round_bf16(X)
    Wr, Wb = orc.round_bf16(W)
    dX = upload(ow, Xb, np.uint16) if x_bf16 else upload(ow, X)
    dW = upload(ow, Wb, np.uint16)
    dbias = upload(ow, bias)
    Y = ow.DeviceBuffer.empty(rows * out_f)
    ow.ops.linear_bf16(dX, dW, dbias, Y, rows, in_f, out_f, activation=act, x_bf16=x_bf16)
    got = Y.to_host().reshape(rows, out_f)
    ref, absdot = orc.mat_mul_rows(Xr, Wr, rows, in_f, out_f, bias=bias, b_transposed=True, act=act)
    err = np.abs(got.astype(np.float64) - ref) / (1e-4 * absdot + 1e-6)
    assert float(err.max()) <= 1.0
    full, _ = orc.mat_mul_rows(X, W, rows, in_f, out_f, bias=bias, b_transposed=True, act=act)
    if full.size >= 64:  # NRMSE / cosine are statistics over many outputs
        nrmse, cos = nrmse_cos(got, full)
        assert nrmse <= 1e-2 and cos >= 0.999, (nrmse, cos)


@pytest.mark.parametrize("rows,in_f,out_f", [(33, 100, 70), (17, 1001, 129)])
def test_linear_bf16_unaligned_k(ow, orc, rows, in_f, out_f):
    X = orc.fill_normal(rows * in_f, SEED, 4, 0.0, 1.0)
    W = orc.fill_normal(out_f * in_f, SEED, 5, 0.0, 0.05)
    Xr, _ = orc.round_bf16(X)
    Wr, Wb = orc.round_bf16(W)
    dX, dW = upload(ow, X), upload(ow, Wb, np.uint16)
    Y = ow.DeviceBuffer.empty(rows * out_f)
    ow.ops.linear_bf16(dX, dW, None, Y, rows, in_f, out_f)
    ref, absdot = orc.mat_mul_rows(Xr, Wr, rows, in_f, out_f, b_transposed=True)
    assert float((np.abs(Y.to_host().reshape(rows, out_f) - ref) / (1e-4 * absdot + 1e-6)).max()) <= 1.0


@pytest.mark.slow
def test_config3_bf16_full_size_sampled(ow, orc):
    """Config 3 bf16 variant: relu(A @ B + bias) at 4096^3 with A, W bf16-rounded; 128 sampled rows."""
    n = 4096
    orc.set_threads(16)
    A = orc.fill_normal(n * n, SEED, 300, 0.0, 1.0 / 64, mt=True)
    W = orc.fill_normal(n * n, SEED, 301, 0.0, 1.0 / 64, mt=True)
    bias = orc.fill_uniform(n, SEED, 302, -0.1, 0.1)
    Ar, Ab = orc.round_bf16(A)
    Wr, Wb = orc.round_bf16(W)
    dA, dW, dbias = upload(ow, Ab, np.uint16), upload(ow, Wb, np.uint16), upload(ow, bias)
    Y = ow.DeviceBuffer.empty(n * n)
    ow.ops.linear_bf16(dA, dW, dbias, Y, n, n, n, activation="relu", x_bf16=True)
    rows = np.arange(0, n, 32)
    ref, absdot = orc.mat_mul_rows(Ar, Wr, n, n, n, rows=rows, bias=bias, b_transposed=True, act="relu")
    got = Y.to_host().reshape(n, n)[rows]
    assert float((np.abs(got - ref) / (1e-4 * absdot + 1e-6)).max()) <= 1.0


@pytest.mark.parametrize("rows,in_f,out_f", [(1, 2048, 2048), (1, 8192, 2048), (1, 2048, 513), (1, 100, 37),
                                             (2, 2048, 512), (15, 2048, 3072), (16, 2048, 2048), (16, 100, 64),
                                             (7, 4104, 33)])
def test_linear_bf16_weights_keep_fp32_inputs(ow, orc, rows, in_f, out_f):
    """ops::linear<bf16> (reference include/ops/linear.cuh:99-153): fp32 X against bf16 weights widened
    exactly, fp32 accumulation, at every row count (the GEMV at rows == 1, the fp32 GEMM with a widened
    B operand above). Bars: against the oracle on the widened weights, K-scaled 1e-4; against the float64
    product of the fp32 inputs and the widened weights, 1e-6 * sum|x w| per element, which a path that
    rounds X to bf16 (typically 3e-5 to 1e-4 of sum|x w| at these widths) cannot meet. in % 8 != 0 takes the scalar GEMV."""
    X = orc.fill_normal(rows * in_f, SEED, 11, 0.0, 1.0)
    W = orc.fill_normal(out_f * in_f, SEED, 12, 0.0, 0.02)
    Wr, Wb = orc.round_bf16(W)
    dX, dW = upload(ow, X), upload(ow, Wb, np.uint16)
    Y = ow.DeviceBuffer.empty(rows * out_f)
    ow.ops.linear_wbf16(dX, dW, Y, rows, in_f, out_f)
    got = Y.to_host().reshape(rows, out_f).astype(np.float64)
    ref, absdot = orc.mat_mul_rows(X, Wr, rows, in_f, out_f, b_transposed=True)
    assert float(np.max(np.abs(got - ref) / (1e-4 * absdot + 1e-6))) <= 1.0
    exact = X.reshape(rows, in_f).astype(np.float64) @ Wr.reshape(out_f, in_f).astype(np.float64).T
    assert float(np.max(np.abs(got - exact) / (1e-6 * absdot + 1e-12))) <= 1.0
    if rows == 1:  # the reference's GEMV (fp32 x, widened bf16 row) agrees too
        assert float(np.max(np.abs(got[0] - orc.gemv(X, Wr, in_f, out_f)) / (1e-4 * absdot[0] + 1e-6))) <= 1.0

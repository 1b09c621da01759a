"""GPU parity of the fp32 MFMA GEMM (ops::mat_mul, the fused MatmulBuilder
path, ops::linear incl. the rows == 1 GEMV) against the oracle's k-ascending
fmaf chains. Bar (north_star): |gpu - ref| <= 1e-4 * (sum_k |a_ik b_kj| + |bias_j|)
per element, i.e. relative 1e-4 K-scaled. Shapes use the reference's names:
A is M x N, B is N x K, C is M x K."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
SEED = 1234
KTOL = 1e-4


def upload(ow, arr):
    return ow.DeviceBuffer.from_host(np.ascontiguousarray(arr, np.float32))


def check_kscaled(got, ref, absdot, tol=KTOL, floor=1e-6):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = tol * absdot + floor
    worst = float(np.max(err / bound)) if err.size else 0.0
    assert worst <= 1.0, f"K-scaled error {worst:.3g} x bound"


def test_integer_known_answer(ow):
    # tests/unit/framework.cu:201-218 (3x5x7 integer inputs; exact in fp32)
    a = np.array([i % 7 - 3 for i in range(15)], np.float32)
    b = np.array([i % 5 - 2 for i in range(35)], np.float32)
    c = ow.DeviceBuffer.empty(21)
    da, db = upload(ow, a), upload(ow, b)  # keep the buffers alive across the launch
    ow.ops.mat_mul(da, db, c, 3, 5, 7)
    want = a.reshape(3, 5).astype(np.float64) @ b.reshape(5, 7).astype(np.float64)
    assert np.array_equal(c.to_host().reshape(3, 7), want.astype(np.float32))
    # zero reduction dim writes epilogue(0) (framework.cu:219-221)
    c.copy_from_host(np.full(21, 7.0, np.float32))
    ow.ops.mat_mul(None, None, c, 3, 0, 7)
    assert np.all(c.to_host() == 0)


SHAPES = [(1, 1, 1), (3, 5, 7), (64, 64, 64), (127, 33, 129), (128, 128, 128), (200, 300, 100), (257, 1000, 515),
          (512, 2048, 384), (130, 4, 260)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("b_t", [False, True])
@pytest.mark.parametrize("act", ["none", "relu", "gelu"])
def test_fused_matmul_matches_oracle(ow, orc, M, N, K, b_t, act):
    A = orc.fill_normal(M * N, SEED, 1, 0.0, 1.0)
    B = orc.fill_normal(N * K, SEED, 2, 0.0, 1.0)
    bias = orc.fill_uniform(K, SEED, 3, -0.1, 0.1)
    C = ow.DeviceBuffer.empty(M * K)
    dA, dB, dbias = upload(ow, A), upload(ow, B), upload(ow, bias)
    ow.ops.mat_mul_fused(dA, dB, dbias, C, M, N, K, b_transposed=b_t, activation=act)
    ref, absdot = orc.mat_mul_rows(A, B, M, N, K, bias=bias, b_transposed=b_t, act=act)
    check_kscaled(C.to_host().reshape(M, K), ref, absdot)


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (127, 33, 129), (130, 4, 260), (257, 1000, 515),
                                   (2048, 64, 1024), (4096, 96, 4096), (6, 9, 11)])
@pytest.mark.parametrize("b_t", [False, True])
@pytest.mark.parametrize("act", ["none", "relu"])
def test_fused_matmul_transposed_a(ow, orc, M, N, K, b_t, act):
    """MatmulBuilder::transpose_a (reference include/builders/matmul.cuh:19-20,35): op(A) = A^T with A stored
    N x M; the GEMM stages it in place. The oracle gets the transposed copy. M % 4 != 0 takes the scalar
    staging path; 4096 x 4096 outputs take the 256 x 256 tiles."""
    At = orc.fill_normal(N * M, SEED, 21, 0.0, 1.0)  # stored N x M
    B = orc.fill_normal(N * K, SEED, 22, 0.0, 1.0)
    bias = orc.fill_uniform(K, SEED, 23, -0.1, 0.1)
    C = ow.DeviceBuffer.empty(M * K)
    ow.ops.mat_mul_fused_ex(upload(ow, At), upload(ow, B), upload(ow, bias), C, M, N, K, True, b_t, activation=act)
    A = np.ascontiguousarray(At.reshape(N, M).T).ravel()
    rows = None if M <= 512 else np.arange(0, M, 61)
    ref, absdot = orc.mat_mul_rows(A, B, M, N, K, rows=rows, bias=bias, b_transposed=b_t, act=act)
    got = C.to_host().reshape(M, K)
    check_kscaled(got if rows is None else got[rows], ref, absdot)


@pytest.mark.parametrize("M,N,K", [(4100, 40, 4000), (4100, 37, 3999), (4096, 64, 4096), (520, 72, 16400),
                                   (520, 37, 16400)])
@pytest.mark.parametrize("b_t", [False, True])
def test_big_tile_path_every_element(ow, orc, M, N, K, b_t):
    """Outputs with at least 256 tiles of 256 x 256 take the 8-wave 256 x 256 kernel, outputs with
    fewer but at least 256 tiles of 256 x 128 (M = 520, 16400 columns: 195 and 387) the 8-wave
    256 x 128 one; ragged edges, an odd number of K tiles (inner dim 72), the scalar-load variant
    (inner dim 37) and both B layouts, every output element checked."""
    A = orc.fill_normal(M * N, SEED, 6, 0.0, 1.0)
    B = orc.fill_normal(N * K, SEED, 7, 0.0, 1.0)
    bias = orc.fill_uniform(K, SEED, 8, -0.1, 0.1)
    C = ow.DeviceBuffer.empty(M * K)
    dA, dB, dbias = upload(ow, A), upload(ow, B), upload(ow, bias)
    ow.ops.mat_mul_fused(dA, dB, dbias, C, M, N, K, b_transposed=b_t, activation="relu")
    orc.set_threads(16)
    ref, absdot = orc.mat_mul_rows(A, B, M, N, K, bias=bias, b_transposed=b_t, act="relu")
    check_kscaled(C.to_host().reshape(M, K), ref, absdot)


@pytest.mark.parametrize("M,N,K", [(5, 7, 9), (129, 130, 131), (256, 512, 128)])
def test_plain_matmul_and_misaligned(ow, orc, M, N, K):
    A = orc.fill_normal(M * N + 1, SEED, 4, 0.0, 1.0)
    B = orc.fill_normal(N * K + 1, SEED, 5, 0.0, 1.0)
    dA, dB = upload(ow, A), upload(ow, B)
    C = ow.DeviceBuffer.empty(M * K + 1)
    # offset by one float: not 16-byte aligned, takes the guarded scalar-load kernel
    ow.ops.mat_mul(dA.offset(1), dB.offset(1), C.offset(1), M, N, K)
    ref, absdot = orc.mat_mul_rows(A[1:], B[1:], M, N, K)
    check_kscaled(C.to_host()[1:].reshape(M, K), ref, absdot)


@pytest.mark.parametrize("rows,in_f,out_f", [(1, 2048, 2048), (1, 2048, 512), (1, 8192, 2048), (1, 100, 37),
                                             (1, 64, 2049), (2, 64, 64), (7, 2048, 3072), (512, 2048, 2048)])
def test_linear_matches_oracle(ow, orc, rows, in_f, out_f):
    X = orc.fill_normal(rows * in_f, SEED, 6, 0.0, 1.0)
    W = orc.fill_normal(out_f * in_f, SEED, 7, 0.0, 0.02)
    Y = ow.DeviceBuffer.empty(rows * out_f)
    dX, dW = upload(ow, X), upload(ow, W)
    ow.ops.linear(dX, dW, Y, rows, in_f, out_f)
    ref, absdot = orc.mat_mul_rows(X, W, rows, in_f, out_f, b_transposed=True)
    got = Y.to_host().reshape(rows, out_f)
    check_kscaled(got, ref, absdot)
    if rows == 1:  # the reference's own GEMV order agrees too
        check_kscaled(got[0], orc.gemv(X, W, in_f, out_f), absdot[0])


@pytest.mark.parametrize("rows,in_f,out_f", [(512, 2048, 3072), (300, 1000, 600), (1024, 8192, 512)])
def test_linear_bf16x6_path_has_fp32_accuracy(ow, rows, in_f, out_f):
    """ops::linear with fp32 weights at these sizes runs the bf16x6 kernel (three bf16 parts per
    operand, six MFMAs per product). Against float64 on sampled rows its error stays at fp32's
    level, 2e-6 of sum_k |x w| (the fp32 MFMA kernel's worst on the same data is of the same
    order), far inside the 1e-4 bar; ragged tiles (300 x 600) and a K tail (1000 = 31 x 32 + 8)."""
    rng = np.random.default_rng(SEED + rows)
    X = rng.standard_normal((rows, in_f)).astype(np.float32)
    W = (rng.standard_normal((out_f, in_f)) * 0.02).astype(np.float32)
    Y = ow.DeviceBuffer.empty(rows * out_f)
    dX, dW = upload(ow, X.ravel()), upload(ow, W.ravel())
    ow.ops.linear(dX, dW, Y, rows, in_f, out_f)
    got = Y.to_host().reshape(rows, out_f)
    sample = np.unique(np.concatenate([np.arange(0, rows, 37), [rows - 1]]))
    Xs, W64 = X[sample].astype(np.float64), W.astype(np.float64)
    ref = Xs @ W64.T
    absdot = np.abs(Xs) @ np.abs(W64).T
    check_kscaled(got[sample], ref, absdot, tol=2e-6, floor=0.0)


@pytest.mark.parametrize("M,N,K", [(512, 2048, 3072), (300, 1000, 604), (1024, 8192, 512)])
def test_matmul_bf16x6_kn_path_has_fp32_accuracy(ow, M, N, K):
    """ops::mat_mul with B as [N][K] (the reference's layout; inner dimension N here) runs the bf16x6
    kernel with B transposed while staged; same fp32-level bar as the nk form, ragged tiles and a
    tail of the inner dimension (1000 = 31 x 32 + 8)."""
    rng = np.random.default_rng(SEED + M + 1)
    A = rng.standard_normal((M, N)).astype(np.float32)
    B = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    C = ow.DeviceBuffer.empty(M * K)
    dA, dB = upload(ow, A.ravel()), upload(ow, B.ravel())
    ow.ops.mat_mul(dA, dB, C, M, N, K)
    got = C.to_host().reshape(M, K)
    sample = np.unique(np.concatenate([np.arange(0, M, 37), [M - 1]]))
    As, B64 = A[sample].astype(np.float64), B.astype(np.float64)
    check_kscaled(got[sample], As @ B64, np.abs(As) @ np.abs(B64), tol=2e-6, floor=0.0)


@pytest.mark.slow
def test_config3_full_size_sampled(ow, orc):
    """Config 3: C = relu(A @ B + bias), M = N = K = 4096, A, B ~ N(0, 1/64), bias ~ U[-0.1, 0.1];
    every 31st row (133 rows x 4096 columns) checked against the oracle."""
    M = N = K = 4096
    orc.set_threads(16)
    dA, dB, dbias, dC = (ow.DeviceBuffer.empty(s) for s in (M * N, N * K, K, M * K))
    ow.fill_normal(dA, SEED, 300, 0.0, 1.0 / 64)
    ow.fill_normal(dB, SEED, 301, 0.0, 1.0 / 64)
    ow.fill_uniform(dbias, SEED, 302, -0.1, 0.1)
    ow.ops.mat_mul_fused(dA, dB, dbias, dC, M, N, K, activation="relu")
    A = orc.fill_normal(M * N, SEED, 300, 0.0, 1.0 / 64, mt=True)
    B = orc.fill_normal(N * K, SEED, 301, 0.0, 1.0 / 64, mt=True)
    bias = orc.fill_uniform(K, SEED, 302, -0.1, 0.1)
    rows = np.arange(0, M, 31)  # 133 rows covering every row residue of the 16- and 256-row tiles
    ref, absdot = orc.mat_mul_rows(A, B, M, N, K, rows=rows, bias=bias, act="relu")
    got = dC.to_host().reshape(M, K)[rows]
    check_kscaled(got, ref, absdot)
    # fp32 arithmetic, not a reduced-precision path: against the float64 product, every element within
    # 1e-6 * (sum_k |a b| + |bias|) and NRMSE <= 5e-6. fp32 accumulation over K = 4096 sits near 1e-7 of
    # that sum; tf32-class inputs (10-bit mantissas) near 1e-5, bf16 inputs near 1e-4.
    exact = np.maximum(A.reshape(M, N)[rows].astype(np.float64) @ B.reshape(N, K).astype(np.float64)
                       + bias.astype(np.float64), 0.0)
    check_kscaled(got, exact, absdot, tol=1e-6, floor=1e-12)
    err = got.astype(np.float64) - exact
    assert float(np.sqrt(np.mean(err ** 2)) / np.sqrt(np.mean(exact ** 2))) <= 5e-6

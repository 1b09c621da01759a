// matrix_multiplication challenge: out(m x k) = a(m x n) * b(n x k), row-major
// (reference adapter: tests/integration/matrix_multiplication.cu:3).
#include "adapter_common.hpp"

extern "C" void solve(const float *a, const float *b, float *out, int m, int n, int k) {
    opworks_adapter::guarded("matrix_multiplication", [&] { opworks::ops::mat_mul(a, b, out, m, n, k); });
}

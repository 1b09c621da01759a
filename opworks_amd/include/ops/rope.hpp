#pragma once

// ops::rope — in-place rotary embedding on x[rows][heads * D] at absolute
// positions pos_start + row (reference: include/ops/rope.cuh:10-46). Pairs
// are (i, i + D/2) (rotate-half); angle = float(pos) * inv_freq[i];
// lo = a cos - b sin, hi = b cos + a sin, each evaluated as one fma over a
// rounded product. inv_freq holds D/2 host-computed frequencies.

#include <limits>
#include <type_traits>

#include "../core/hip_utils.hpp"
#include "elementwise.hpp"

namespace opworks::detail {

__device__ __forceinline__ void rope_rotate(float &a, float &b, float c, float s) {
    const float lo = fmaf(a, c, -(b * s));
    const float hi = fmaf(b, c, a * s);
    a = lo;
    b = hi;
}

// A template (like every kernel in these headers) so that translation units
// that include the header share one definition instead of colliding at link.
template <typename T>
__global__ __launch_bounds__(kThreads) void rope_kernel(T *__restrict__ x, const float *__restrict__ inv_freq,
                                                        int rows, int heads, int D, int pos_start) {
    static_assert(std::is_same_v<T, float>, "rope_kernel is instantiated for float activations only");
    const int half = D / 2;
    OPWORKS_GRID_LOOP(i, int64_t(rows) * heads * half) {
        const int p = static_cast<int>(i % half);
        const int64_t th = i / half; // row * heads + head
        const int row = static_cast<int>(th / heads);
        T *base = x + th * D;
        const float angle = float(pos_start + row) * inv_freq[p];
        float a = base[p], b = base[p + half];
        rope_rotate(a, b, cosf(angle), sinf(angle));
        base[p] = a;
        base[p + half] = b;
    }
}

} // namespace opworks::detail

namespace opworks::ops {

inline void rope(float *x, const float *inv_freq, int rows, int heads, int head_dim, int pos_start,
                 hipStream_t stream = nullptr) {
    detail::validate_size(rows);
    if (rows == 0)
        return;
    detail::require(heads > 0 && head_dim > 0 && head_dim % 2 == 0, "rope requires even positive head_dim");
    detail::require(pos_start >= 0, "rope position must be nonnegative");
    detail::require(x && inv_freq, "rope requires non-null pointers");
    const int64_t pairs = int64_t(rows) * heads * (head_dim / 2);
    detail::require(pairs <= std::numeric_limits<int>::max(), "rope input exceeds the supported INT_MAX pairs");
    detail::require(int64_t(pos_start) + rows <= std::numeric_limits<int>::max(), "rope positions exceed INT_MAX");
    launch_async(stream, detail::rope_kernel<float>, detail::stream_grid(pairs), kThreads, x, inv_freq, rows, heads,
                 head_dim, pos_start);
}

} // namespace opworks::ops

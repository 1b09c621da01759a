#pragma once

// Elementwise steps of the decoder block, on the streaming map kernel:
//   ops::add      out = a + b, in place allowed     (reference: include/ops/add.cuh:7-25)
//   ops::swiglu   out = g / (1 + exp(-g)) * u       (reference: include/ops/swiglu.cuh:7-26)
//   ops::causal_scale   scores *= scale where key <= query position, else -inf
//                                                   (reference: include/ops/causal_scale.cuh:9-33)

#include <cmath>
#include <limits>

#include "elementwise.hpp"

namespace opworks::detail {

struct AddOp {
    static constexpr int kArity = 2;
    __device__ float operator()(float a, float b) const { return a + b; }
};

struct SwigluOp {
    static constexpr int kArity = 2;
    __device__ float operator()(float g, float u) const { return g / (1.f + expf(-g)) * u; }
};

// scores [rows][cols]; query row r sits at absolute position cols - rows + r.
// Each lane owns four consecutive columns of one row when cols % 4 == 0.
template <bool kPacked>
__global__ __launch_bounds__(kThreads) void causal_scale_kernel(float *__restrict__ s, int rows, int cols,
                                                                float scale) {
    const int shift = cols - rows;
    if constexpr (kPacked) {
        const int c4 = cols / 4;
        OPWORKS_GRID_LOOP(i, int64_t(rows) * c4) {
            const int row = static_cast<int>(i / c4);
            const int col = 4 * static_cast<int>(i % c4);
            const int last = shift + row; // last visible key
            f32x4 *p = reinterpret_cast<f32x4 *>(s) + i;
            if (col + 3 <= last) {
                *p = *p * scale;
            } else if (col > last) {
                *p = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            } else {
                f32x4 v = *p;
                v.x = col <= last ? v.x * scale : -INFINITY;
                v.y = col + 1 <= last ? v.y * scale : -INFINITY;
                v.z = col + 2 <= last ? v.z * scale : -INFINITY;
                v.w = -INFINITY; // col + 3 > last here
                *p = v;
            }
        }
    } else {
        OPWORKS_GRID_LOOP(i, int64_t(rows) * cols) {
            const int row = static_cast<int>(i / cols);
            const int col = static_cast<int>(i % cols);
            s[i] = col <= shift + row ? s[i] * scale : -INFINITY;
        }
    }
}

inline void check_flat_size(int64_t n, const char *what) {
    require(n >= 0, what);
    require(n <= std::numeric_limits<int>::max(), "input exceeds the supported INT_MAX elements");
}

} // namespace opworks::detail

namespace opworks::ops {

inline void add(const float *a, const float *b, float *out, int64_t n, hipStream_t stream = nullptr) {
    detail::check_flat_size(n, "add size must be nonnegative");
    if (n == 0)
        return;
    detail::require(a && b && out, "add requires non-null pointers");
    map(a, b, out, static_cast<int>(n), detail::AddOp{}, stream);
}

inline void swiglu(const float *gate, const float *up, float *out, int64_t n, hipStream_t stream = nullptr) {
    detail::check_flat_size(n, "swiglu size must be nonnegative");
    if (n == 0)
        return;
    detail::require(gate && up && out, "swiglu requires non-null pointers");
    map(gate, up, out, static_cast<int>(n), detail::SwigluOp{}, stream);
}

inline void causal_scale(float *scores, int rows, int cols, float scale, hipStream_t stream = nullptr) {
    detail::validate_matrix(rows, cols);
    if (rows == 0)
        return;
    detail::require(cols >= rows, "causal scores need at least as many keys as queries");
    detail::require(scores && scale > 0.f, "causal_scale requires a buffer and a positive scale");
    if (cols % 4 == 0 && detail::aligned16(scores))
        launch_async(stream, detail::causal_scale_kernel<true>, detail::stream_grid(int64_t(rows) * cols / 4),
                     kThreads, scores, rows, cols, scale);
    else
        launch_async(stream, detail::causal_scale_kernel<false>, detail::stream_grid(int64_t(rows) * cols), kThreads,
                     scores, rows, cols, scale);
}

} // namespace opworks::ops

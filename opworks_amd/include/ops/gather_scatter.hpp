#pragma once

// ops::gather and ops::scatter — the kernels behind GatherScatterBuilder (the
// reference's builder carries input, output, int32 indices, count and the
// operation, include/builders/gather_scatter.cuh:7-30, and ships no kernel).
//
//   gather:  out[i] = in[idx[i]]   for i < count; an index outside
//            [0, in_size) writes a quiet NaN instead of reading out of bounds;
//   scatter: out[idx[i]] = in[i]   for i < count; an index outside
//            [0, out_size) is skipped. When several i share one index, which
//            of them lands is unspecified (they race, as in any parallel
//            scatter without a combine).
//
// gfx950 design: HBM-bound, one pass. A lane handles four consecutive i, so
// the index and the contiguous side move as 16-byte packs when their pointers
// allow; the indexed side is one 4-byte access per element (a random index
// stream costs a whole memory sector per element on that side).

#include <cmath>
#include <cstdint>

#include "../core/hip_utils.hpp"
#include "elementwise.hpp" // f32x4, aligned16, stream_grid

namespace opworks::detail {

using i32x4 = int __attribute__((ext_vector_type(4)));

template <bool kVec>
__global__ __launch_bounds__(kThreads) void gather_kernel(const float *__restrict__ in, int64_t in_size,
                                                          const int *__restrict__ idx, float *__restrict__ out,
                                                          int64_t count) {
    const float nan = __builtin_nanf("");
    for (int64_t q = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; 4 * q < count;
         q += int64_t(gridDim.x) * blockDim.x) {
        const int64_t i = 4 * q;
        if (kVec && i + 4 <= count) {
            const i32x4 j = *reinterpret_cast<const i32x4 *>(idx + i);
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[e] = (j[e] >= 0 && j[e] < in_size) ? in[j[e]] : nan;
            *reinterpret_cast<f32x4 *>(out + i) = v;
        } else {
            for (int64_t k = i; k < i + 4 && k < count; ++k) {
                const int j = idx[k];
                out[k] = (j >= 0 && j < in_size) ? in[j] : nan;
            }
        }
    }
}

template <bool kVec>
__global__ __launch_bounds__(kThreads) void scatter_kernel(const float *__restrict__ in, const int *__restrict__ idx,
                                                           float *__restrict__ out, int64_t out_size,
                                                           int64_t count) {
    for (int64_t q = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; 4 * q < count;
         q += int64_t(gridDim.x) * blockDim.x) {
        const int64_t i = 4 * q;
        if (kVec && i + 4 <= count) {
            const i32x4 j = *reinterpret_cast<const i32x4 *>(idx + i);
            const f32x4 v = *reinterpret_cast<const f32x4 *>(in + i);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (j[e] >= 0 && j[e] < out_size)
                    out[j[e]] = v[e];
        } else {
            for (int64_t k = i; k < i + 4 && k < count; ++k) {
                const int j = idx[k];
                if (j >= 0 && j < out_size)
                    out[j] = in[k];
            }
        }
    }
}

} // namespace opworks::detail

namespace opworks::ops {

// out[i] = in[idx[i]] (NaN for an index outside [0, in_size)), i < count.
inline void gather(const float *in, int64_t in_size, const int *idx, float *out, int count,
                   hipStream_t stream = nullptr) {
    detail::validate_size(count);
    detail::require(in_size >= 0, "gather input size must be nonnegative");
    if (count == 0)
        return;
    detail::require(idx && out && (in || in_size == 0), "gather requires non-null pointers");
    const int grid = detail::stream_grid(detail::blocks_for64(count, 4));
    if (detail::aligned16(idx) && detail::aligned16(out))
        launch_async(stream, detail::gather_kernel<true>, grid, kThreads, in, in_size, idx, out, int64_t(count));
    else
        launch_async(stream, detail::gather_kernel<false>, grid, kThreads, in, in_size, idx, out, int64_t(count));
}

// out[idx[i]] = in[i] for i < count; indices outside [0, out_size) are skipped.
inline void scatter(const float *in, const int *idx, float *out, int64_t out_size, int count,
                    hipStream_t stream = nullptr) {
    detail::validate_size(count);
    detail::require(out_size >= 0, "scatter output size must be nonnegative");
    if (count == 0)
        return;
    detail::require(in && idx && (out || out_size == 0), "scatter requires non-null pointers");
    const int grid = detail::stream_grid(detail::blocks_for64(count, 4));
    if (detail::aligned16(idx) && detail::aligned16(in))
        launch_async(stream, detail::scatter_kernel<true>, grid, kThreads, in, idx, out, out_size, int64_t(count));
    else
        launch_async(stream, detail::scatter_kernel<false>, grid, kThreads, in, idx, out, out_size, int64_t(count));
}

} // namespace opworks::ops

#pragma once

// bf16-weight linear layers on the matrix cores.
//  * ops::linear_mma_bf16(X fp32, W bf16, Y): Y = bf16(X) @ W^T, fp32 accumulate
//    (reference: include/ops/linear_mma.cuh:99-115);
//  * ops::linear_bf16_fused: the same with a bias + activation epilogue, and
//    with X given either as fp32 or as bf16;
//  * ops::convert_f32_to_bf16: nearest-even rounding of an fp32 array.

#include <type_traits>

#include "../core/bf16.hpp"
#include "../core/hip_utils.hpp"
#include "gemm_bf16.hpp"
#include "matmul.hpp"

namespace opworks::detail {

__global__ __launch_bounds__(256) static void convert_f32_bf16_kernel(const float *__restrict__ src,
                                                                      uint16_t *__restrict__ dst, int64_t n) {
    OPWORKS_GRID_LOOP(i, n) { dst[i] = float_to_bf16_rne(src[i]); }
}

template <typename TA>
inline void linear_bf16_validate(const TA *X, const uint16_t *W, float *Y, int rows, int in_features,
                                 int out_features) {
    validate_matrix(rows, in_features);
    validate_matrix(out_features, in_features);
    validate_matrix(rows, out_features);
    if (rows == 0 || out_features == 0)
        return;
    require(X && W && Y, "linear_mma_bf16 requires non-null pointers");
    require(in_features > 0, "linear_mma_bf16 requires a positive reduction dim");
}

// fp32 X: the register-staged GEMM (rounded as staged); bf16 X: the direct-load GEMM on tiles
// sized to the row count (no workspace, so no split-K).
template <typename TA, typename Epi>
inline void linear_bf16_launch(const TA *X, const uint16_t *W, const float *bias, float *Y, int rows, int in_features,
                               int out_features, Epi epi, hipStream_t stream) {
    if constexpr (std::is_same_v<TA, uint16_t>)
        gemm_bf16_launch_direct<Epi, GemmStore::store>(X, W, bias, Y, rows, out_features, in_features, epi, nullptr, 0,
                                                       stream);
    else
        gemm_bf16_launch(X, W, bias, Y, rows, out_features, in_features, epi, stream);
}

template <typename TA>
inline void linear_bf16_act(const TA *X, const uint16_t *W, const float *bias, float *Y, int rows, int in_features,
                            int out_features, ops::Activation act, hipStream_t stream) {
    linear_bf16_validate(X, W, Y, rows, in_features, out_features);
    if (rows == 0 || out_features == 0)
        return;
    switch (act) {
    case ops::Activation::none:
        linear_bf16_launch(X, W, bias, Y, rows, in_features, out_features, ops::PassThrough{}, stream);
        break;
    case ops::Activation::relu:
        linear_bf16_launch(X, W, bias, Y, rows, in_features, out_features, ops::ReluEpilogue{}, stream);
        break;
    case ops::Activation::gelu:
        linear_bf16_launch(X, W, bias, Y, rows, in_features, out_features, ops::GeluEpilogue{}, stream);
        break;
    default: throw std::invalid_argument("unknown activation");
    }
}

} // namespace opworks::detail

namespace opworks::ops {

inline void linear_mma_bf16(const float *X, const bf16 *W, float *Y, int rows, int in_features, int out_features,
                            hipStream_t stream = nullptr) {
    detail::linear_bf16_act(X, reinterpret_cast<const uint16_t *>(W), nullptr, Y, rows, in_features, out_features,
                            Activation::none, stream);
}

inline void linear_bf16_fused(const float *X, const bf16 *W, const float *bias, float *Y, int rows, int in_features,
                              int out_features, Activation act, hipStream_t stream = nullptr) {
    detail::linear_bf16_act(X, reinterpret_cast<const uint16_t *>(W), bias, Y, rows, in_features, out_features, act,
                            stream);
}

inline void linear_bf16_fused(const bf16 *X, const bf16 *W, const float *bias, float *Y, int rows, int in_features,
                              int out_features, Activation act, hipStream_t stream = nullptr) {
    detail::linear_bf16_act(reinterpret_cast<const uint16_t *>(X), reinterpret_cast<const uint16_t *>(W), bias, Y,
                            rows, in_features, out_features, act, stream);
}

inline void convert_f32_to_bf16(const float *src, bf16 *dst, int64_t n, hipStream_t stream = nullptr) {
    detail::require(n >= 0, "size must be nonnegative");
    if (n == 0)
        return;
    detail::require(src && dst, "convert requires non-null pointers");
    launch_async(stream, detail::convert_f32_bf16_kernel, detail::stream_grid(n), 256, src,
                 reinterpret_cast<uint16_t *>(dst), n);
}

} // namespace opworks::ops

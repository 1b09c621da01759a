#pragma once

// ops::linear — Y[rows, out] = X[rows, in] @ W[out, in]^T with weights in the
// HF [out, in] layout (reference: include/ops/linear.cuh:125-153).
//  * rows >= 2: the fp32 MFMA GEMM with the k-contiguous (nk) B layout;
//  * rows == 1: an HBM-bound GEMV. Each wave owns kGemvRows output rows and
//    streams them with 16-byte loads (kGemvUnroll packs per row per lane in
//    flight); x is read through the cache once per wave; one DPP reduction
//    per row. One weight byte is read once per call.

#include "../core/hip_utils.hpp"
#include "../core/wave.hpp"
#include "gemm_f32.hpp"

namespace opworks::detail {

constexpr int kGemvRows = 4;
constexpr int kGemvUnroll = 4;
constexpr int kGemvThreads = 256;

// y[o] = dot(x, W[o, :]) for o in [0, out); in % 4 == 0 and 16-byte aligned W, x.
__global__ __launch_bounds__(kGemvThreads) static void gemv_f32_kernel(const float *__restrict__ x,
                                                                       const float *__restrict__ W,
                                                                       float *__restrict__ y, int in, int out) {
    const int lane = threadIdx.x % kWaveSize;
    const int wave_global = blockIdx.x * (kGemvThreads / kWaveSize) + threadIdx.x / kWaveSize;
    const int row0 = wave_global * kGemvRows;
    if (row0 >= out)
        return;
    const int n4 = in / 4;
    const f32x4 *x4 = reinterpret_cast<const f32x4 *>(x);
    float acc[kGemvRows] = {};
    const f32x4 *w4[kGemvRows];
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
        w4[r] = reinterpret_cast<const f32x4 *>(W + int64_t(row0 + r < out ? row0 + r : row0) * in);
    for (int base = lane; base < n4; base += kWaveSize * kGemvUnroll) {
        f32x4 wv[kGemvRows][kGemvUnroll], xv[kGemvUnroll];
#pragma unroll
        for (int u = 0; u < kGemvUnroll; ++u) {
            const int c = base + u * kWaveSize;
            if (c < n4) {
                xv[u] = x4[c];
#pragma unroll
                for (int r = 0; r < kGemvRows; ++r)
                    wv[r][u] = __builtin_nontemporal_load(w4[r] + c);
            }
        }
#pragma unroll
        for (int u = 0; u < kGemvUnroll; ++u) {
            if (base + u * kWaveSize < n4) {
#pragma unroll
                for (int r = 0; r < kGemvRows; ++r) {
                    acc[r] = fmaf(wv[r][u][0], xv[u][0], acc[r]);
                    acc[r] = fmaf(wv[r][u][1], xv[u][1], acc[r]);
                    acc[r] = fmaf(wv[r][u][2], xv[u][2], acc[r]);
                    acc[r] = fmaf(wv[r][u][3], xv[u][3], acc[r]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r) {
        const float s = wave::sum(acc[r]);
        if (lane == 0 && row0 + r < out)
            y[row0 + r] = s;
    }
}

// Any alignment / width: one wave per output row, scalar loads.
__global__ __launch_bounds__(kGemvThreads) static void gemv_f32_scalar_kernel(const float *__restrict__ x,
                                                                              const float *__restrict__ W,
                                                                              float *__restrict__ y, int in,
                                                                              int out) {
    const int lane = threadIdx.x % kWaveSize;
    const int row = blockIdx.x * (kGemvThreads / kWaveSize) + threadIdx.x / kWaveSize;
    if (row >= out)
        return;
    const float *w = W + int64_t(row) * in;
    float acc = 0.f;
    for (int i = lane; i < in; i += kWaveSize)
        acc = fmaf(w[i], x[i], acc);
    acc = wave::sum(acc);
    if (lane == 0)
        y[row] = acc;
}

inline void gemv_f32_launch(const float *x, const float *W, float *y, int in, int out, hipStream_t stream) {
    constexpr int waves_per_block = kGemvThreads / kWaveSize;
    if (in % 4 == 0 && aligned16(x) && aligned16(W)) {
        const int waves = static_cast<int>(blocks_for64(out, kGemvRows));
        launch_async(stream, gemv_f32_kernel, static_cast<int>(blocks_for64(waves, waves_per_block)), kGemvThreads,
                     x, W, y, in, out);
    } else {
        launch_async(stream, gemv_f32_scalar_kernel, static_cast<int>(blocks_for64(out, waves_per_block)),
                     kGemvThreads, x, W, y, in, out);
    }
}

} // namespace opworks::detail

namespace opworks::ops {

inline void linear(const float *X, const float *W, float *Y, int rows, int in_features, int out_features,
                   hipStream_t stream = nullptr) {
    detail::validate_matrix(rows, in_features);
    detail::validate_matrix(out_features, in_features);
    detail::validate_matrix(rows, out_features);
    if (rows == 0 || out_features == 0)
        return;
    detail::require(X && W && Y, "linear requires non-null pointers");
    detail::require(in_features > 0, "linear requires a positive reduction dim");
    if (rows == 1) {
        detail::gemv_f32_launch(X, W, Y, in_features, out_features, stream);
        return;
    }
    detail::gemm_f32_launch<detail::BLayout::nk>(X, W, nullptr, Y, rows, out_features, in_features,
                                                 detail::IdentityEpilogue{}, stream);
}

} // namespace opworks::ops

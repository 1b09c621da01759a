#pragma once

// ops::linear<WT> — Y[rows, out] = X[rows, in] @ W[out, in]^T with weights in
// the HF [out, in] layout, WT = float or bf16; X, Y and the accumulation are
// fp32 and bf16 weights are widened exactly (reference: template ops::linear,
// include/ops/linear.cuh:125-153, with its rows == 1 GEMVs at :77-121).
//  * rows >= 2: the fp32 MFMA GEMM with the k-contiguous (nk) B layout; a
//    bf16 B operand is widened to fp32 while it is staged in LDS;
//  * rows == 1: an HBM-bound GEMV. Each wave owns kGemvRows output rows and
//    streams them in 16-byte weight packs (4 fp32 or 8 bf16), kGemvUnroll
//    packs per row per lane in flight; x is read through the cache once per
//    wave; one DPP reduction per row. Each weight byte is read once per call.
// This is the fp32-input path at every row count; the bf16-input matrix-core
// path is ops::linear_mma_bf16 (ops/linear_bf16.hpp).

#include <type_traits>

#include "../core/hip_utils.hpp"
#include "../core/wave.hpp"
#include "../core/weight_pack.hpp"
#include "gemm_f32.hpp"

namespace opworks::detail {

constexpr int kGemvRows = 4;
constexpr int kGemvUnroll = 4;
constexpr int kGemvThreads = 256;

// y[o] = dot(x, W[o, :]) for o in [0, out); in % WPack<WT>::kElems == 0 and
// 16-byte aligned W, x.
template <typename WT>
__global__ __launch_bounds__(kGemvThreads) static void gemv_kernel(const float *__restrict__ x,
                                                                   const WT *__restrict__ W, float *__restrict__ y,
                                                                   int in, int out) {
    constexpr int E = WPack<WT>::kElems;
    using Pack = typename WPack<WT>::type;
    const int lane = threadIdx.x % kWaveSize;
    const int wave_global = blockIdx.x * (kGemvThreads / kWaveSize) + threadIdx.x / kWaveSize;
    const int row0 = wave_global * kGemvRows;
    if (row0 >= out)
        return;
    const int packs = in / E;
    const f32x4 *x4 = reinterpret_cast<const f32x4 *>(x);
    float acc[kGemvRows] = {};
    const WT *rows[kGemvRows];
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
        rows[r] = W + int64_t(row0 + r < out ? row0 + r : row0) * in;
    for (int base = lane; base < packs; base += kWaveSize * kGemvUnroll) {
        Pack wv[kGemvRows][kGemvUnroll];
        f32x4 xv[kGemvUnroll][E / 4];
#pragma unroll
        for (int u = 0; u < kGemvUnroll; ++u) {
            const int c = base + u * kWaveSize;
            if (c < packs) {
#pragma unroll
                for (int q = 0; q < E / 4; ++q)
                    xv[u][q] = x4[int64_t(c) * (E / 4) + q];
#pragma unroll
                for (int r = 0; r < kGemvRows; ++r)
                    wv[r][u] = load_wpack(rows[r], c);
            }
        }
#pragma unroll
        for (int u = 0; u < kGemvUnroll; ++u) {
            if (base + u * kWaveSize < packs) {
#pragma unroll
                for (int r = 0; r < kGemvRows; ++r)
                    acc[r] = dot_wpack<WT>(wv[r][u], xv[u], acc[r]);
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
template <typename WT>
__global__ __launch_bounds__(kGemvThreads) static void gemv_scalar_kernel(const float *__restrict__ x,
                                                                          const WT *__restrict__ W,
                                                                          float *__restrict__ y, int in, int out) {
    const int lane = threadIdx.x % kWaveSize;
    const int row = blockIdx.x * (kGemvThreads / kWaveSize) + threadIdx.x / kWaveSize;
    if (row >= out)
        return;
    const WT *w = W + int64_t(row) * in;
    float acc = 0.f;
    for (int i = lane; i < in; i += kWaveSize)
        acc = fmaf(widen(w[i]), x[i], acc);
    acc = wave::sum(acc);
    if (lane == 0)
        y[row] = acc;
}

template <typename WT>
inline void gemv_launch(const float *x, const WT *W, float *y, int in, int out, hipStream_t stream) {
    constexpr int waves_per_block = kGemvThreads / kWaveSize;
    if (in % WPack<WT>::kElems == 0 && aligned16(x) && aligned16(W)) {
        const int64_t waves = blocks_for64(out, kGemvRows);
        launch_async(stream, gemv_kernel<WT>, static_cast<int>(blocks_for64(waves, waves_per_block)), kGemvThreads, x,
                     W, y, in, out);
    } else {
        launch_async(stream, gemv_scalar_kernel<WT>, static_cast<int>(blocks_for64(out, waves_per_block)),
                     kGemvThreads, x, W, y, in, out);
    }
}

} // namespace opworks::detail

namespace opworks::ops {

template <typename WT>
inline void linear(const float *X, const WT *W, float *Y, int rows, int in_features, int out_features,
                   hipStream_t stream = nullptr) {
    static_assert(std::is_same_v<WT, float> || std::is_same_v<WT, bf16>, "linear weights are float or bf16");
    detail::validate_matrix(rows, in_features);
    detail::validate_matrix(out_features, in_features);
    detail::validate_matrix(rows, out_features);
    if (rows == 0 || out_features == 0)
        return;
    detail::require(X && W && Y, "linear requires non-null pointers");
    detail::require(in_features > 0, "linear requires a positive reduction dim");
    if (rows == 1) {
        detail::gemv_launch<WT>(X, W, Y, in_features, out_features, stream);
        return;
    }
    using detail::BLayout;
    using detail::IdentityEpilogue;
    if constexpr (std::is_same_v<WT, float>)
        detail::gemm_f32_launch<BLayout::nk>(X, W, nullptr, Y, rows, out_features, in_features, IdentityEpilogue{},
                                             stream);
    else
        detail::gemm_f32_launch<BLayout::nk, IdentityEpilogue, detail::GemmStore::store, uint16_t>(
            X, reinterpret_cast<const uint16_t *>(W), nullptr, Y, rows, out_features, in_features, IdentityEpilogue{},
            stream);
}

} // namespace opworks::ops

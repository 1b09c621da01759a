#pragma once

// ops::argmax — index of the largest of x[0..n) into out[0] on the device
// (reference: include/ops/argmax.cuh:9-63). Ties go to the lowest index, NaN
// never wins, and an all-NaN input yields 0x7fffffff. The order of combining
// does not change the result (value first, then lowest index), so one
// 1024-lane workgroup reads x with 16-byte loads, eight in flight per lane.

#include <cmath>

#include "../core/hip_utils.hpp"
#include "elementwise.hpp"

namespace opworks::detail {

__device__ __forceinline__ void argmax_merge(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

__device__ __forceinline__ void wave_argmax(float &v, int &i) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(v, off);
        const int i2 = __shfl_xor(i, off);
        argmax_merge(v, i, v2, i2);
    }
}

// Combines one (value, index) per lane of a workgroup of kWaves waves; the
// winner is returned to every lane.
template <int kWaves> __device__ __forceinline__ int workgroup_argmax(float v, int i) {
    __shared__ float sv[kWaves];
    __shared__ int si[kWaves];
    __shared__ int winner;
    wave_argmax(v, i);
    const int wave = threadIdx.x / kWaveSize;
    if (threadIdx.x % kWaveSize == 0) {
        sv[wave] = v;
        si[wave] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kWaves; ++w)
            argmax_merge(v, i, sv[w], si[w]);
        winner = i;
    }
    __syncthreads();
    return winner;
}

constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxBatch = 8;

template <bool kPacked>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float *__restrict__ x, int n, int *out) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if constexpr (kPacked) {
        const int n4 = n / 4;
        const f32x4 *x4 = reinterpret_cast<const f32x4 *>(x);
        for (int base = threadIdx.x; base < n4; base += kArgmaxThreads * kArgmaxBatch) {
            f32x4 v[kArgmaxBatch];
#pragma unroll
            for (int u = 0; u < kArgmaxBatch; ++u) {
                const int j = base + u * kArgmaxThreads;
                v[u] = j < n4 ? __builtin_nontemporal_load(x4 + j) : f32x4{NAN, NAN, NAN, NAN};
            }
#pragma unroll
            for (int u = 0; u < kArgmaxBatch; ++u) {
                const int j = 4 * (base + u * kArgmaxThreads);
                argmax_merge(bv, bi, v[u].x, j);
                argmax_merge(bv, bi, v[u].y, j + 1);
                argmax_merge(bv, bi, v[u].z, j + 2);
                argmax_merge(bv, bi, v[u].w, j + 3);
            }
        }
        for (int j = 4 * n4 + threadIdx.x; j < n; j += kArgmaxThreads)
            argmax_merge(bv, bi, x[j], j);
    } else {
        for (int j = threadIdx.x; j < n; j += kArgmaxThreads)
            argmax_merge(bv, bi, x[j], j);
    }
    const int w = workgroup_argmax<kArgmaxThreads / kWaveSize>(bv, bi);
    if (threadIdx.x == 0)
        out[0] = w;
}

} // namespace opworks::detail

namespace opworks::ops {

inline void argmax(const float *x, int n, int *out, hipStream_t stream = nullptr) {
    detail::require(n > 0, "argmax requires a nonempty input");
    detail::require(x && out, "argmax requires non-null pointers");
    if (detail::aligned16(x))
        launch_async(stream, detail::argmax_kernel<true>, 1, detail::kArgmaxThreads, x, n, out);
    else
        launch_async(stream, detail::argmax_kernel<false>, 1, detail::kArgmaxThreads, x, n, out);
}

} // namespace opworks::ops

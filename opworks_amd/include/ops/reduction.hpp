#pragma once

// ops::reduce<Op> — full reduction of an fp32 array to one value
// (reference API: include/ops/reduction.cuh:31-67; functor contract: static
// identity() and an associative, commutative combine()).
//
// gfx950 design: two launches, no atomics, deterministic for a given n.
//  1. reduce_partial_kernel: G workgroups stream the input with 16-byte loads,
//     kReduceUnroll independent accumulators per lane, then a DPP wave
//     reduction and an LDS step per workgroup -> partial[b].
//  2. reduce_final_kernel: one workgroup combines the G partials in fixed order.
// G depends only on n, so results are bit-reproducible run to run. Inputs with
// at most one workgroup's worth of work use a single launch and no workspace.
// Empty input writes Op::identity().

#include "../core/block_reduce.hpp"
#include "../core/device_span.hpp"
#include "../core/hip_utils.hpp"
#include "elementwise.hpp"

namespace opworks::detail {

constexpr int kReduceUnroll = 4;
constexpr int kReduceMaxPartials = 1024;
constexpr int kReducePerBlock = kThreads * 4 * kReduceUnroll; // elements per workgroup per sweep

template <typename Op> struct FunctorCombine {
    __device__ float operator()(float a, float b) const { return Op::combine(a, b); }
};

// Reduces `v` over the workgroup; the result is valid in every lane of wave 0.
template <typename Op> __device__ __forceinline__ float workgroup_reduce(float v) {
    __shared__ float partials[kMaxWavesPerBlock];
    const int wid = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    const int nwaves = blockDim.x / kWaveSize;
    v = wave::reduce(v, Op::identity(), FunctorCombine<Op>{});
    if (lane == 0)
        partials[wid] = v;
    __syncthreads();
    float r = Op::identity();
    if (wid == 0) {
        for (int k = 0; k < nwaves; ++k) // fixed order
            r = Op::combine(r, partials[k]);
    }
    return r;
}

template <typename Op, bool kPacked>
__global__ __launch_bounds__(kThreads) void reduce_partial_kernel(const float *__restrict__ in,
                                                                  float *__restrict__ partial, int n) {
    float acc[kReduceUnroll];
#pragma unroll
    for (int u = 0; u < kReduceUnroll; ++u)
        acc[u] = Op::identity();
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if constexpr (kPacked) {
        const int64_t n_pack = n / 4;
        const f32x4 *p = reinterpret_cast<const f32x4 *>(in);
        for (; i + (kReduceUnroll - 1) * stride < n_pack; i += kReduceUnroll * stride) {
            f32x4 v[kReduceUnroll];
#pragma unroll
            for (int u = 0; u < kReduceUnroll; ++u)
                v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
            for (int u = 0; u < kReduceUnroll; ++u)
                acc[u] = Op::combine(acc[u], Op::combine(Op::combine(v[u][0], v[u][1]), Op::combine(v[u][2], v[u][3])));
        }
        for (; i < n_pack; i += stride) {
            f32x4 v = p[i];
            acc[0] = Op::combine(acc[0], Op::combine(Op::combine(v[0], v[1]), Op::combine(v[2], v[3])));
        }
        const int tail = n - static_cast<int>(4 * n_pack);
        if (blockIdx.x == 0 && static_cast<int>(threadIdx.x) < tail)
            acc[1] = Op::combine(acc[1], in[4 * n_pack + threadIdx.x]);
    } else {
        for (; i + (kReduceUnroll - 1) * stride < n; i += kReduceUnroll * stride) {
            float v[kReduceUnroll];
#pragma unroll
            for (int u = 0; u < kReduceUnroll; ++u)
                v[u] = in[i + u * stride];
#pragma unroll
            for (int u = 0; u < kReduceUnroll; ++u)
                acc[u] = Op::combine(acc[u], v[u]);
        }
        for (; i < n; i += stride)
            acc[0] = Op::combine(acc[0], in[i]);
    }
    float a = Op::combine(Op::combine(acc[0], acc[1]), Op::combine(acc[2], acc[3]));
    a = workgroup_reduce<Op>(a);
    if (threadIdx.x == 0)
        partial[blockIdx.x] = a;
}

template <typename Op>
__global__ __launch_bounds__(kThreads) void reduce_final_kernel(const float *__restrict__ partial,
                                                                float *__restrict__ out, int count) {
    float acc = Op::identity();
    for (int i = threadIdx.x; i < count; i += blockDim.x)
        acc = Op::combine(acc, partial[i]);
    acc = workgroup_reduce<Op>(acc);
    if (threadIdx.x == 0)
        out[0] = acc;
}

inline int reduce_partial_count(int n) {
    const int need = static_cast<int>(blocks_for64(n, kReducePerBlock));
    return need < kReduceMaxPartials ? need : kReduceMaxPartials;
}

} // namespace opworks::detail

namespace opworks::ops {

// Workspace size in floats; 0 when one launch suffices.
inline int reduction_workspace_size(int n) {
    detail::validate_size(n);
    const int g = detail::reduce_partial_count(n);
    return g <= 1 ? 0 : g;
}

// Allocation-free asynchronous path; capturable into a HIP graph. The
// workspace must stay alive until the stream completes and must not overlap
// the input, the output or a concurrent reduction.
template <typename Op>
inline void reduce(const float *in, float *out, int n, DeviceSpan<float> workspace, hipStream_t stream = nullptr) {
    const int blocks = reduction_workspace_size(n);
    detail::require(out && (n == 0 || in), "reduction requires valid input/output pointers");
    detail::require(workspace.size() >= blocks, "reduction workspace is too small");
    const bool packed = detail::aligned16(in);
    if (blocks == 0) {
        if (packed)
            launch_async(stream, detail::reduce_partial_kernel<Op, true>, 1, kThreads, in, out, n);
        else
            launch_async(stream, detail::reduce_partial_kernel<Op, false>, 1, kThreads, in, out, n);
        return;
    }
    if (packed)
        launch_async(stream, detail::reduce_partial_kernel<Op, true>, blocks, kThreads, in, workspace.data(), n);
    else
        launch_async(stream, detail::reduce_partial_kernel<Op, false>, blocks, kThreads, in, workspace.data(), n);
    launch_async(stream, detail::reduce_final_kernel<Op>, 1, kThreads, workspace.data(), out, blocks);
}

// Convenience path: stream-ordered scratch (hipMallocAsync / hipFreeAsync).
template <typename Op> inline void reduce(const float *in, float *out, int n, hipStream_t stream = nullptr) {
    const int count = reduction_workspace_size(n);
    detail::require(out && (n == 0 || in), "reduction requires valid input/output pointers");
    float *scratch = nullptr;
    if (count != 0)
        OPWORKS_HIP_CHECK(hipMallocAsync(reinterpret_cast<void **>(&scratch), sizeof(float) * count, stream));
    reduce<Op>(in, out, n, DeviceSpan<float>(scratch, count), stream);
    if (scratch)
        OPWORKS_HIP_CHECK(hipFreeAsync(scratch, stream));
}

} // namespace opworks::ops

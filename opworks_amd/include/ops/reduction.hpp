#pragma once

// ops::reduce<Op> — full reduction of an fp32 array to one value
// (reference API: include/ops/reduction.cuh:31-67; functor contract: static
// identity() and an associative, commutative combine()).
//
// gfx950 design: two launches, no atomics, deterministic for a given n.
//  1. reduce_partial_kernel: workgroup b streams the contiguous chunk
//     [b * kReduceChunk, (b+1) * kReduceChunk) with non-temporal 16-byte loads
//     (kReduceUnroll packs per lane, all issued before any add), reduces it
//     with DPP inside each wave and a fixed-order LDS step -> partial[b].
//     Short-lived workgroups over adjacent chunks stream HBM at ~88% of peak
//     on MI355X, against ~66% for a persistent grid-stride loop.
//  2. reduce_final_kernel: one 1024-thread workgroup combines the partials in
//     a fixed order.
// The geometry depends only on n, so results are bit-reproducible run to run.
// Inputs of at most one chunk use a single launch and no workspace. Empty
// input writes Op::identity().

#include "../core/block_reduce.hpp"
#include "../core/device_span.hpp"
#include "../core/hip_utils.hpp"
#include "elementwise.hpp" // f32x4, aligned16

namespace opworks::detail {

constexpr int kReduceThreads = 512;
constexpr int kReduceUnroll = 4;                                    // 16-byte packs per lane
constexpr int kReduceChunk = kReduceThreads * 4 * kReduceUnroll;    // elements per workgroup (8192)
constexpr int kReduceFinalThreads = 1024;

template <typename Op> struct FunctorCombine {
    __device__ float operator()(float a, float b) const { return Op::combine(a, b); }
};

// Reduces `v` over the workgroup (blockDim a multiple of 64); the result is
// valid in every lane of wave 0. Partials are combined in wave order.
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
        for (int k = 0; k < nwaves; ++k)
            r = Op::combine(r, partials[k]);
    }
    return r;
}

template <typename Op>
__device__ __forceinline__ float combine4(float acc, const f32x4 &v) {
    return Op::combine(acc, Op::combine(Op::combine(v[0], v[1]), Op::combine(v[2], v[3])));
}

template <typename Op, bool kPacked>
__global__ __launch_bounds__(kReduceThreads) void reduce_partial_kernel(const float *__restrict__ in,
                                                                        float *__restrict__ partial, int n) {
    float acc = Op::identity();
    if constexpr (kPacked) {
        const int64_t n_pack = n / 4;
        const f32x4 *p = reinterpret_cast<const f32x4 *>(in);
        constexpr int kPacksPerBlock = kReduceChunk / 4;
        for (int64_t base = static_cast<int64_t>(blockIdx.x) * kPacksPerBlock + threadIdx.x; base < n_pack;
             base += static_cast<int64_t>(gridDim.x) * kPacksPerBlock) {
            f32x4 v[kReduceUnroll];
#pragma unroll
            for (int u = 0; u < kReduceUnroll; ++u) {
                const int64_t i = base + u * kReduceThreads;
                if (i < n_pack)
                    v[u] = __builtin_nontemporal_load(p + i);
            }
#pragma unroll
            for (int u = 0; u < kReduceUnroll; ++u)
                if (base + u * kReduceThreads < n_pack)
                    acc = combine4<Op>(acc, v[u]);
        }
        const int tail = n - static_cast<int>(4 * n_pack);
        if (blockIdx.x == 0 && static_cast<int>(threadIdx.x) < tail)
            acc = Op::combine(acc, in[4 * n_pack + threadIdx.x]);
    } else {
        for (int64_t base = static_cast<int64_t>(blockIdx.x) * kReduceChunk; base < n;
             base += static_cast<int64_t>(gridDim.x) * kReduceChunk) {
            const int64_t end = base + kReduceChunk < n ? base + kReduceChunk : n;
            for (int64_t i = base + threadIdx.x; i < end; i += kReduceThreads)
                acc = Op::combine(acc, in[i]);
        }
    }
    acc = workgroup_reduce<Op>(acc);
    if (threadIdx.x == 0)
        partial[blockIdx.x] = acc;
}

// Every lane issues all of its partial loads (16-byte when aligned) before
// combining, so the pass costs about one memory latency.
template <typename Op>
__global__ __launch_bounds__(kReduceFinalThreads) void reduce_final_kernel(const float *__restrict__ partial,
                                                                          float *__restrict__ out, int count) {
    constexpr int kBatch = 8;
    float acc = Op::identity();
    if ((reinterpret_cast<uintptr_t>(partial) & 15u) == 0) {
        const int n4 = count / 4;
        const f32x4 *p = reinterpret_cast<const f32x4 *>(partial);
        for (int base = threadIdx.x; base < n4; base += kBatch * kReduceFinalThreads) {
            f32x4 v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (base + u * kReduceFinalThreads < n4)
                    v[u] = p[base + u * kReduceFinalThreads];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (base + u * kReduceFinalThreads < n4)
                    acc = combine4<Op>(acc, v[u]);
        }
        if (static_cast<int>(threadIdx.x) < count - 4 * n4)
            acc = Op::combine(acc, partial[4 * n4 + threadIdx.x]);
    } else {
        for (int i = threadIdx.x; i < count; i += kReduceFinalThreads)
            acc = Op::combine(acc, partial[i]);
    }
    acc = workgroup_reduce<Op>(acc);
    if (threadIdx.x == 0)
        out[0] = acc;
}

inline int reduce_partial_count(int n) { return static_cast<int>(blocks_for64(n, kReduceChunk)); }

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
    constexpr int T = detail::kReduceThreads;
    if (blocks == 0) {
        if (packed)
            launch_async(stream, detail::reduce_partial_kernel<Op, true>, 1, T, in, out, n);
        else
            launch_async(stream, detail::reduce_partial_kernel<Op, false>, 1, T, in, out, n);
        return;
    }
    if (packed)
        launch_async(stream, detail::reduce_partial_kernel<Op, true>, blocks, T, in, workspace.data(), n);
    else
        launch_async(stream, detail::reduce_partial_kernel<Op, false>, blocks, T, in, workspace.data(), n);
    launch_async(stream, detail::reduce_final_kernel<Op>, 1, detail::kReduceFinalThreads, workspace.data(), out,
                 blocks);
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

#pragma once

// Host plumbing of the operator API on the HIP runtime: the checked-call
// macro, argument contracts, grid sizing, stride loops and kernel enqueue.
// Public names, argument meaning and contract messages follow the reference's
// include/core/cuda_utils.cuh:13-118 (drop-in callers match on them); the
// code is organised around three pieces of its own:
//  * detail::hip_check, through which every runtime call passes; a failure
//    prints the call and aborts (runtime errors are not recoverable);
//  * detail::device_props, a per-host-thread table of the properties grid
//    sizing needs, filled on first use of each device;
//  * detail::enqueue, the one launch path: it validates the dimensions
//    (std::invalid_argument before anything is queued), launches and checks
//    the launch itself. Execution errors surface at synchronize().

#include <hip/hip_runtime.h>

#include <array>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <stdexcept>

#include "config.hpp"

namespace opworks::detail {

[[noreturn]] inline void hip_fail(hipError_t status, const char *call, const char *file, int line) {
    std::fprintf(stderr, "[OpWorks] HIP error %s at %s:%d: %s\n", call, file, line, hipGetErrorString(status));
    std::abort();
}

inline void hip_check(hipError_t status, const char *call, const char *file, int line) {
    if (status != hipSuccess)
        hip_fail(status, call, file, line);
}

} // namespace opworks::detail

#define OPWORKS_HIP_CHECK(call) ::opworks::detail::hip_check((call), #call, __FILE__, __LINE__)

namespace opworks {

namespace detail {

// Contract check: a violated precondition is the caller's error.
inline void require(bool condition, const char *message) {
    if (!condition)
        throw std::invalid_argument(message);
}

inline void validate_size(int n) { require(n >= 0, "size must be nonnegative"); }

// Element counts are int in this API (as in the reference), so a matrix must
// hold at most INT_MAX elements.
inline void validate_matrix(int rows, int cols) {
    validate_size(rows);
    validate_size(cols);
    const int64_t elems = static_cast<int64_t>(rows) * static_cast<int64_t>(cols);
    require(elems <= std::numeric_limits<int>::max(), "matrix exceeds the supported INT_MAX elements");
}

// Workgroups of `per_block` units covering n units, computed in 64 bits.
inline int64_t blocks_for64(int64_t n, int64_t per_block) { return (n + per_block - 1) / per_block; }

// Workgroups of `threads` lanes covering n lanes (exact at n = INT_MAX).
inline int blocks_for(int n, int threads = kThreads) {
    validate_size(n);
    require(threads > 0, "block size must be positive");
    return static_cast<int>(blocks_for64(n, threads));
}

struct DeviceProps {
    int compute_units = 0;
    int threads_per_cu = 0;
};

// Up to this many visible devices per process are tracked.
constexpr int kMaxDevices = 64;

inline const DeviceProps &device_props() {
    int dev = 0;
    OPWORKS_HIP_CHECK(hipGetDevice(&dev));
    require(dev >= 0 && dev < kMaxDevices, "device ordinal outside the supported range");
    thread_local std::array<DeviceProps, kMaxDevices> table{};
    DeviceProps &p = table[static_cast<size_t>(dev)];
    if (p.compute_units == 0) {
        OPWORKS_HIP_CHECK(hipDeviceGetAttribute(&p.threads_per_cu, hipDeviceAttributeMaxThreadsPerMultiProcessor, dev));
        OPWORKS_HIP_CHECK(hipDeviceGetAttribute(&p.compute_units, hipDeviceAttributeMultiprocessorCount, dev));
    }
    return p;
}

// Compute units of the current device (256 on an MI355X).
inline int cu_count() { return device_props().compute_units; }

__device__ __forceinline__ int64_t grid_lane() { return static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; }
__device__ __forceinline__ int64_t grid_lanes() { return static_cast<int64_t>(gridDim.x) * blockDim.x; }
__device__ __forceinline__ int block_lane_flat() {
    return static_cast<int>(threadIdx.x + blockDim.x * (threadIdx.y + blockDim.y * threadIdx.z));
}
__device__ __forceinline__ int block_lanes_flat() { return static_cast<int>(blockDim.x * blockDim.y * blockDim.z); }

// Workgroup barrier that orders LDS accesses only. __syncthreads() fences every address space,
// which compiles to s_waitcnt vmcnt(0) lgkmcnt(0): each wave waits for all of its outstanding
// global loads before the barrier. With the fences restricted to LDS only lgkmcnt(0) is waited
// for, so loads issued earlier (GEMV weights, K/V rows) stay in flight across the barrier. Use
// it where the barrier protects LDS data only.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

inline bool launch_dims_positive(dim3 grid, dim3 block) {
    return grid.x != 0 && grid.y != 0 && grid.z != 0 && block.x != 0 && block.y != 0 && block.z != 0;
}

template <typename... Params, typename... Args>
inline void enqueue(hipStream_t stream, size_t lds_bytes, void (*kernel)(Params...), dim3 grid, dim3 block,
                    const Args &...args) {
    require(launch_dims_positive(grid, block), "launch dimensions must be positive");
    hipLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds_bytes), stream, static_cast<Params>(args)...);
    OPWORKS_HIP_CHECK(hipGetLastError());
}

} // namespace detail

// Grid size for n lanes of kThreads-wide workgroups, capped at kNumWaves
// rounds of the workgroups the current device holds resident.
inline int num_blocks_for(int n) {
    detail::validate_size(n);
    if (n == 0)
        return 0;
    const detail::DeviceProps &p = detail::device_props();
    const int64_t cap = static_cast<int64_t>(p.compute_units) * (p.threads_per_cu / kThreads) * kNumWaves;
    const int64_t need = detail::blocks_for(n);
    return static_cast<int>(need < cap ? need : cap);
}

// Stride loops for custom kernels: over the whole grid, over one workgroup's
// x lanes, and over every lane of a 2-D/3-D workgroup.
#define OPWORKS_GRID_LOOP(i, n)                                                                                        \
    for (int64_t i = ::opworks::detail::grid_lane(); i < (n); i += ::opworks::detail::grid_lanes())

#define OPWORKS_BLOCK_LOOP(i, n) for (int64_t i = threadIdx.x; i < (n); i += blockDim.x)

#define OPWORKS_BLOCK_LOOP_FLAT(i, n)                                                                                  \
    for (int i = ::opworks::detail::block_lane_flat(); i < (n); i += ::opworks::detail::block_lanes_flat())

// Enqueue on `stream`; inputs and outputs must stay alive until the stream
// reaches the kernel.
template <typename... Params, typename... Args>
inline void launch_async(hipStream_t stream, void (*kernel)(Params...), dim3 grid, dim3 block, Args... args) {
    detail::enqueue(stream, 0, kernel, grid, block, args...);
}

// The same with `lds_bytes` of dynamic LDS.
template <typename... Params, typename... Args>
inline void launch_async_lds(hipStream_t stream, size_t lds_bytes, void (*kernel)(Params...), dim3 grid, dim3 block,
                             Args... args) {
    detail::enqueue(stream, lds_bytes, kernel, grid, block, args...);
}

inline void synchronize(hipStream_t stream = nullptr) { OPWORKS_HIP_CHECK(hipStreamSynchronize(stream)); }

// Enqueue on the null stream.
template <typename... Params, typename... Args>
inline void launch(void (*kernel)(Params...), dim3 grid, dim3 block, Args... args) {
    detail::enqueue(nullptr, 0, kernel, grid, block, args...);
}

// Enqueue, then wait for the stream to drain.
template <typename... Params, typename... Args>
inline void launch_sync(hipStream_t stream, void (*kernel)(Params...), dim3 grid, dim3 block, Args... args) {
    detail::enqueue(stream, 0, kernel, grid, block, args...);
    synchronize(stream);
}

template <typename... Params, typename... Args>
inline void launch_sync(void (*kernel)(Params...), dim3 grid, dim3 block, Args... args) {
    launch_sync(nullptr, kernel, grid, block, args...);
}

} // namespace opworks

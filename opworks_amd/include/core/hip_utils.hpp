#pragma once

// Error checks, argument contracts, grid sizing, stride loops and launch
// helpers. Same names and semantics as the reference's
// include/core/cuda_utils.cuh:13-118, on the HIP runtime:
//  * contract violations throw std::invalid_argument before anything is enqueued;
//  * HIP runtime failures print and abort (fail-fast, not recoverable);
//  * launch_async only enqueues and checks the launch itself.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <stdexcept>
#include <unordered_map>

#include "config.hpp"

#define OPWORKS_HIP_CHECK(expr)                                                                                        \
    do {                                                                                                               \
        hipError_t err_ = (expr);                                                                                      \
        if (err_ != hipSuccess) {                                                                                      \
            std::fprintf(stderr, "[OpWorks] HIP error %s at %s:%d: %s\n", #expr, __FILE__, __LINE__,                   \
                         hipGetErrorString(err_));                                                                     \
            std::abort();                                                                                              \
        }                                                                                                              \
    } while (0)

namespace opworks {

namespace detail {

inline void require(bool condition, const char *message) {
    if (!condition)
        throw std::invalid_argument(message);
}

inline void validate_size(int n) { require(n >= 0, "size must be nonnegative"); }

inline void validate_matrix(int rows, int cols) {
    validate_size(rows);
    validate_size(cols);
    require(static_cast<int64_t>(rows) * cols <= std::numeric_limits<int>::max(),
            "matrix exceeds the supported INT_MAX elements");
}

// ceil(n / threads) without overflow at n = INT_MAX.
inline int blocks_for(int n, int threads = kThreads) {
    validate_size(n);
    require(threads > 0, "block size must be positive");
    return n / threads + (n % threads != 0);
}

inline int64_t blocks_for64(int64_t n, int64_t per_block) { return n / per_block + (n % per_block != 0); }

// Number of compute units of the current device, cached per (host thread, device).
inline int cu_count() {
    int dev = 0;
    OPWORKS_HIP_CHECK(hipGetDevice(&dev));
    static thread_local std::unordered_map<int, int> cache;
    auto it = cache.find(dev);
    if (it == cache.end()) {
        int cus = 0;
        OPWORKS_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        it = cache.emplace(dev, cus).first;
    }
    return it->second;
}

} // namespace detail

// Adaptive grid size: enough kThreads-wide workgroups to cover n, capped at
// kNumWaves rounds of the workgroups a device can hold resident. Cached per
// current device and host thread (reference: core/cuda_utils.cuh:56-74).
inline int num_blocks_for(int n) {
    detail::validate_size(n);
    if (n == 0)
        return 0;
    int dev = 0;
    OPWORKS_HIP_CHECK(hipGetDevice(&dev));
    static thread_local std::unordered_map<int, int> cache;
    auto found = cache.find(dev);
    if (found == cache.end()) {
        int cus = 0, tpm = 0;
        OPWORKS_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        OPWORKS_HIP_CHECK(hipDeviceGetAttribute(&tpm, hipDeviceAttributeMaxThreadsPerMultiProcessor, dev));
        found = cache.emplace(dev, cus * (tpm / kThreads) * kNumWaves).first;
    }
    const int need = detail::blocks_for(n);
    return need < found->second ? need : found->second;
}

// Stride loops for custom kernels.
#define OPWORKS_GRID_LOOP(i, n)                                                                                        \
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < (n);                             \
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)

#define OPWORKS_BLOCK_LOOP(i, n) for (int64_t i = threadIdx.x; i < (n); i += blockDim.x)

#define OPWORKS_BLOCK_LOOP_FLAT(i, n)                                                                                  \
    for (int i = threadIdx.x + threadIdx.y * blockDim.x + threadIdx.z * blockDim.x * blockDim.y; i < (n);              \
         i += blockDim.x * blockDim.y * blockDim.z)

// Enqueue and check the launch only; execution errors surface at synchronize.
template <typename... Params, typename... Args>
inline void launch_async(hipStream_t stream, void (*kernel)(Params...), dim3 grid, dim3 block, Args... args) {
    detail::require(grid.x && grid.y && grid.z && block.x && block.y && block.z, "launch dimensions must be positive");
    kernel<<<grid, block, 0, stream>>>(static_cast<Params>(args)...);
    OPWORKS_HIP_CHECK(hipGetLastError());
}

// Same, with dynamic LDS bytes.
template <typename... Params, typename... Args>
inline void launch_async_lds(hipStream_t stream, size_t lds_bytes, void (*kernel)(Params...), dim3 grid, dim3 block,
                             Args... args) {
    detail::require(grid.x && grid.y && grid.z && block.x && block.y && block.z, "launch dimensions must be positive");
    kernel<<<grid, block, lds_bytes, stream>>>(static_cast<Params>(args)...);
    OPWORKS_HIP_CHECK(hipGetLastError());
}

inline void synchronize(hipStream_t stream = nullptr) { OPWORKS_HIP_CHECK(hipStreamSynchronize(stream)); }

template <typename... Params, typename... Args>
inline void launch(void (*kernel)(Params...), dim3 grid, dim3 block, Args... args) {
    launch_async(nullptr, kernel, grid, block, args...);
}

template <typename... Params, typename... Args>
inline void launch_sync(hipStream_t stream, void (*kernel)(Params...), dim3 grid, dim3 block, Args... args) {
    launch_async(stream, kernel, grid, block, args...);
    synchronize(stream);
}

template <typename... Params, typename... Args>
inline void launch_sync(void (*kernel)(Params...), dim3 grid, dim3 block, Args... args) {
    launch_sync(nullptr, kernel, grid, block, args...);
}

} // namespace opworks

// opw_reduce_f32_noalloc: the reduction of opw_reduce_f32 for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc). Its partials live in a file-scope
// device array instead of a caller or library allocation.
//
// The array holds kNoAllocPartials floats (256 KiB): one partial per
// 8192-element chunk, so inputs of up to kNoAllocPartials * 8192 = 2^29
// elements; longer inputs are rejected. Each GPU the library runs on holds its
// own copy until the process ends. Every call on a GPU shares that copy, so
// calls that overlap on one GPU (different streams, different host threads)
// race; the partial kernel writes every partial the final kernel reads, so
// nothing has to start at zero.

#include <hip/hip_runtime.h>

#include <array>
#include <mutex>

#include "../include/ops/reduction.hpp"
#include "c_api_common.hpp"

namespace {

constexpr int kNoAllocPartials = 65536;
constexpr int64_t kNoAllocMaxElements = int64_t(kNoAllocPartials) * opworks::detail::kReduceChunk;

__device__ __align__(256) float scratch[kNoAllocPartials];

struct Sum {
    static __device__ float identity() { return 0.f; }
    static __device__ float combine(float a, float b) { return a + b; }
};
struct Max {
    static __device__ float identity() { return -INFINITY; }
    static __device__ float combine(float a, float b) { return fmaxf(a, b); }
};
struct Product {
    static __device__ float identity() { return 1.f; }
    static __device__ float combine(float a, float b) { return a * b; }
};

// Device address of `scratch` on the current device, looked up once per device
// with that device current. Host code passes this pointer, never the array's
// name (a host-side stand-in). The lookup is set-up work, not stream work, so it
// is done on a call made outside graph capture: a first call on a device that
// arrives while `s` is capturing is refused instead of resolving the symbol
// inside the capture.
float *scratch_on_current_device(hipStream_t s) {
    static std::mutex lock;
    static std::array<float *, opworks::detail::kMaxDevices> addresses{};
    int dev = 0;
    OPWORKS_HIP_CHECK(hipGetDevice(&dev));
    opworks::detail::require(dev >= 0 && dev < opworks::detail::kMaxDevices, "device ordinal outside the supported range");
    std::lock_guard<std::mutex> hold(lock);
    float *&p = addresses[static_cast<size_t>(dev)];
    if (!p) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        if (s != nullptr)
            OPWORKS_HIP_CHECK(hipStreamIsCapturing(s, &capture));
        opworks::detail::require(capture == hipStreamCaptureStatusNone,
                                 "opw_reduce_f32_noalloc: make the first call on a device outside graph capture "
                                 "(it looks up the device's scratch address)");
        void *addr = nullptr;
        const hipError_t st = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        if (st != hipSuccess)
            throw std::runtime_error(std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(st));
        p = static_cast<float *>(addr);
    }
    return p;
}

template <typename Op> void reduce_into_scratch(const float *in, float *out, int n, hipStream_t s) {
    opworks::ops::reduce<Op>(in, out, n, opworks::DeviceSpan<float>(scratch_on_current_device(s), kNoAllocPartials), s);
}

} // namespace

extern "C" {

int opw_reduce_f32_noalloc(const float *in, float *out, int n, int op, void *stream) {
    return opworks::capi::guard([&] {
        opworks::detail::require(n >= 0, "size must be nonnegative");
        opworks::detail::require(int64_t(n) <= kNoAllocMaxElements,
                                 "opw_reduce_f32_noalloc: n exceeds the 536870912-element limit of its static scratch");
        hipStream_t s = static_cast<hipStream_t>(stream);
        switch (op) {
        case 0: reduce_into_scratch<Sum>(in, out, n, s); break;
        case 1: reduce_into_scratch<Max>(in, out, n, s); break;
        case 2: reduce_into_scratch<Product>(in, out, n, s); break;
        default: throw std::invalid_argument("unknown reduction op (0 sum, 1 max, 2 product)");
        }
        return 0;
    });
}

} // extern "C"

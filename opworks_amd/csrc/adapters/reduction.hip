// reduction challenge: *out = sum(in[0..n)) (reference adapter:
// tests/integration/reduction.cu:10-22). The partials workspace is kept per
// device and host thread and grows on demand, so repeated calls allocate
// nothing; calls finish before returning, so reuse on one thread is safe.
#include <memory>

#include "adapter_common.hpp"

namespace {
struct Sum {
    static __device__ float identity() { return 0.f; }
    static __device__ float combine(float a, float b) { return a + b; }
};

constexpr int kMaxDevices = 64;

opworks::DeviceBuffer &workspace_for(int device, int required) {
    static thread_local std::unique_ptr<opworks::DeviceBuffer> slots[kMaxDevices];
    opworks::detail::require(device >= 0 && device < kMaxDevices, "device ordinal out of range");
    auto &slot = slots[device];
    if (!slot || slot->size() < required)
        slot = std::make_unique<opworks::DeviceBuffer>(required);
    return *slot;
}
} // namespace

extern "C" void solve(const float *in, float *out, int n) {
    opworks_adapter::guarded("reduction", [&] {
        opworks::detail::validate_size(n);
        int device = 0;
        OPWORKS_HIP_CHECK(hipGetDevice(&device));
        auto &ws = workspace_for(device, opworks::ops::reduction_workspace_size(n));
        opworks::ops::reduce<Sum>(in, out, n, ws.view());
    });
}

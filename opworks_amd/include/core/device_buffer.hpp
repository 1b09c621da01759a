#pragma once

// DeviceBuffer: the fp32 owner the operator API and the builders use. It is
// TypedDeviceBuffer<float> with the reference's int-sized surface
// (include/core/device_buffer.cuh:9-81): sizes are int (at most INT_MAX
// elements), host transfers block on the given stream, to_host_scalar needs
// exactly one element, and view() lends a DeviceSpan only from an lvalue
// owner, so a span can never outlive a temporary.

#include <limits>
#include <vector>

#include "device_span.hpp"
#include "typed_device_buffer.hpp"

namespace opworks {

class DeviceBuffer {
  public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(int n) : store_((detail::validate_size(n), n)) {}

    static DeviceBuffer from_host(const std::vector<float> &host, hipStream_t stream = nullptr) {
        detail::require(host.size() <= static_cast<size_t>(std::numeric_limits<int>::max()),
                        "buffer exceeds the supported INT_MAX elements");
        return DeviceBuffer(TypedDeviceBuffer<float>::from_host(host, stream));
    }

    std::vector<float> to_host(hipStream_t stream = nullptr) const { return store_.to_host(stream); }
    float to_host_scalar(hipStream_t stream = nullptr) const { return store_.to_host_scalar(stream); }

    DeviceSpan<float> view() & { return {data(), size()}; }
    DeviceSpan<const float> view() const & { return {data(), size()}; }
    DeviceSpan<float> view() && = delete;
    DeviceSpan<const float> view() const && = delete;

    float *data() { return store_.data(); }
    const float *data() const { return store_.data(); }
    int size() const { return static_cast<int>(store_.size()); }

  private:
    explicit DeviceBuffer(TypedDeviceBuffer<float> &&store) : store_(std::move(store)) {}

    TypedDeviceBuffer<float> store_;
};

} // namespace opworks

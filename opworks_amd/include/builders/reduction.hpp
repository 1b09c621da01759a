#pragma once

// ReductionBuilder — reduces a borrowed span into a new one-element
// DeviceBuffer (reference: include/builders/reduction.cuh:8-28).

#include "../core/device_buffer.hpp"
#include "../ops/reduction.hpp"

namespace opworks {

class ReductionBuilder {
  public:
    explicit ReductionBuilder(DeviceSpan<const float> in) : in_(in) {}
    explicit ReductionBuilder(const DeviceBuffer &in) : ReductionBuilder(in.view()) {}
    ReductionBuilder(const DeviceBuffer &&) = delete;

    // Stream-ordered scratch (ops::reduce convenience overload).
    template <typename Op> DeviceBuffer apply(hipStream_t stream = nullptr) const {
        DeviceBuffer out(1);
        ops::reduce<Op>(in_.data(), out.data(), in_.size(), stream);
        return out;
    }

    // Caller-provided workspace of ops::reduction_workspace_size(n) floats.
    template <typename Op> DeviceBuffer apply(DeviceSpan<float> workspace, hipStream_t stream = nullptr) const {
        DeviceBuffer out(1);
        ops::reduce<Op>(in_.data(), out.data(), in_.size(), workspace, stream);
        return out;
    }

  private:
    DeviceSpan<const float> in_;
};

} // namespace opworks

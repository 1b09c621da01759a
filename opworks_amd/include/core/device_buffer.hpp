#pragma once

// Move-only owner of an fp32 device allocation (reference:
// include/core/device_buffer.cuh:9-81). Host copies are blocking on the given
// stream; empty buffers allocate nothing.

#include <limits>
#include <vector>

#include "device_span.hpp"

namespace opworks {

class DeviceBuffer {
  public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(int n) : n_(n) {
        detail::validate_size(n);
        if (n != 0)
            OPWORKS_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&ptr_), sizeof(float) * static_cast<size_t>(n_)));
    }
    ~DeviceBuffer() {
        if (ptr_)
            (void)hipFree(ptr_);
    }

    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    DeviceBuffer(DeviceBuffer &&o) noexcept : ptr_(o.ptr_), n_(o.n_) {
        o.ptr_ = nullptr;
        o.n_ = 0;
    }
    DeviceBuffer &operator=(DeviceBuffer &&o) noexcept {
        if (this != &o) {
            if (ptr_)
                (void)hipFree(ptr_);
            ptr_ = o.ptr_;
            n_ = o.n_;
            o.ptr_ = nullptr;
            o.n_ = 0;
        }
        return *this;
    }

    static DeviceBuffer from_host(const std::vector<float> &h, hipStream_t stream = nullptr) {
        detail::require(h.size() <= static_cast<size_t>(std::numeric_limits<int>::max()),
                        "buffer exceeds the supported INT_MAX elements");
        DeviceBuffer buf(static_cast<int>(h.size()));
        if (!h.empty()) {
            OPWORKS_HIP_CHECK(
                hipMemcpyAsync(buf.ptr_, h.data(), sizeof(float) * h.size(), hipMemcpyHostToDevice, stream));
            synchronize(stream);
        }
        return buf;
    }

    std::vector<float> to_host(hipStream_t stream = nullptr) const {
        std::vector<float> h(static_cast<size_t>(n_));
        if (n_ != 0) {
            OPWORKS_HIP_CHECK(hipMemcpyAsync(h.data(), ptr_, sizeof(float) * h.size(), hipMemcpyDeviceToHost, stream));
            synchronize(stream);
        }
        return h;
    }

    float to_host_scalar(hipStream_t stream = nullptr) const {
        detail::require(n_ == 1, "scalar copy requires exactly one element");
        return to_host(stream)[0];
    }

    DeviceSpan<float> view() & { return {ptr_, n_}; }
    DeviceSpan<const float> view() const & { return {ptr_, n_}; }
    DeviceSpan<float> view() && = delete;
    DeviceSpan<const float> view() const && = delete;

    float *data() { return ptr_; }
    const float *data() const { return ptr_; }
    int size() const { return n_; }

  private:
    float *ptr_ = nullptr;
    int n_ = 0;
};

} // namespace opworks

#pragma once

// Owning device buffer for the element types the model runtime stores: fp32,
// int32 and bf16 (reference: include/core/typed_device_buffer.cuh:15-92).
// Sizes are int64 so a 1 GiB embedding table fits.

#include <cstdint>
#include <type_traits>
#include <vector>

#include "bf16.hpp"
#include "device_span.hpp"

namespace opworks {

template <typename T> class TypedDeviceBuffer {
    static_assert(std::is_same_v<T, float> || std::is_same_v<T, int32_t> || std::is_same_v<T, bf16>,
                  "TypedDeviceBuffer supports float, int32_t and bf16");

  public:
    TypedDeviceBuffer() = default;
    explicit TypedDeviceBuffer(int64_t n) : n_(n) {
        detail::require(n >= 0, "size must be nonnegative");
        if (n_ != 0)
            OPWORKS_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&ptr_), sizeof(T) * static_cast<size_t>(n_)));
    }
    ~TypedDeviceBuffer() {
        if (ptr_)
            (void)hipFree(ptr_);
    }

    TypedDeviceBuffer(const TypedDeviceBuffer &) = delete;
    TypedDeviceBuffer &operator=(const TypedDeviceBuffer &) = delete;
    TypedDeviceBuffer(TypedDeviceBuffer &&o) noexcept : ptr_(o.ptr_), n_(o.n_) {
        o.ptr_ = nullptr;
        o.n_ = 0;
    }
    TypedDeviceBuffer &operator=(TypedDeviceBuffer &&o) noexcept {
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

    static TypedDeviceBuffer from_host(const std::vector<T> &h, hipStream_t stream = nullptr) {
        return from_host(h.data(), static_cast<int64_t>(h.size()), stream);
    }

    static TypedDeviceBuffer from_host(const T *data, int64_t n, hipStream_t stream = nullptr) {
        TypedDeviceBuffer buf(n);
        if (n != 0) {
            OPWORKS_HIP_CHECK(
                hipMemcpyAsync(buf.ptr_, data, sizeof(T) * static_cast<size_t>(n), hipMemcpyHostToDevice, stream));
            synchronize(stream);
        }
        return buf;
    }

    std::vector<T> to_host(hipStream_t stream = nullptr) const {
        std::vector<T> h(static_cast<size_t>(n_));
        if (n_ != 0) {
            OPWORKS_HIP_CHECK(hipMemcpyAsync(h.data(), ptr_, sizeof(T) * h.size(), hipMemcpyDeviceToHost, stream));
            synchronize(stream);
        }
        return h;
    }

    T to_host_scalar(hipStream_t stream = nullptr) const {
        detail::require(n_ == 1, "scalar copy requires exactly one element");
        return to_host(stream)[0];
    }

    T *data() { return ptr_; }
    const T *data() const { return ptr_; }
    int64_t size() const { return n_; }

  private:
    T *ptr_ = nullptr;
    int64_t n_ = 0;
};

} // namespace opworks

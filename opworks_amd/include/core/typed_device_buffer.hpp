#pragma once

// Owning device memory. One owner type, TypedDeviceBuffer<T>, holds an
// allocation of `count` elements as a unique_ptr whose deleter calls hipFree;
// its count travels with the pointer when it moves, so a moved-from buffer is
// empty (null pointer, size 0). Host transfers are blocking on the given
// stream. DeviceBuffer (core/device_buffer.hpp) is the fp32, int-sized view of
// this owner that the operator API takes.
//
// Interface of the reference's include/core/typed_device_buffer.cuh:15-92:
// element types float / int32_t / bf16, int64 sizes, move-only,
// from_host(vector) / from_host(pointer, n) / to_host / to_host_scalar.

#include <cstdint>
#include <memory>
#include <type_traits>
#include <utility>
#include <vector>

#include "bf16.hpp"
#include "hip_utils.hpp"

namespace opworks {

namespace detail {

struct HipFree {
    void operator()(void *p) const noexcept { (void)hipFree(p); }
};

template <typename T> using device_unique_ptr = std::unique_ptr<T, HipFree>;

template <typename T> device_unique_ptr<T> device_alloc(int64_t count) {
    if (count == 0)
        return device_unique_ptr<T>();
    void *raw = nullptr;
    OPWORKS_HIP_CHECK(hipMalloc(&raw, sizeof(T) * static_cast<size_t>(count)));
    return device_unique_ptr<T>(static_cast<T *>(raw));
}

// Copies `bytes` with hipMemcpyAsync on `stream` and waits for the stream, so
// the host side may be reused or read as soon as this returns.
inline void copy_and_wait(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, hipStream_t stream) {
    if (bytes == 0)
        return;
    OPWORKS_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, kind, stream));
    synchronize(stream);
}

// A device allocation and its element count, moved together.
template <typename T> struct Allocation {
    device_unique_ptr<T> ptr;
    int64_t count = 0;

    Allocation() = default;
    explicit Allocation(int64_t n) : ptr(device_alloc<T>(n)), count(n) {}
    Allocation(Allocation &&other) noexcept : ptr(std::move(other.ptr)), count(std::exchange(other.count, 0)) {}
    Allocation &operator=(Allocation &&other) noexcept {
        ptr = std::move(other.ptr);
        count = std::exchange(other.count, 0);
        return *this;
    }
};

} // namespace detail

template <typename T> class TypedDeviceBuffer {
    static_assert(std::is_same_v<T, float> || std::is_same_v<T, int32_t> || std::is_same_v<T, bf16>,
                  "TypedDeviceBuffer supports float, int32_t and bf16");

  public:
    using value_type = T;

    TypedDeviceBuffer() = default;
    explicit TypedDeviceBuffer(int64_t n) : mem_(checked_count(n)) {}

    TypedDeviceBuffer(const TypedDeviceBuffer &) = delete;
    TypedDeviceBuffer &operator=(const TypedDeviceBuffer &) = delete;
    TypedDeviceBuffer(TypedDeviceBuffer &&) noexcept = default;
    TypedDeviceBuffer &operator=(TypedDeviceBuffer &&) noexcept = default;

    static TypedDeviceBuffer from_host(const std::vector<T> &host, hipStream_t stream = nullptr) {
        return from_host(host.data(), static_cast<int64_t>(host.size()), stream);
    }

    static TypedDeviceBuffer from_host(const T *host, int64_t n, hipStream_t stream = nullptr) {
        TypedDeviceBuffer buf(n);
        detail::copy_and_wait(buf.data(), host, buf.bytes(), hipMemcpyHostToDevice, stream);
        return buf;
    }

    std::vector<T> to_host(hipStream_t stream = nullptr) const {
        std::vector<T> host(static_cast<size_t>(size()));
        detail::copy_and_wait(host.data(), data(), bytes(), hipMemcpyDeviceToHost, stream);
        return host;
    }

    T to_host_scalar(hipStream_t stream = nullptr) const {
        detail::require(size() == 1, "scalar copy requires exactly one element");
        T value{};
        detail::copy_and_wait(&value, data(), sizeof(T), hipMemcpyDeviceToHost, stream);
        return value;
    }

    T *data() { return mem_.ptr.get(); }
    const T *data() const { return mem_.ptr.get(); }
    int64_t size() const { return mem_.count; }
    size_t bytes() const { return sizeof(T) * static_cast<size_t>(mem_.count); }

  private:
    static int64_t checked_count(int64_t n) {
        detail::require(n >= 0, "size must be nonnegative");
        return n;
    }

    detail::Allocation<T> mem_;
};

} // namespace opworks

#pragma once

// ElementwiseBuilder: borrows one or two equal-length fp32 inputs and applies
// a map functor into a new DeviceBuffer. The inputs are kept as an array of
// spans plus their arity; apply<Op>() checks Op::kArity against it and
// forwards the first kArity spans to ops::map.
//
// Interface of the reference's include/builders/elementwise.cuh:8-43 (names,
// overloads, messages): owners are borrowed, so constructors taking an
// rvalue DeviceBuffer are deleted; a functor with state (ScaleAdd{alpha})
// travels to the kernel by value.

#include <array>
#include <cstddef>
#include <utility>

#include "../core/device_buffer.hpp"
#include "../ops/elementwise.hpp"

namespace opworks {

class ElementwiseBuilder {
  public:
    ElementwiseBuilder(DeviceSpan<const float> a, DeviceSpan<const float> b) : inputs_{a, b}, arity_(2) {
        detail::require(a.size() == b.size(), "elementwise inputs must have equal lengths");
    }
    ElementwiseBuilder(const DeviceBuffer &a, const DeviceBuffer &b) : ElementwiseBuilder(a.view(), b.view()) {}
    explicit ElementwiseBuilder(DeviceSpan<const float> a) : inputs_{a, DeviceSpan<const float>{}}, arity_(1) {}
    explicit ElementwiseBuilder(const DeviceBuffer &a) : ElementwiseBuilder(a.view()) {}

    ElementwiseBuilder(const DeviceBuffer &&) = delete;
    ElementwiseBuilder(const DeviceBuffer &&, const DeviceBuffer &) = delete;
    ElementwiseBuilder(const DeviceBuffer &, const DeviceBuffer &&) = delete;
    ElementwiseBuilder(const DeviceBuffer &&, const DeviceBuffer &&) = delete;

    template <typename Op> DeviceBuffer apply(const Op &op = Op{}, hipStream_t stream = nullptr) const {
        static_assert(Op::kArity == 1 || Op::kArity == 2, "elementwise arity must be 1 or 2");
        detail::require(arity_ == Op::kArity, "functor arity does not match builder inputs");
        DeviceBuffer out(length());
        map_into(out.data(), op, stream, std::make_index_sequence<Op::kArity>{});
        return out;
    }

    int arity() const { return arity_; }
    int length() const { return inputs_[0].size(); }

  private:
    template <typename Op, size_t... I>
    void map_into(float *out, const Op &op, hipStream_t stream, std::index_sequence<I...>) const {
        ops::map(inputs_[I].data()..., out, length(), op, stream);
    }

    std::array<DeviceSpan<const float>, 2> inputs_;
    int arity_;
};

} // namespace opworks

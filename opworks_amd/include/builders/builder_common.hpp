#pragma once

// Callback extension point shared by the config builders
// (reference: include/builders/builder_common.cuh:7-9): every builder exposes
// apply(fn) which hands the validated builder to fn and returns fn's result.

#include "../core/device_span.hpp"
#include "../core/hip_utils.hpp"

namespace opworks {

template <typename Builder, typename Fn> decltype(auto) apply_builder(const Builder &builder, Fn &&fn) {
    return static_cast<Fn &&>(fn)(builder);
}

namespace detail {

// CRTP mix-in giving a builder its apply(fn) member.
template <typename Derived> struct CallbackBuilder {
    template <typename Fn> decltype(auto) apply(Fn &&fn) const {
        return apply_builder(static_cast<const Derived &>(*this), static_cast<Fn &&>(fn));
    }
};

} // namespace detail
} // namespace opworks

#pragma once

// Callback extension point shared by the config builders
// (reference: include/builders/builder_common.cuh:7-9).

#include "../core/device_span.hpp"

namespace opworks {

template <typename Builder, typename Fn> decltype(auto) apply_builder(const Builder &builder, Fn &&fn) {
    return static_cast<Fn &&>(fn)(builder);
}

} // namespace opworks

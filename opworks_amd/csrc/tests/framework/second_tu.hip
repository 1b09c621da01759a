// Second translation unit of the framework test: including <opworks> here as
// well proves the headers link cleanly twice (no non-inline definitions) and
// that kernels instantiated in both units run.
#include <opworks>

#include <stdexcept>

namespace {
struct Negate {
    __device__ float operator()(float x) const { return -x; }
};
} // namespace

void second_translation_unit() {
    auto in = opworks::DeviceBuffer::from_host({1.f, -2.f, 3.5f});
    opworks::DeviceBuffer out(3);
    opworks::ops::map(in.data(), out.data(), 3, Negate{});
    const auto h = out.to_host();
    if (h[0] != -1.f || h[1] != 2.f || h[2] != -3.5f)
        throw std::runtime_error("second translation unit: map result");
}

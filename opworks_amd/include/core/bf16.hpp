#pragma once

// bfloat16 storage type and the conversions the kernels use. The round to
// nearest-even from fp32 is the bit recipe the reference's tests use to build
// bf16 weights (tests/model/ops_test.cu:77-82); NaN inputs are not expected
// on this path.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace opworks {

struct bf16 {
    uint16_t bits;
};
static_assert(sizeof(bf16) == 2, "bf16 must be two bytes");

__host__ __device__ inline float bf16_to_float(uint16_t b) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

__host__ __device__ inline uint16_t float_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

} // namespace opworks

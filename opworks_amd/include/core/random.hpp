#pragma once

// Counter-based synthetic data. Element i of stream `s` under seed `seed` is a
// pure function of (seed, s, i), so the GPU fills HBM directly and a CPU
// checker regenerates bit-identical arrays without any data transfer:
//  * bits:    splitmix64 finalizer of key + (i+1) * golden ratio (Steele et al.
//             2014, "Fast splittable pseudorandom number generators");
//  * uniform: u = (top 24 bits) * 2^-24 (exact), value = fmaf(u, hi - lo, lo);
//  * normal:  Irwin-Hall sum of four 24-bit uniforms, centred and scaled to
//             unit variance in integer arithmetic, one int->float rounding,
//             value = fmaf(z, stddev, mean). Bounded at +-2*sqrt(3) sigma.
// Every step is integer arithmetic or a single correctly rounded IEEE
// operation, so host and device results are identical.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace opworks::rng {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(seed ^ mix64(stream + kGolden));
}

__host__ __device__ inline uint64_t bits(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGolden); }

__host__ __device__ inline float uniform(uint64_t key, uint64_t i, float lo, float hi) {
    const float u = static_cast<float>(static_cast<uint32_t>(bits(key, i) >> 40)) * 0x1p-24f;
    return fmaf(u, hi - lo, lo);
}

__host__ __device__ inline float normal(uint64_t key, uint64_t i, float mean, float stddev) {
    const uint64_t a = bits(key, 2 * i), b = bits(key, 2 * i + 1);
    const int32_t s = static_cast<int32_t>(a >> 40) + static_cast<int32_t>((a >> 16) & 0xFFFFFFu) +
                      static_cast<int32_t>(b >> 40) + static_cast<int32_t>((b >> 16) & 0xFFFFFFu) - (1 << 25);
    const float z = static_cast<float>(s) * 0x1.bb67aep-24f; // sqrt(3) / 2^24
    return fmaf(z, stddev, mean);
}

} // namespace opworks::rng

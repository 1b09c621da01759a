#pragma once

// 16-byte weight packs for the GEMV kernels: a lane streams 4 fp32 or 8 bf16
// weights per load. bf16 is widened exactly (its bits become the high half
// of an fp32 word) and every product is accumulated in fp32, the arithmetic
// of the reference's gemv_bf16_kernel (include/ops/linear.cuh:99-121).

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "bf16.hpp"

namespace opworks::detail {

using f32x4 = float __attribute__((ext_vector_type(4)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

template <typename WT> struct WPack;
template <> struct WPack<float> {
    static constexpr int kElems = 4;
    using type = f32x4;
    __device__ static float at(const f32x4 &p, int j) { return p[j]; }
};
template <> struct WPack<bf16> {
    static constexpr int kElems = 8;
    using type = u32x4;
    __device__ static float at(const u32x4 &p, int j) {
        const uint32_t w = p[j >> 1];
        return __builtin_bit_cast(float, (j & 1) ? (w & 0xffff0000u) : (w << 16));
    }
};

// Pack `pack` of a row, loaded non-temporally (weights are read once).
template <typename WT> __device__ __forceinline__ typename WPack<WT>::type load_wpack(const WT *row, int64_t pack) {
    return __builtin_nontemporal_load(reinterpret_cast<const typename WPack<WT>::type *>(row) + pack);
}

template <typename WT> __device__ __forceinline__ float widen(WT v) {
    if constexpr (std::is_same_v<WT, bf16>)
        return bf16_to_float(v.bits);
    else
        return v;
}

// acc += sum_j w[j] * x[j] over one pack, in j order (x: the pack's kElems inputs).
template <typename WT>
__device__ __forceinline__ float dot_wpack(const typename WPack<WT>::type &w, const f32x4 (&x)[WPack<WT>::kElems / 4],
                                           float acc) {
    constexpr int E = WPack<WT>::kElems;
#pragma unroll
    for (int q = 0; q < E / 4; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc = fmaf(WPack<WT>::at(w, 4 * q + j), x[q][j], acc);
    return acc;
}

} // namespace opworks::detail

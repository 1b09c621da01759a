#pragma once

// 64-lane wavefront reductions on DPP row operations (GFX9 encodings, valid on
// gfx950). A full reduction is 6 DPP steps plus one v_readlane: no LDS traffic
// and no barriers. The result is returned wave-uniform.

#include <hip/hip_runtime.h>

#include "config.hpp"

namespace opworks::wave {

// DPP control words.
enum : int {
    kQuadSwap1 = 0xB1,     // quad_perm [1,0,3,2]: lane ^ 1
    kQuadSwap2 = 0x4E,     // quad_perm [2,3,0,1]: lane ^ 2
    kRowMirror = 0x140,    // lane i <- lane 15-i within each 16-lane row
    kRowHalfMirror = 0x141, // lane i <- lane 7-i within each 8-lane half row
    kRowBcast15 = 0x142,   // lane 15 of row r -> every lane of row r+1
    kRowBcast31 = 0x143,   // lane 31 -> every lane of rows 2 and 3
};

// Lanes not selected by row_mask, or whose source is invalid, return `old`.
template <int ctrl, int row_mask = 0xf>
__device__ __forceinline__ float dpp(float old, float src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, src),
                                                                ctrl, row_mask, 0xf, false));
}

template <int ctrl, int row_mask = 0xf>
__device__ __forceinline__ int dpp(int old, int src) {
    return __builtin_amdgcn_update_dpp(old, src, ctrl, row_mask, 0xf, false);
}

__device__ __forceinline__ float readlane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ int readlane(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// Reduces v over the wave with an associative, commutative combine.
// `lanes` is 64, or 32 for a wave whose upper half does not exist (the tail
// wave of a workgroup of 32*(2k+1) threads); it must be wave-uniform.
template <typename Combine>
__device__ __forceinline__ float reduce(float v, float identity, Combine combine, int lanes = kWaveSize) {
    v = combine(v, dpp<kQuadSwap1>(v, v));
    v = combine(v, dpp<kQuadSwap2>(v, v));
    v = combine(v, dpp<kRowHalfMirror>(v, v));
    v = combine(v, dpp<kRowMirror>(v, v)); // every lane holds its 16-lane row total
    v = combine(v, dpp<kRowBcast15, 0xa>(identity, v)); // rows 1, 3 hold rows 0+1, 2+3
    if (lanes == kWaveSize) {
        v = combine(v, dpp<kRowBcast31, 0xc>(identity, v)); // row 3 holds the wave total
        return readlane(v, 63);
    }
    return readlane(v, 31);
}

struct Add {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct Max {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

__device__ __forceinline__ float sum(float v) { return reduce(v, 0.f, Add{}); }
__device__ __forceinline__ float max(float v) { return reduce(v, kNegInf, Max{}); }

} // namespace opworks::wave

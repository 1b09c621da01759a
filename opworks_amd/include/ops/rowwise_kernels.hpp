#pragma once

// Shared machinery of the row-wise kernels (softmax, layer_norm, rms_norm).
//
// Register-resident rows: a row of `cols` fp32 values is split over kW waves;
// each lane holds kV 16-byte packs, pack p of the row living in lane
// p % 64 of wave (p / 64) % kW at slot p / (64 * kW). A wave-load therefore
// reads 1 KiB of contiguous row. The row is read from HBM exactly once and
// written once (8 bytes per element of traffic). Row statistics are reduced
// with DPP inside each wave; rows spanning several waves exchange one partial
// per wave through LDS and combine them in a fixed order, so every wave of the
// row gets the identical value. Shapes the register plan cannot hold (cols not
// a multiple of 4, misaligned rows, or more than 32768 columns) use a
// streaming kernel that re-reads the row.

#include <cstdint>
#include <type_traits>

#include "../core/block_reduce.hpp"
#include "../core/hip_utils.hpp"
#include "../core/wave.hpp"
#include "elementwise.hpp"

namespace opworks::detail {

constexpr int kRowMaxRegCols = 32768;

template <int kW> struct RowShape {
    static constexpr int kRowsPerBlock = kW >= 4 ? 1 : 4 / kW;
    static constexpr int kBlock = kRowsPerBlock * kW * kWaveSize;
};

struct RowPos {
    int64_t row;     // row index of this wave
    int wave_in_row; // which of the row's kW waves
    int row_in_block;
    int lane;
    bool active; // row < rows (wave-uniform)
};

template <int kW> __device__ __forceinline__ RowPos row_position(int rows) {
    RowPos p;
    const int wave = threadIdx.x / kWaveSize;
    p.lane = threadIdx.x % kWaveSize;
    p.row_in_block = wave / kW;
    p.wave_in_row = wave % kW;
    p.row = static_cast<int64_t>(blockIdx.x) * RowShape<kW>::kRowsPerBlock + p.row_in_block;
    p.active = p.row < rows;
    return p;
}

template <int kW> __device__ __forceinline__ int pack_index(const RowPos &p, int k) {
    return (k * kW + p.wave_in_row) * kWaveSize + p.lane;
}

// True when pack k of this lane lies inside the row (always, for exact plans).
template <int kW, bool kExact> __device__ __forceinline__ bool pack_valid(const RowPos &p, int k, int n4) {
    return kExact || pack_index<kW>(p, k) < n4;
}

// Loads this lane's kV packs of its row as one unpredicated batch: a wave past
// the last row reads the last row and a pack past the row end reads the row's
// last pack, so every address is valid and no load sits behind a branch.
// Used by softmax, where the predicated form compiled to one branch and one
// vmcnt(0) wait per pack (4096 x 1024: 6.13 against 6.96 us). RMSNorm keeps
// its predicated loads, which measured faster for its 8 packs per lane
// (8192 x 2048: 21.4 against 22.9 us). Callers mask invalid packs with
// pack_valid and store only for active waves.
template <int kW, int kV, bool kExact>
__device__ __forceinline__ void load_row_packs(const float *__restrict__ in, int rows, int cols, const RowPos &p,
                                               f32x4 (&v)[kV]) {
    const int64_t row = p.active ? p.row : rows - 1;
    const int n4 = cols / 4;
    const f32x4 *src = reinterpret_cast<const f32x4 *>(in + row * cols);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int q = pack_index<kW>(p, k);
        v[k] = __builtin_nontemporal_load(src + (kExact || q < n4 ? q : n4 - 1));
    }
}

// Combines one value per wave across the kW waves of a row (fixed order).
template <int kW, typename Combine>
__device__ __forceinline__ float row_combine(float v, const RowPos &p, Combine combine) {
    if constexpr (kW == 1) {
        return v;
    } else {
        __shared__ float slots[RowShape<kW>::kRowsPerBlock * kW];
        if (p.lane == 0)
            slots[p.row_in_block * kW + p.wave_in_row] = v;
        __syncthreads();
        float r = slots[p.row_in_block * kW];
#pragma unroll
        for (int k = 1; k < kW; ++k)
            r = combine(r, slots[p.row_in_block * kW + k]);
        __syncthreads(); // slots are reused by the next combine
        return r;
    }
}

// Register plan for a row of `cols` floats: kW waves, kV packs per lane.
struct RowPlan {
    int waves = 0; // 0 = streaming kernel
    int packs = 0;
};

inline RowPlan plan_row(int cols, bool packed) {
    if (!packed || cols % 4 != 0 || cols > kRowMaxRegCols)
        return {};
    const int n4 = cols / 4;
    if (n4 <= 64)
        return {1, 1};
    if (n4 <= 128)
        return {1, 2};
    if (n4 <= 256)
        return {1, 4};
    if (n4 <= 512)
        return {1, 8};
    if (n4 <= 1024)
        return {2, 8};
    if (n4 <= 2048)
        return {4, 8};
    if (n4 <= 4096)
        return {8, 8};
    return {16, 8};
}

// The plan for `rows` rows: a short matrix (fewer than 2048 row waves, 8 per CU) spreads each
// row over more waves with fewer packs each, down to 2 packs per lane, so the GPU has enough
// waves in flight: 512 x 2048 (a 512-token prefill's RMSNorm) runs 4 waves of 2 packs per row
// instead of 1 wave of 8. Only the row ops whose dispatch carries these shapes use it.
inline RowPlan plan_row_for_rows(int rows, int cols, bool packed) {
    RowPlan p = plan_row(cols, packed);
    while (p.waves != 0 && p.packs >= 4 && p.waves <= 4 && int64_t(rows) * p.waves < 2048) {
        p.waves *= 2;
        p.packs /= 2;
    }
    return p;
}

// Calls fn(W{}, V{}) with std::integral_constant tags of the plan's
// instantiation (C++17 generic lambdas read them back as constants).
template <int N> using IntTag = std::integral_constant<int, N>;

template <typename Fn> inline void dispatch_row_plan(const RowPlan &plan, Fn &&fn) {
    switch (plan.waves * 100 + plan.packs) {
    case 101: fn(IntTag<1>{}, IntTag<1>{}); break;
    case 102: fn(IntTag<1>{}, IntTag<2>{}); break;
    case 104: fn(IntTag<1>{}, IntTag<4>{}); break;
    case 108: fn(IntTag<1>{}, IntTag<8>{}); break;
    case 208: fn(IntTag<2>{}, IntTag<8>{}); break;
    case 408: fn(IntTag<4>{}, IntTag<8>{}); break;
    case 808: fn(IntTag<8>{}, IntTag<8>{}); break;
    case 1608: fn(IntTag<16>{}, IntTag<8>{}); break;
    default: throw std::invalid_argument("row plan has no kernel instantiation");
    }
}

// dispatch_row_plan plus the shapes plan_row_for_rows can add.
template <typename Fn> inline void dispatch_row_plan_for_rows(const RowPlan &plan, Fn &&fn) {
    switch (plan.waves * 100 + plan.packs) {
    case 202: fn(IntTag<2>{}, IntTag<2>{}); break;
    case 204: fn(IntTag<2>{}, IntTag<4>{}); break;
    case 402: fn(IntTag<4>{}, IntTag<2>{}); break;
    case 404: fn(IntTag<4>{}, IntTag<4>{}); break;
    case 802: fn(IntTag<8>{}, IntTag<2>{}); break;
    case 804: fn(IntTag<8>{}, IntTag<4>{}); break;
    default: dispatch_row_plan(plan, fn);
    }
}

// True when the plan's kW * kV * 64 packs cover the row exactly: the kernels
// then drop the per-lane bounds test, which keeps every load of a lane in one
// unpredicated batch.
template <int kW, int kV> inline bool row_plan_exact(int cols) { return cols / 4 == kW * kV * kWaveSize; }

template <int kW> inline int row_grid(int rows) {
    return static_cast<int>(blocks_for64(rows, RowShape<kW>::kRowsPerBlock));
}

} // namespace opworks::detail

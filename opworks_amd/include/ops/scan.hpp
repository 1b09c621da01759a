#pragma once

// ops::scan — inclusive or exclusive prefix sum / prefix maximum of an fp32
// array, the kernel behind ScanBuilder (the reference's builder carries the
// operation metadata, include/builders/scan.cuh:7-17, and ships no kernel).
//
//   inclusive: out[i] = x[0] (+) x[1] (+) ... (+) x[i]
//   exclusive: out[0] = identity, out[i] = x[0] (+) ... (+) x[i-1]
// (+) is + (identity 0) for ScanOp::sum and fmaxf (identity -inf) for
// ScanOp::maximum; fmaxf drops NaN operands, so a prefix of NaNs alone scans
// to -inf.
//
// gfx950 design: reduce-then-scan over tiles of kScanTile elements, three
// launches, no atomics and no inter-workgroup waiting, so the result is the
// same bit pattern on every run for a given n.
//  1. scan_tile_reduce_kernel: workgroup b combines tile b -> partial[b].
//  2. scan_partials_kernel: one workgroup turns partial[] into exclusive tile
//     prefixes in place (each lane scans a contiguous run, then a workgroup
//     scan of the run totals).
//  3. scan_tile_kernel: workgroup b rescans tile b in four rounds of 2048
//     contiguous elements: a lane scans its 16-byte pack, a wave scans the
//     lane totals with DPP row shifts and row broadcasts, LDS carries the
//     wave totals, and the tile prefix enters as the first operand.
// Inputs of at most one tile take launch 3 alone and need no workspace.
// The partial buffer must be 16-byte aligned (any hipMalloc'd workspace is).
// HBM traffic is 12 B per element (two reads, one write) against 8 B of
// compulsory traffic. In-place scans (out == in) are allowed: every element
// is read by the lane that later writes it, before the write.

#include <cmath>

#include "../core/device_span.hpp"
#include "../core/hip_utils.hpp"
#include "../core/wave.hpp"
#include "elementwise.hpp" // f32x4, aligned16

namespace opworks::detail {

constexpr int kScanThreads = 512;
constexpr int kScanRounds = 4;
constexpr int kScanRound = kScanThreads * 4;           // elements per round (2048)
constexpr int kScanTile = kScanRound * kScanRounds;    // elements per workgroup (8192)
constexpr int kScanPartialThreads = 1024;
constexpr int kScanPartialBatch = 4;                   // 16-byte packs a lane loads per round trip

struct ScanSumOp {
    static __device__ __forceinline__ float identity() { return 0.f; }
    static __device__ __forceinline__ float combine(float a, float b) { return a + b; }
};
struct ScanMaxOp {
    static __device__ __forceinline__ float identity() { return -INFINITY; }
    static __device__ __forceinline__ float combine(float a, float b) { return fmaxf(a, b); }
};

// DPP row shifts (GFX9 encoding row_shr:n = 0x110 + n) and wave_shr:1.
enum : int { kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118, kWaveShr1 = 0x138 };

// Inclusive scan over the 64 lanes: Hillis-Steele inside each 16-lane row,
// then row 0's total into row 1 and row 2's into row 3, then row 1's running
// total into rows 2 and 3. Lanes whose DPP source does not exist read the
// identity.
template <typename Op> __device__ __forceinline__ float wave_inclusive_scan(float v) {
    const float id = Op::identity();
    v = Op::combine(v, wave::dpp<kRowShr1>(id, v));
    v = Op::combine(v, wave::dpp<kRowShr2>(id, v));
    v = Op::combine(v, wave::dpp<kRowShr4>(id, v));
    v = Op::combine(v, wave::dpp<kRowShr8>(id, v));
    v = Op::combine(v, wave::dpp<wave::kRowBcast15, 0xa>(id, v));
    v = Op::combine(v, wave::dpp<wave::kRowBcast31, 0xc>(id, v));
    return v;
}

// The value of lane - 1 (identity in lane 0).
template <typename Op> __device__ __forceinline__ float wave_shift_up(float v) {
    return wave::dpp<kWaveShr1>(Op::identity(), v);
}

// Loads the pack of 4 elements starting at element `e` (of n), identity past
// the end; 16-byte non-temporal loads when the pointer allows and the pack is
// whole (the input streams through once per pass).
template <typename Op, bool kPacked>
__device__ __forceinline__ f32x4 scan_load(const float *in, int64_t e, int64_t n) {
    if (kPacked && e + 4 <= n)
        return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(in + e));
    f32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        v[k] = e + k < n ? in[e + k] : Op::identity();
    return v;
}

template <typename Op, bool kPacked>
__global__ __launch_bounds__(kScanThreads) void scan_tile_reduce_kernel(const float *__restrict__ in,
                                                                        float *__restrict__ partial, int64_t n) {
    const int64_t base = int64_t(blockIdx.x) * kScanTile + 4 * threadIdx.x;
    f32x4 v[kScanRounds];
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r)
        v[r] = scan_load<Op, kPacked>(in, base + int64_t(r) * kScanRound, n);
    float acc = Op::identity();
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r)
        acc = Op::combine(acc, Op::combine(Op::combine(v[r][0], v[r][1]), Op::combine(v[r][2], v[r][3])));
    acc = wave::reduce(acc, Op::identity(), [](float a, float b) { return Op::combine(a, b); });
    __shared__ float totals[kScanThreads / kWaveSize];
    const int wid = threadIdx.x / kWaveSize;
    if (threadIdx.x % kWaveSize == 0)
        totals[wid] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = Op::identity();
#pragma unroll
        for (int w = 0; w < kScanThreads / kWaveSize; ++w)
            t = Op::combine(t, totals[w]);
        partial[blockIdx.x] = t;
    }
}

// partial[0..count) -> exclusive prefixes, in place. Lane t owns the
// contiguous run [t * per, (t + 1) * per) with per a multiple of 4, which it
// reads as 16-byte packs, kScanPartialBatch per round trip, and keeps in
// registers between the run total and the rewrite.
template <typename Op>
__global__ __launch_bounds__(kScanPartialThreads) void scan_partials_kernel(float *__restrict__ partial, int count) {
    constexpr int kWaves = kScanPartialThreads / kWaveSize;
    constexpr int kPer = 4 * kScanPartialBatch;
    const int per = ((count + kScanPartialThreads - 1) / kScanPartialThreads + 3) / 4 * 4;
    const int begin = threadIdx.x * per;
    const int end = begin + per < count ? begin + per : count;
    auto load_batch = [&](int b, f32x4 *v) {
#pragma unroll
        for (int j = 0; j < kScanPartialBatch; ++j) {
            const int i = b + 4 * j;
            if (i + 4 <= end) {
                v[j] = *reinterpret_cast<const f32x4 *>(partial + i);
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    v[j][k] = i + k < end ? partial[i + k] : Op::identity();
            }
        }
    };
    float run = Op::identity();
    for (int b = begin; b < end; b += kPer) {
        f32x4 v[kScanPartialBatch];
        load_batch(b, v);
#pragma unroll
        for (int j = 0; j < kScanPartialBatch; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                run = Op::combine(run, v[j][k]);
    }
    const float incl = wave_inclusive_scan<Op>(run);
    const float excl = wave_shift_up<Op>(incl);
    __shared__ float wave_tot[kWaves];
    const int wid = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    if (lane == kWaveSize - 1)
        wave_tot[wid] = incl;
    __syncthreads();
    float prefix = Op::identity();
    for (int w = 0; w < wid; ++w)
        prefix = Op::combine(prefix, wave_tot[w]);
    prefix = Op::combine(prefix, excl);
    for (int b = begin; b < end; b += kPer) {
        f32x4 v[kScanPartialBatch];
        load_batch(b, v);
#pragma unroll
        for (int j = 0; j < kScanPartialBatch; ++j) {
            const int i = b + 4 * j;
            f32x4 y;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                y[k] = prefix;
                prefix = Op::combine(prefix, v[j][k]);
            }
            if (i + 4 <= end) {
                *reinterpret_cast<f32x4 *>(partial + i) = y;
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (i + k < end)
                        partial[i + k] = y[k];
            }
        }
    }
}

// `tile_prefix` is null for a single-tile scan (prefix = identity).
template <typename Op, bool kPacked, bool kInclusive>
__global__ __launch_bounds__(kScanThreads) void scan_tile_kernel(const float *in, float *out,
                                                                 const float *__restrict__ tile_prefix, int64_t n) {
    constexpr int kWaves = kScanThreads / kWaveSize;
    __shared__ float wave_tot[kScanRounds][kWaves];
    const int wid = threadIdx.x / kWaveSize;
    const int64_t tile = int64_t(blockIdx.x) * kScanTile;
    float carry = tile_prefix ? tile_prefix[blockIdx.x] : Op::identity();
    f32x4 x[kScanRounds];
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r)
        x[r] = scan_load<Op, kPacked>(in, tile + int64_t(r) * kScanRound + 4 * threadIdx.x, n);
    // lane and wave scans of all rounds first, so one barrier serves the tile
    f32x4 s[kScanRounds];
    float lane_excl[kScanRounds];
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r) {
        s[r][0] = x[r][0];
        s[r][1] = Op::combine(s[r][0], x[r][1]);
        s[r][2] = Op::combine(s[r][1], x[r][2]);
        s[r][3] = Op::combine(s[r][2], x[r][3]);
        const float incl = wave_inclusive_scan<Op>(s[r][3]);
        lane_excl[r] = wave_shift_up<Op>(incl);
        if (threadIdx.x % kWaveSize == kWaveSize - 1)
            wave_tot[r][wid] = incl;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r) {
        float before = carry, round_total = carry;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            if (w < wid)
                before = Op::combine(before, wave_tot[r][w]);
            round_total = Op::combine(round_total, wave_tot[r][w]);
        }
        const float base = Op::combine(before, lane_excl[r]);
        f32x4 y;
        if constexpr (kInclusive) {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                y[k] = Op::combine(base, s[r][k]);
        } else {
            y[0] = base;
#pragma unroll
            for (int k = 1; k < 4; ++k)
                y[k] = Op::combine(base, s[r][k - 1]);
        }
        const int64_t e = tile + int64_t(r) * kScanRound + 4 * threadIdx.x;
        if (kPacked && e + 4 <= n) {
            __builtin_nontemporal_store(y, reinterpret_cast<f32x4 *>(out + e));
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (e + k < n)
                    out[e + k] = y[k];
        }
        carry = round_total;
    }
}

inline int scan_tile_count(int n) { return static_cast<int>(blocks_for64(n, kScanTile)); }

template <typename Op, bool kPacked, bool kInclusive>
void scan_launch(const float *in, float *out, int n, float *partial, hipStream_t stream) {
    const int tiles = scan_tile_count(n);
    if (tiles <= 1) {
        launch_async(stream, scan_tile_kernel<Op, kPacked, kInclusive>, 1, kScanThreads, in, out,
                     static_cast<const float *>(nullptr), static_cast<int64_t>(n));
        return;
    }
    launch_async(stream, scan_tile_reduce_kernel<Op, kPacked>, tiles, kScanThreads, in, partial,
                 static_cast<int64_t>(n));
    launch_async(stream, scan_partials_kernel<Op>, 1, kScanPartialThreads, partial, tiles);
    launch_async(stream, scan_tile_kernel<Op, kPacked, kInclusive>, tiles, kScanThreads, in, out,
                 static_cast<const float *>(partial), static_cast<int64_t>(n));
}

template <typename Op>
void scan_dispatch(const float *in, float *out, int n, bool inclusive, float *partial, hipStream_t stream) {
    const bool packed = aligned16(in) && aligned16(out);
    if (packed && inclusive)
        scan_launch<Op, true, true>(in, out, n, partial, stream);
    else if (packed)
        scan_launch<Op, true, false>(in, out, n, partial, stream);
    else if (inclusive)
        scan_launch<Op, false, true>(in, out, n, partial, stream);
    else
        scan_launch<Op, false, false>(in, out, n, partial, stream);
}

} // namespace opworks::detail

namespace opworks::ops {

// Workspace size in floats: one per 8192-element tile, 0 for a single tile.
inline int scan_workspace_size(int n) {
    detail::validate_size(n);
    const int tiles = detail::scan_tile_count(n);
    return tiles <= 1 ? 0 : tiles;
}

// Allocation-free asynchronous path; capturable into a HIP graph. `maximum`
// selects the prefix maximum, else the prefix sum. The workspace must stay
// alive until the stream completes and must not overlap the input or output.
inline void scan(const float *in, float *out, int n, bool maximum, bool inclusive, DeviceSpan<float> workspace,
                 hipStream_t stream = nullptr) {
    const int need = scan_workspace_size(n);
    if (n == 0)
        return;
    detail::require(in && out, "scan requires non-null pointers");
    detail::require(workspace.size() >= need, "scan workspace is too small");
    detail::require(need == 0 || detail::aligned16(workspace.data()), "scan workspace must be 16-byte aligned");
    if (maximum)
        detail::scan_dispatch<detail::ScanMaxOp>(in, out, n, inclusive, workspace.data(), stream);
    else
        detail::scan_dispatch<detail::ScanSumOp>(in, out, n, inclusive, workspace.data(), stream);
}

// Convenience path: stream-ordered scratch (hipMallocAsync / hipFreeAsync).
inline void scan(const float *in, float *out, int n, bool maximum, bool inclusive, hipStream_t stream = nullptr) {
    const int need = scan_workspace_size(n);
    if (n == 0)
        return;
    detail::require(in && out, "scan requires non-null pointers");
    float *scratch = nullptr;
    if (need != 0)
        OPWORKS_HIP_CHECK(hipMallocAsync(reinterpret_cast<void **>(&scratch), sizeof(float) * need, stream));
    scan(in, out, n, maximum, inclusive, DeviceSpan<float>(scratch, need), stream);
    if (scratch)
        OPWORKS_HIP_CHECK(hipFreeAsync(scratch, stream));
}

} // namespace opworks::ops

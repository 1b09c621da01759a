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
// gfx950 design: one pass over tiles of kScanTile elements. Each workgroup
// takes the next tile index from a counter (so every lower tile is already
// running or done), loads its tile into registers, publishes the tile total,
// then builds its tile prefix from totals published by lower tiles:
//   prefix(t) = S(super groups before t's) (+) G(groups before t's in its
//               super group) (+) T(tiles before t in its group),
// with 64 tiles to a group and 64 groups to a super group. Each of the three
// terms is one wave's inclusive scan over at most 64 published values, so
// its association is fixed by the tile index alone: the result is the same
// bit pattern on every run, whatever order the workgroups ran in. The last
// tile of a group publishes the group total (a scan over its 64 tile totals)
// and the last group's last tile the super-group total, so no tile waits on
// a chain longer than three levels. Totals travel as 64-bit words holding the
// value and a valid flag, written and read with agent-scope atomics (sc1
// accesses, coherent across the XCDs' L2 caches). Every wait is on a lower
// tile, bounded, and counts a timeout into the workspace.
//
// A fill kernel clears the counter and the flags before each scan, so the
// workspace can be any caller memory. The tile then rescans its elements in
// four rounds of 2048 contiguous elements: a lane scans its 16-byte pack, a
// wave scans the lane totals with DPP row shifts and row broadcasts, LDS
// carries the wave totals, and the tile prefix enters as the first operand.
// Inputs of at most one tile take a single workgroup and need no workspace.
// HBM traffic is 8 B per element (one read, one write), the compulsory
// amount. In-place scans (out == in) are allowed: every element is read by
// the lane that later writes it, before the write.

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

inline int scan_tile_count(int n) { return static_cast<int>(blocks_for64(n, kScanTile)); }

// Workspace, in 32-bit words from a 16-byte aligned base: word 0 the tile
// counter, word 1 the count of waits that timed out (both on a 256-byte line
// of their own), then the tile totals, the group totals and the super-group
// totals, one 64-bit word each: value bits in the low half, 1 in the high
// half once published, 0 while not.
constexpr int kScanGroup = 64;          // tiles per group, groups per super group
constexpr int kScanHeaderWords = 64;
constexpr int kScanSpinLimit = 1 << 18; // polls before a wait gives up (a fraction of a second)

struct ScanLayout {
    int tiles, groups, supers;
    __host__ __device__ int64_t words() const { return kScanHeaderWords + 2 * (int64_t(tiles) + groups + supers); }
};

inline ScanLayout scan_layout(int n) {
    const int tiles = scan_tile_count(n);
    const int groups = (tiles + kScanGroup - 1) / kScanGroup;
    return {tiles, groups, (groups + kScanGroup - 1) / kScanGroup};
}

__device__ __forceinline__ uint64_t scan_publishable(float v) {
    return (uint64_t(1) << 32) | __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ void scan_publish(uint64_t *slot, float v) {
    __hip_atomic_store(slot, scan_publishable(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls a published total of a lower tile (agent-coherent 64-bit loads, so the value and its
// flag arrive together). A wait that outlasts kScanSpinLimit polls counts itself in `timeouts`
// and returns NaN, so a broken protocol ends the kernel and shows in the output.
__device__ __forceinline__ float scan_wait_total(const uint64_t *slot, uint32_t *timeouts) {
    for (int spin = 0;; ++spin) {
        const uint64_t w = __hip_atomic_load(const_cast<uint64_t *>(slot), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (w >> 32)
            return __builtin_bit_cast(float, uint32_t(w));
        if (spin == kScanSpinLimit) {
            __hip_atomic_fetch_add(timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return __builtin_nanf("");
        }
        __builtin_amdgcn_s_sleep(2);
    }
}

// Zeroes `quads` 16-byte words of the workspace: the counter, the timeout count and every flag.
__global__ __launch_bounds__(256) static void scan_clear_kernel(uint4 *ws, int64_t quads) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < quads)
        ws[i] = make_uint4(0u, 0u, 0u, 0u);
}

// One workgroup per tile. kOnePass = false: the single-tile scan (tile 0, no workspace).
template <typename Op, bool kPacked, bool kInclusive, bool kOnePass>
__global__ __launch_bounds__(kScanThreads) void scan_kernel(const float *in, float *out, uint32_t *ws,
                                                            ScanLayout lay, int64_t n) {
    constexpr int kWaves = kScanThreads / kWaveSize;
    __shared__ float wave_tot[kScanRounds][kWaves];
    __shared__ float level[3]; // exclusive prefixes over super groups, groups, tiles
    __shared__ float own_group_total;
    __shared__ int tile_id;
    const int wid = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    int t = 0;
    if constexpr (kOnePass) {
        if (threadIdx.x == 0)
            tile_id = __hip_atomic_fetch_add(reinterpret_cast<int *>(ws), 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        t = tile_id;
    }
    const int64_t tile = int64_t(t) * kScanTile;
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
        if (lane == kWaveSize - 1)
            wave_tot[r][wid] = incl;
    }
    __syncthreads();
    float carry = Op::identity();
    if constexpr (kOnePass) {
        // The tile total in a fixed order (rounds, then waves), published at once.
        float total = Op::identity();
#pragma unroll
        for (int r = 0; r < kScanRounds; ++r)
#pragma unroll
            for (int w = 0; w < kWaves; ++w)
                total = Op::combine(total, wave_tot[r][w]);
        uint64_t *tile_tot = reinterpret_cast<uint64_t *>(ws + kScanHeaderWords);
        uint64_t *group_tot = tile_tot + lay.tiles;
        uint64_t *super_tot = group_tot + lay.groups;
        uint32_t *timeouts = ws + 1;
        if (threadIdx.x == 0)
            scan_publish(tile_tot + t, total);
        const int g = t / kScanGroup, j = t % kScanGroup, sg = g / kScanGroup, gj = g % kScanGroup;
        const bool closes_group = j == kScanGroup - 1, closes_super = closes_group && gj == kScanGroup - 1;
        // Waves 0, 1, 2 scan the totals of the lower tiles in this group, the lower groups in this
        // super group and the lower super groups. Lane 63 of wave 0 carries this tile's own total,
        // which completes the group total when this is the group's last tile.
        float v = Op::identity();
        if (wid < 3) {
            const uint64_t *src = wid == 0 ? tile_tot + int64_t(g) * kScanGroup
                                  : wid == 1 ? group_tot + int64_t(sg) * kScanGroup
                                             : super_tot;
            const int count = wid == 0 ? j : wid == 1 ? gj : sg;
            if (lane < count)
                v = scan_wait_total(src + lane, timeouts);
            if (wid == 0 && lane == kWaveSize - 1)
                v = total;
            const float incl = wave_inclusive_scan<Op>(v);
            const float before = count == 0 ? Op::identity() : wave::readlane(incl, count - 1);
            if (lane == 0)
                level[wid] = before;
            if (wid == 0 && closes_group && lane == kWaveSize - 1) {
                scan_publish(group_tot + g, incl);
                own_group_total = incl;
            }
        }
        __syncthreads();
        if (closes_super && wid == 1) {
            const float incl = wave_inclusive_scan<Op>(lane == kWaveSize - 1 ? own_group_total : v);
            if (lane == kWaveSize - 1)
                scan_publish(super_tot + sg, incl);
        }
        carry = Op::combine(Op::combine(level[2], level[1]), level[0]);
    }
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

template <typename Op, bool kPacked, bool kInclusive>
void scan_launch(const float *in, float *out, int n, float *workspace, hipStream_t stream) {
    const ScanLayout lay = scan_layout(n);
    if (lay.tiles <= 1) {
        launch_async(stream, scan_kernel<Op, kPacked, kInclusive, false>, 1, kScanThreads, in, out,
                     static_cast<uint32_t *>(nullptr), lay, static_cast<int64_t>(n));
        return;
    }
    uint32_t *ws = reinterpret_cast<uint32_t *>(workspace);
    const int64_t quads = (lay.words() + 3) / 4;
    launch_async(stream, scan_clear_kernel, static_cast<int>(blocks_for64(quads, 256)), 256,
                 reinterpret_cast<uint4 *>(ws), quads);
    launch_async(stream, scan_kernel<Op, kPacked, kInclusive, true>, lay.tiles, kScanThreads, in, out, ws, lay,
                 static_cast<int64_t>(n));
}

template <typename Op>
void scan_dispatch(const float *in, float *out, int n, bool inclusive, float *workspace, hipStream_t stream) {
    const bool packed = aligned16(in) && aligned16(out);
    if (packed && inclusive)
        scan_launch<Op, true, true>(in, out, n, workspace, stream);
    else if (packed)
        scan_launch<Op, true, false>(in, out, n, workspace, stream);
    else if (inclusive)
        scan_launch<Op, false, true>(in, out, n, workspace, stream);
    else
        scan_launch<Op, false, false>(in, out, n, workspace, stream);
}

} // namespace opworks::detail

namespace opworks::ops {

// Workspace size in floats (32-bit words): 0 for a single tile of 8192
// elements, else a 64-word header plus two words per tile, per group of 64
// tiles and per super group of 4096 tiles, rounded up to a 16-byte multiple.
// Its contents on entry do not matter: each scan clears what it uses.
inline int scan_workspace_size(int n) {
    detail::validate_size(n);
    const detail::ScanLayout lay = detail::scan_layout(n);
    return lay.tiles <= 1 ? 0 : static_cast<int>((lay.words() + 3) / 4 * 4);
}

// Allocation-free asynchronous path; capturable into a HIP graph. `maximum`
// selects the prefix maximum, else the prefix sum. The workspace must stay
// alive until the stream completes and must not overlap the input or output;
// scans that share a workspace must not run at the same time.
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

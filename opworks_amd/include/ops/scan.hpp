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
// gfx950 design: one pass over units of elements: a pair of 8192-element
// tiles when input and output are 16-byte aligned (one tile in registers, the
// other loaded straight into LDS), else one tile. Each workgroup takes the
// next unit index from a counter (so every lower unit is already running or
// done), loads its unit, publishes the unit's total, then builds its prefix
// from totals published by lower units:
//   prefix(t) = S(super groups before t's) (+) G(groups before t's in its
//               super group) (+) T(units before t in its group),
// with 64 units to a group and 64 groups to a super group. Each of the three
// terms is one wave's inclusive scan over at most 64 published values, so
// its association is fixed by the unit index alone: the result is the same
// bit pattern on every run, whatever order the workgroups ran in. The last
// unit of a group publishes the group total (a scan over its 64 unit totals)
// and the last group's last unit the super-group total. A unit waits on unit
// and group totals of its own super group, which do not chain; the super-group
// totals do form a chain, since the unit that closes super group s publishes
// after its workgroup barrier, which follows its wait for the totals of super
// groups 0 .. s-1 (at most 2^31 / 2^26 = 32 links). Totals travel as 64-bit
// words holding the value and flags, written and read with agent-scope atomics
// (sc1 accesses, coherent across the XCDs' L2 caches). Every wait is on a lower
// unit and bounded: a wait that gives up counts a timeout into the workspace
// and poisons the unit, whose outputs are then NaN (for the prefix maximum as
// well, where a NaN operand would otherwise vanish in fmaxf), and so is every
// group or super-group total it publishes; a unit that reads a poisoned total
// is poisoned in turn.
//
// A fill kernel clears the counter and the flags before each scan, so the
// workspace can be any caller memory. A tile is then rescanned in four rounds
// of 2048 contiguous elements: a lane scans its 16-byte pack, a wave scans
// the lane totals with DPP row shifts and row broadcasts, LDS carries the
// wave totals, and the prefix enters as the first operand. Inputs of at most
// one unit take a single workgroup and need no workspace.
// HBM traffic is 8 B per element (one read, one write), the compulsory
// amount. In-place scans (out == in) are allowed: every element is read by
// the lane that later writes it, before the write.

#include <cmath>

#include "../core/device_span.hpp"
#include "../core/lds_direct.hpp"
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

// Workspace, in 32-bit words from a 16-byte aligned base: word 0 the unit
// counter, word 1 the count of waits that timed out (both on a 256-byte line
// of their own), then the unit totals, the group totals and the super-group
// totals, one 64-bit word each: value bits in the low half, 1 in the high
// half once published, 0 while not.
constexpr int kScanGroup = 64;          // units per group, groups per super group
constexpr int kScanHeaderWords = 64;
constexpr int kScanSpinLimit = 1 << 18; // polls before a wait gives up (a fraction of a second)

struct ScanLayout {
    int units, groups, supers; // units: pairs of tiles
    __host__ __device__ int64_t words() const { return kScanHeaderWords + 2 * (int64_t(units) + groups + supers); }
};

inline ScanLayout scan_pair_layout(int n) {
    const int pairs = static_cast<int>(blocks_for64(n, 2 * kScanTile));
    const int groups = (pairs + kScanGroup - 1) / kScanGroup;
    return {pairs, groups, (groups + kScanGroup - 1) / kScanGroup};
}

// High half of a published word: bit 0 = published, bit 1 = poisoned (the total depends on a
// wait that gave up).
constexpr uint32_t kScanPublished = 1u, kScanPoisoned = 2u;

__device__ __forceinline__ void scan_publish(uint64_t *slot, float v, bool poisoned = false) {
    const uint64_t flags = kScanPublished | (poisoned ? kScanPoisoned : 0u);
    __hip_atomic_store(slot, (flags << 32) | __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Polls a published total of a lower tile (agent-coherent 64-bit loads, so the value and its
// flags arrive together). A wait that outlasts `spin_limit` polls counts itself in `timeouts`,
// sets `poisoned` and returns NaN; so does reading a poisoned total, without the count.
__device__ __forceinline__ float scan_wait_total(const uint64_t *slot, uint32_t *timeouts, bool &poisoned,
                                                 int spin_limit = kScanSpinLimit) {
    for (int spin = 0;; ++spin) {
        const uint64_t w = __hip_atomic_load(const_cast<uint64_t *>(slot), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t flags = uint32_t(w >> 32);
        if (flags & kScanPublished) {
            if (flags & kScanPoisoned) {
                poisoned = true;
                return __builtin_nanf("");
            }
            return __builtin_bit_cast(float, uint32_t(w));
        }
        if (spin >= spin_limit) {
            __hip_atomic_fetch_add(timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            poisoned = true;
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

constexpr int kScanWaves = kScanThreads / kWaveSize;
constexpr int kScanPair = 2 * kScanTile; // elements of a unit (a pair of tiles)

// Lane and wave scans of a tile held as kScanRounds packs per lane: s = the lane's inclusive
// scan of each pack, lane_excl = the wave-exclusive prefix of its pack total, wave_tot[r][w] =
// wave w's round-r total (read after a barrier).
template <typename Op>
__device__ __forceinline__ void scan_tile_local(const f32x4 (&x)[kScanRounds], f32x4 (&s)[kScanRounds],
                                                float (&lane_excl)[kScanRounds], float (*wave_tot)[kScanWaves],
                                                int wid, int lane) {
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
}

// Writes the tile starting at element `base`: every output combines the running carry, the
// wave totals before it, its lane's prefix and its own pack scan; carry leaves as the carry
// into the next tile.
template <typename Op, bool kPacked, bool kInclusive>
__device__ __forceinline__ void scan_tile_emit(float *out, int64_t base, int64_t n, float &carry,
                                               const f32x4 (&s)[kScanRounds], const float (&lane_excl)[kScanRounds],
                                               const float (*wave_tot)[kScanWaves], int wid, bool poisoned = false) {
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r) {
        float before = carry, round_total = carry;
#pragma unroll
        for (int w = 0; w < kScanWaves; ++w) {
            if (w < wid)
                before = Op::combine(before, wave_tot[r][w]);
            round_total = Op::combine(round_total, wave_tot[r][w]);
        }
        const float b0 = Op::combine(before, lane_excl[r]);
        f32x4 y;
        if constexpr (kInclusive) {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                y[k] = Op::combine(b0, s[r][k]);
        } else {
            y[0] = b0;
#pragma unroll
            for (int k = 1; k < 4; ++k)
                y[k] = Op::combine(b0, s[r][k - 1]);
        }
        if (poisoned)
            y = f32x4{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
        const int64_t e = base + int64_t(r) * kScanRound + 4 * threadIdx.x;
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

// LDS of the prefix protocol.
struct ScanPrefixLds {
    float level[3]; // exclusive prefixes over super groups, groups, units
    float own_group_total;
    int poisoned[3]; // the wave's level depends on a wait that gave up
};

// The exclusive prefix of unit t whose total is `total` (every thread calls this; it
// publishes the unit's total and, for the last unit of a group or super group, that total).
// `poisoned` is set in every thread when the prefix depends on a wait that gave up; the
// returned prefix is then NaN.
template <typename Op>
__device__ __forceinline__ float scan_unit_prefix(uint32_t *ws, const ScanLayout &lay, int t, float total,
                                                  ScanPrefixLds &sh, int wid, int lane, bool &poisoned,
                                                  int spin_limit = kScanSpinLimit) {
    uint64_t *unit_tot = reinterpret_cast<uint64_t *>(ws + kScanHeaderWords);
    uint64_t *group_tot = unit_tot + lay.units;
    uint64_t *super_tot = group_tot + lay.groups;
    uint32_t *timeouts = ws + 1;
    if (threadIdx.x == 0)
        scan_publish(unit_tot + t, total);
    const int g = t / kScanGroup, j = t % kScanGroup, sg = g / kScanGroup, gj = g % kScanGroup;
    const bool closes_group = j == kScanGroup - 1, closes_super = closes_group && gj == kScanGroup - 1;
    // Waves 0, 1, 2 scan the totals of the lower units in this group, the lower groups in this
    // super group and the lower super groups. Lane 63 of wave 0 carries this unit's own total,
    // which completes the group total when this is the group's last unit.
    float v = Op::identity();
    if (wid < 3) {
        const uint64_t *src = wid == 0 ? unit_tot + int64_t(g) * kScanGroup
                              : wid == 1 ? group_tot + int64_t(sg) * kScanGroup
                                         : super_tot;
        const int count = wid == 0 ? j : wid == 1 ? gj : sg;
        bool lane_bad = false;
        if (lane < count)
            v = scan_wait_total(src + lane, timeouts, lane_bad, spin_limit);
        if (wid == 0 && lane == kWaveSize - 1)
            v = total;
        const bool wave_bad = __builtin_amdgcn_ballot_w64(lane_bad) != 0;
        const float incl = wave_inclusive_scan<Op>(v);
        const float before = count == 0 ? Op::identity() : wave::readlane(incl, count - 1);
        if (lane == 0) {
            sh.level[wid] = before;
            sh.poisoned[wid] = wave_bad;
        }
        if (wid == 0 && closes_group && lane == kWaveSize - 1) {
            scan_publish(group_tot + g, incl, wave_bad);
            sh.own_group_total = incl;
        }
    }
    __syncthreads();
    if (closes_super && wid == 1) {
        const float incl = wave_inclusive_scan<Op>(lane == kWaveSize - 1 ? sh.own_group_total : v);
        if (lane == kWaveSize - 1)
            scan_publish(super_tot + sg, incl, sh.poisoned[0] || sh.poisoned[1]);
    }
    poisoned = sh.poisoned[0] || sh.poisoned[1] || sh.poisoned[2];
    if (poisoned)
        return __builtin_nanf("");
    return Op::combine(Op::combine(sh.level[2], sh.level[1]), sh.level[0]);
}

__device__ __forceinline__ int scan_take_unit(uint32_t *ws, int *slot) {
    if (threadIdx.x == 0)
        *slot = __hip_atomic_fetch_add(reinterpret_cast<int *>(ws), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    return *slot;
}

// A scan of at most one tile: one workgroup, no workspace.
template <typename Op, bool kPacked, bool kInclusive>
__global__ __launch_bounds__(kScanThreads) void scan_kernel(const float *in, float *out, int64_t n) {
    __shared__ float wave_tot[kScanRounds][kScanWaves];
    const int wid = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    f32x4 x[kScanRounds];
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r)
        x[r] = scan_load<Op, kPacked>(in, int64_t(r) * kScanRound + 4 * threadIdx.x, n);
    f32x4 s[kScanRounds];
    float lane_excl[kScanRounds];
    scan_tile_local<Op>(x, s, lane_excl, wave_tot, wid, lane);
    __syncthreads();
    float carry = Op::identity();
    scan_tile_emit<Op, kPacked, kInclusive>(out, 0, n, carry, s, lane_excl, wave_tot, wid);
}

// One workgroup per pair of tiles: tile A is loaded into registers and tile B into LDS
// (straight from global memory when the input is 16-byte aligned and the tile is whole), so a
// workgroup holds 64 KB at the register cost of 32 KB and twice the bytes are in flight while
// units wait for their prefixes (2^28 elements: 498 -> 410 us against one tile per workgroup).
// The pair's total is A's total then B's; B's outputs continue A's carry. Aligned and unaligned
// inputs take the same steps, so their results are the same bits. kOnePass = false: a single
// pair, no workspace.
template <typename Op, bool kPacked, bool kInclusive, bool kOnePass>
__global__ __launch_bounds__(kScanThreads) void scan_pair_kernel(const float *in, float *out, uint32_t *ws,
                                                                 ScanLayout lay, int64_t n, int spin_limit) {
    __shared__ float wave_tot[kScanRounds][kScanWaves];
    __shared__ float wave_tot_b[kScanWaves];
    __shared__ ScanPrefixLds sh;
    __shared__ int unit;
    __shared__ __attribute__((aligned(16))) float tile_b[kScanTile];
    const int wid = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    if (n < 0) // never runs: an ordinary store, so the compiler treats tile_b as written
        tile_b[threadIdx.x] = 0.f;
    const int t = kOnePass ? scan_take_unit(ws, &unit) : 0;
    const int64_t base_a = int64_t(t) * kScanPair, base_b = base_a + kScanTile;
    // Tile B: wave instruction i fills the 1 KB block 8 i + wave of the tile; a tile that
    // ends past n is loaded through registers instead, with the identity past the end.
    const bool b_whole = kPacked && base_b + kScanTile <= n;
    if (b_whole) {
#pragma unroll
        for (int i = 0; i < kScanTile / (256 * kScanWaves); ++i) {
            const int blk = kScanWaves * i + wid;
            load_lds16(in + base_b + 256 * blk + 4 * lane, tile_b + 256 * blk);
        }
    }
    f32x4 x[kScanRounds];
#pragma unroll
    for (int r = 0; r < kScanRounds; ++r)
        x[r] = scan_load<Op, kPacked>(in, base_a + int64_t(r) * kScanRound + 4 * threadIdx.x, n);
    if (!b_whole) {
#pragma unroll
        for (int r = 0; r < kScanRounds; ++r)
            *reinterpret_cast<f32x4 *>(tile_b + r * kScanRound + 4 * threadIdx.x) =
                scan_load<Op, kPacked>(in, base_b + int64_t(r) * kScanRound + 4 * threadIdx.x, n);
    }
    f32x4 s[kScanRounds];
    float lane_excl[kScanRounds];
    scan_tile_local<Op>(x, s, lane_excl, wave_tot, wid, lane);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0Only); // this wave's direct loads of tile B have landed
    __syncthreads();
    {   // tile B's total, read from LDS in the order the output pass reads it
        float bsum = Op::identity();
#pragma unroll
        for (int r = 0; r < kScanRounds; ++r) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(tile_b + r * kScanRound + 4 * threadIdx.x);
            bsum = Op::combine(bsum, Op::combine(Op::combine(v[0], v[1]), Op::combine(v[2], v[3])));
        }
        bsum = wave::reduce(bsum, Op::identity(), [](float p, float q) { return Op::combine(p, q); });
        if (lane == 0)
            wave_tot_b[wid] = bsum;
    }
    __syncthreads();
    float carry = Op::identity();
    bool poisoned = false;
    if constexpr (kOnePass) {
        float total_a = Op::identity(), total_b = Op::identity();
#pragma unroll
        for (int r = 0; r < kScanRounds; ++r)
#pragma unroll
            for (int w = 0; w < kScanWaves; ++w)
                total_a = Op::combine(total_a, wave_tot[r][w]);
#pragma unroll
        for (int w = 0; w < kScanWaves; ++w)
            total_b = Op::combine(total_b, wave_tot_b[w]);
        carry = scan_unit_prefix<Op>(ws, lay, t, Op::combine(total_a, total_b), sh, wid, lane, poisoned, spin_limit);
    }
    scan_tile_emit<Op, kPacked, kInclusive>(out, base_a, n, carry, s, lane_excl, wave_tot, wid, poisoned);
    __syncthreads(); // tile A's wave totals have been read
    {
        f32x4 xb[kScanRounds];
#pragma unroll
        for (int r = 0; r < kScanRounds; ++r)
            xb[r] = *reinterpret_cast<const f32x4 *>(tile_b + r * kScanRound + 4 * threadIdx.x);
        scan_tile_local<Op>(xb, s, lane_excl, wave_tot, wid, lane);
    }
    __syncthreads();
    scan_tile_emit<Op, kPacked, kInclusive>(out, base_b, n, carry, s, lane_excl, wave_tot, wid, poisoned);
}


template <typename Op, bool kPacked, bool kInclusive>
void scan_launch(const float *in, float *out, int n, float *workspace, hipStream_t stream) {
    if (n <= kScanTile) {
        launch_async(stream, scan_kernel<Op, kPacked, kInclusive>, 1, kScanThreads, in, out, static_cast<int64_t>(n));
        return;
    }
    const ScanLayout lay = scan_pair_layout(n);
    if (lay.units == 1) {
        launch_async(stream, scan_pair_kernel<Op, kPacked, kInclusive, false>, 1, kScanThreads, in, out,
                     static_cast<uint32_t *>(nullptr), lay, static_cast<int64_t>(n), kScanSpinLimit);
        return;
    }
    uint32_t *ws = reinterpret_cast<uint32_t *>(workspace);
    const int64_t quads = (lay.words() + 3) / 4;
    launch_async(stream, scan_clear_kernel, static_cast<int>(blocks_for64(quads, 256)), 256,
                 reinterpret_cast<uint4 *>(ws), quads);
    launch_async(stream, scan_pair_kernel<Op, kPacked, kInclusive, true>, lay.units, kScanThreads, in, out, ws, lay,
                 static_cast<int64_t>(n), kScanSpinLimit);
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

// Workspace size in floats (32-bit words): 0 up to one pair of 8192-element
// tiles (16384 elements), else a 64-word header plus two words per pair, per
// group of 64 pairs and per super group of 4096 pairs, rounded up to a
// 16-byte multiple. Its contents on entry do not matter: each scan clears
// what it uses.
inline int scan_workspace_size(int n) {
    detail::validate_size(n);
    const detail::ScanLayout lay = detail::scan_pair_layout(n);
    return lay.units <= 1 ? 0 : static_cast<int>((lay.words() + 3) / 4 * 4);
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

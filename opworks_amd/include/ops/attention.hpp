#pragma once

// Causal GQA attention over a KV cache, fp32.
//
// Layouts (reference: include/ops/attention_prefill.cuh:21-24,
// include/ops/attention_decode.cuh:8-11):
//   q_heads [qh][T][D]   queries at absolute positions q_offset + [0, T)
//   k/v cache [kvh][cap][D], S valid entries; kv head of q head h = h / kv_rep
//   out [qh][T][D]
// A query at position p sees keys 0..min(p, S-1); scores are scaled by
// 1/sqrt(D); a row that sees no key writes zeros.
//
// ---- prefill (flash) -----------------------------------------------------
// One workgroup = one kv head x one 16-query tile, with one wave per q head of
// the GQA group, so each 32-key K/V tile is read from HBM once per group and
// shared through LDS (double buffered). Each wave computes the transposed
// products
//   S^T = K Q^T  and  O^T += V^T P^T
// on v_mfma_f32_16x16x4_f32. In that orientation lane l owns query l % 16 in
// every tile: the running max is a register reduction plus a combine over the
// four 16-lane rows (permlane swaps), the row sum stays per lane until the
// end, and the rescale of O is a per-lane multiply. In the QK^T chain lane
// group g supplies reduction index (D/4) g + s at step s; its S^T accumulator
// register r is key 4g + r of the block, which is exactly the P^T operand it
// supplies at step r of the P V chain, so P never moves. Q stays in registers,
// pre-scaled by scale * log2(e) so the softmax is exp2.
// 16-query tiles keep the longest serial chain (the last tile, over all S
// keys) at half the MFMA work of a 32-query tile and give four resident
// workgroups per CU; tiles are dispatched heaviest first in alternating passes
// (prefill_tile_of_rank) so each CU's share of KV tiles is about equal.
// With head_dim 32 or 64 the same products run on bf16 MFMAs with every operand
// split into three bf16 parts ("bf16x6", fp32 accuracy): K and V are split once
// when staged, Q once per workgroup, P once per tile.
//
// ---- decode (split-KV) ---------------------------------------------------
// One workgroup = one kv head x one chunk of kAttnChunk keys: the chunk's K/V
// rows are read once for all q heads of the group, each wave (one q head)
// produces a partial (max, sum, unnormalised output) for the chunk, and a
// combine kernel merges the chunks. The valid length can be read from device
// memory, so one graph serves every decode position.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <type_traits>

#include "../core/bf16.hpp"
#include "../core/bf16x6.hpp"
#include "../core/hip_utils.hpp"
#include "../core/wave.hpp"
#include "elementwise.hpp"
#include "gemm_f32.hpp"

namespace opworks::detail {

constexpr int kAttnQTile = 16;     // queries per wave (columns of a 16x16 MFMA tile)
constexpr int kAttnKTile = 32;     // keys per staged K/V tile (two 16-key MFMA row blocks)
constexpr int kAttnMaxD = 64;
constexpr int kAttnMaxRep = 16;    // q heads per kv head (waves per decode workgroup)
constexpr float kLog2e = 1.4426950408889634f;

// ints from one kv head's arrival counter to the next (256 B): every counter sits on a cache
// line of its own, so the chunk workgroups of different kv heads never queue behind each
// other's atomics on one line (at 2048 keys: 8.35 against 10.4 us per fused call).
constexpr int kAttnCounterStride = 64;

// s_waitcnt operand of gfx9 for vmcnt(0) with expcnt and lgkmcnt left at their maxima
// (vmcnt bits [3:0] and [15:14] = 0, expcnt [6:4] = 7, lgkmcnt [11:8] = 15): waits until
// every vector memory access of the wave, stores included, has completed.
constexpr int kWaitVmcnt0 = 0x0F70;

template <bool kCoherent> __device__ __forceinline__ float record_load(const float *p) {
    if constexpr (kCoherent)
        return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        return *p;
}
template <bool kCoherent> __device__ __forceinline__ void record_store(float *p, float v) {
    if constexpr (kCoherent)
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}

// c(x[l], x[l ^ 16]) then c(., .[l ^ 32]): the combine over the four 16-lane
// rows of a wave, by gfx950's v_permlane16_swap / v_permlane32_swap (a VGPR
// exchange between rows, no LDS round trip). Both lanes of a pair combine the
// operands in the same order, so every lane of a column ends bit-identical.
template <typename Combine> __device__ __forceinline__ float column_combine(float v, Combine c) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = c(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return c(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// kDT = head_dim / 16 (16-wide head-dim tiles); kWaves = q heads handled by
// one workgroup (a GQA group, or an 8-head slice of a larger one); kTiles =
// adjacent query tiles per workgroup, one wave per (tile, head): with 2 every
// staged K/V tile feeds twice as many MFMA chains (used when the grid still
// fills every CU's four workgroup slots).
template <int kDT, int kWaves, int kTiles, bool kX6 = false> struct PrefillShape {
    static constexpr int kD = 16 * kDT;                        // head_dim
    static constexpr int kLd = kD + 4;                         // LDS row stride of K and V (floats)
    static constexpr int kThreads = kTiles * kWaves * kWaveSize;
    static constexpr int kChunks = kAttnKTile * kD / 4;        // 16-byte chunks per K (or V) tile
    static constexpr int kPerThread = (kChunks + kThreads - 1) / kThreads;
    static constexpr int kQ = kD / 4;                          // Q values per lane = QK^T MFMA steps per block
    // kX6 stage: K as three bf16 parts [part][key][kRowK] and V transposed as three parts
    // [part][dim][kRowV], rows unpadded with their 16-byte chunks XOR-swizzled (x6_k_chunk,
    // x6_v_chunk)
    static constexpr int kRowK = kD, kRowV = kAttnKTile;                     // bf16 elements
    static constexpr int kStageX6 = 3 * kAttnKTile * kRowK + 3 * kD * kRowV;  // bf16 elements per stage
    static constexpr int kLdsBytes = kX6 ? 2 * 2 * kStageX6 : 4 * 4 * kAttnKTile * kLd; // double buffered
};

// fp32 products on bf16 MFMAs ("bf16x6"): core/bf16x6.hpp.
// Key slot of V^T rows: lane group g's eight keys of a 32-key tile (16 (j / 4) + 4 g + j % 4,
// the keys its S^T registers hold) sit at slots 8 g + j, so one 16-byte read fetches them.
__device__ __forceinline__ int x6_key_slot(int key) { return 8 * ((key % 16) / 4) + 4 * (key / 16) + key % 4; }

// Dispatch order of query tiles. Work per tile grows with its index (causal),
// and the grid is the query tiles x kv heads (x head slices). Ranks go out in
// passes of `pass_width` tiles (one workgroup per CU per pass); passes run
// from the heaviest tiles down, alternating direction, so the workgroups one
// CU receives from successive passes sum to about the same number of KV tiles.
__device__ __forceinline__ int prefill_tile_of_rank(int rank, int ntq, int pass_width) {
    const int pass = rank / pass_width, c = rank % pass_width;
    const int width = min(pass_width, ntq - pass * pass_width);
    const int pos = pass * pass_width + ((pass & 1) ? width - 1 - c : c);
    return ntq - 1 - pos;
}

// ---- split of the heaviest query-tile groups (workspace form) --------------
// A causal grid's last query tiles carry the longest K/V ranges. Measured per CU, a CU whose
// heavier workgroup ran 56-64 K/V tiles finished 6-8% after the others: once its lighter
// workgroup is done, one 8-wave workgroup runs the long chain alone. In the workspace form the
// groups with more than `thr` K/V tiles run as two workgroups, one per half of the range, and the
// one that finishes last merges the halves. Units go out in descending order of work (a half
// counts n/2 tiles), so the big units start first and the small ones fill the slots that free up.
struct PrefillGeom {
    int kTiles, ntq, S, q_offset;
    // K/V tiles of query-tile group g: its last query tile's causal range
    __host__ __device__ int tiles(int g) const {
        const int last = g * kTiles + kTiles - 1 < ntq - 1 ? g * kTiles + kTiles - 1 : ntq - 1;
        const int end = q_offset + last * kAttnQTile + kAttnQTile;
        return ((end < S ? end : S) + kAttnKTile - 1) / kAttnKTile;
    }
    // First tile of the second half: half the range, and no later than the group's first query
    // position, so every query row of the group sees the second half's first key.
    __host__ __device__ int split_point(int g) const {
        const int half = tiles(g) / 2, first = (q_offset + g * kTiles * kAttnQTile) / kAttnKTile;
        return half < first ? half : first;
    }
    __host__ __device__ bool is_split(int g, int thr) const { return tiles(g) > thr && split_point(g) >= 1; }
    // The split groups are a suffix of the group indices (tiles and split point never decrease
    // with g): the first of them, or ngroups if none.
    __host__ __device__ int first_split(int ngroups, int thr) const {
        int lo = 0, hi = ngroups;
        while (lo < hi) {
            const int mid = (lo + hi) / 2;
            if (is_split(mid, thr))
                hi = mid;
            else
                lo = mid + 1;
        }
        return lo;
    }
};

struct PrefillUnit {
    int g;        // query-tile group
    int half;     // -1: the whole K/V range; 0 or 1: a half
    int kt_begin, kt_end;
    int slot;     // split groups only: g - first split group
};

// Unit of dispatch rank r: the halves (key n tiles each, groups from the last down, half 0 first)
// merged with the unsplit groups (key 2n, from gs - 1 down) in descending key order, ties to the
// halves. The number i of halves among the first r units comes from a binary search along the
// merge path.
__device__ __forceinline__ PrefillUnit prefill_unit_of_rank(int r, int ngroups, int thr, const PrefillGeom &geo) {
    const int gs = geo.first_split(ngroups, thr);
    const int na = 2 * (ngroups - gs), nb = gs;
    auto key_a = [&](int i) { return geo.tiles(ngroups - 1 - i / 2); };
    auto key_b = [&](int j) { return 2 * geo.tiles(gs - 1 - j); };
    int lo = r - nb > 0 ? r - nb : 0, hi = r < na ? r : na;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (mid == 0 || r - mid == nb || key_a(mid - 1) >= key_b(r - mid))
            lo = mid;
        else
            hi = mid - 1;
    }
    const int i = lo, j = r - i;
    if (i < na && (j == nb || key_a(i) >= key_b(j))) {
        const int g = ngroups - 1 - i / 2, half = i % 2, h = geo.split_point(g);
        return {g, half, half ? h : 0, half ? geo.tiles(g) : h, g - gs};
    }
    const int g = gs - 1 - j;
    return {g, -1, 0, geo.tiles(g), 0};
}

// Merge state of the split units: per (split group, kv head x slice) workgroup pair, two records
// of kRec x threads floats ([value][thread], coalesced) and one arrival counter on a 256-byte line
// of its own, zero between launches (the merging workgroup resets it).
struct PrefillSplit {
    float *rec;
    int *counters;
    int thr;       // groups with more K/V tiles than this split (when their split point is >= 1)
    int alternate; // nonzero: units go out in passes of alternating direction, not in descending order
};

// Where output row q of head h goes: element h * head_stride + q * row_stride, then head_dim
// consecutive values, fp32 or (bf16 != 0) rounded to bf16 nearest-even. The reference's layout
// [qh][T][D] is head_stride T * D, row_stride D; [T][qh * D] (the heads merged, as the output
// projection reads them) is head_stride D, row_stride qh * D.
struct PrefillOut {
    int64_t head_stride, row_stride;
    int bf16;
};

// amdgpu_waves_per_eu: with four or more waves per workgroup the register budget is 128
// (four resident waves per SIMD, as many as the LDS allows); the bound also makes the
// compiler keep the MFMA accumulators in VGPRs rather than AGPRs. kSplit: the workspace form
// (units from prefill_unit_of_rank, halves merged through `sp`). kX6: QK^T and P V on bf16
// MFMAs with every operand in three parts (the bf16x6 products above; head_dim 32 or 64).
template <int kDT, int kWaves, int kTiles, bool kSplit = false, bool kX6 = false>
__global__ __launch_bounds__(kTiles *kWaves *kWaveSize)
__attribute__((amdgpu_waves_per_eu(kWaves >= 4 ? 4 : 2, kWaves >= 4 ? 4 : 2))) void attention_prefill_kernel(
    const float *__restrict__ q_heads, const float *__restrict__ kcache, const float *__restrict__ vcache,
    float *__restrict__ out, int T, int S, int q_offset, int kv_rep, int num_kv_heads, int cap, float qscale,
    int pass_width, PrefillSplit sp, PrefillOut ol) {
    using Shape = PrefillShape<kDT, kWaves, kTiles, kX6>;
    constexpr int D = Shape::kD, kLd = Shape::kLd, kQ = Shape::kQ;
    static_assert(!kX6 || kDT % 2 == 0, "the bf16x6 path needs head_dim 32 or 64");
    extern __shared__ __attribute__((aligned(16))) float lds[];
    uint16_t *const lds16 = reinterpret_cast<uint16_t *>(lds);

    const int slices = (kv_rep + kWaves - 1) / kWaves; // workgroups per GQA group
    const int per_tile = num_kv_heads * slices;
    const int ntq = (T + kAttnQTile - 1) / kAttnQTile;
    const int ngroups = (ntq + kTiles - 1) / kTiles; // query-tile groups
    const int rank = static_cast<int>(blockIdx.x) / per_tile;
    int grp, kt_begin = 0, kt_end = -1, half = -1, slot = 0; // kt_end < 0: the group's whole range
    if constexpr (kSplit) {
        const PrefillGeom geo{kTiles, ntq, S, q_offset};
        int pos = rank;
        if (sp.alternate) {
            const int nunits = ngroups + (ngroups - geo.first_split(ngroups, sp.thr));
            pos = nunits - 1 - prefill_tile_of_rank(rank, nunits, pass_width);
        }
        const PrefillUnit u = prefill_unit_of_rank(pos, ngroups, sp.thr, geo);
        grp = u.g;
        half = u.half;
        kt_begin = u.kt_begin;
        kt_end = u.kt_end;
        slot = u.slot;
    } else {
        grp = prefill_tile_of_rank(rank, ngroups, pass_width);
    }
    const int kvh = (static_cast<int>(blockIdx.x) % per_tile) / slices;
    const int slice = static_cast<int>(blockIdx.x) % slices;
    const int wave = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    const int l16 = lane % 16, g = lane / 16;
    const int rep = slice * kWaves + wave % kWaves; // head within the group
    const bool head_ok = rep < kv_rep;              // idle waves still stage K/V and join barriers
    const int h = kvh * kv_rep + (head_ok ? rep : 0);
    const int qt_raw = grp * kTiles + wave / kWaves; // this wave's query tile
    const bool tile_ok = qt_raw < ntq;
    const int qt = tile_ok ? qt_raw : ntq - 1;
    const int q0 = qt * kAttnQTile;
    const int q = q0 + l16;                 // this lane's query row (column of every MFMA tile)
    const int qpos = q_offset + q;          // its absolute position
    const int lim = qpos < S - 1 ? qpos : S - 1; // last key it sees

    const float *kh = kcache + int64_t(kvh) * cap * D;
    const float *vh = vcache + int64_t(kvh) * cap * D;

    // Q^T operand: lane (l16, g) keeps Q[q][kQ*g + s] * scale * log2(e), s < kQ, so the
    // scores come out in the base-2 exponent domain. Rows past T read row T-1 and are not stored.
    // kX6: lane (l16, g) keeps the three parts of Q[q][32 c + 8 g + j], j < 8, as the B operand of
    // step c of the 16x16x32 products.
    float qreg[kX6 ? 1 : kQ];
    bf16x8v qx[kX6 ? kDT / 2 : 1][3];
    if constexpr (kX6) {
        const float *qrow = q_heads + (int64_t(h) * T + (q < T ? q : T - 1)) * D + 8 * g;
#pragma unroll
        for (int c = 0; c < kDT / 2; ++c) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(qrow + 32 * c);
            const f32x4 b = *reinterpret_cast<const f32x4 *>(qrow + 32 * c + 4);
            const float v[8] = {a[0] * qscale, a[1] * qscale, a[2] * qscale, a[3] * qscale,
                                b[0] * qscale, b[1] * qscale, b[2] * qscale, b[3] * qscale};
            split3x8(v, qx[c]);
        }
    } else {
        const float *qrow = q_heads + (int64_t(h) * T + (q < T ? q : T - 1)) * D + kQ * g;
#pragma unroll
        for (int c = 0; c < kQ / 4; ++c) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(qrow + 4 * c);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                qreg[4 * c + j] = v[j] * qscale;
        }
    }

    // KV tiles: this wave's own, and the workgroup's (those of its last query tile).
    const int kv_end = (q_offset + q0 + kAttnQTile) < S ? (q_offset + q0 + kAttnQTile) : S;
    const int my_ntiles = tile_ok ? (kv_end + kAttnKTile - 1) / kAttnKTile : 0;
    const int q0_last = (grp * kTiles + kTiles - 1 < ntq ? grp * kTiles + kTiles - 1 : ntq - 1) * kAttnQTile;
    const int kv_end_last = (q_offset + q0_last + kAttnQTile) < S ? (q_offset + q0_last + kAttnQTile) : S;
    const int ntiles = kt_end >= 0 ? kt_end : (kv_end_last + kAttnKTile - 1) / kAttnKTile;

    // K/V tile staging through registers: chunk c = tid + i * threads is row c / (D/4).
    // Loads are unconditional (rows past S read row S-1 and are zeroed when staged, chunks
    // past the tile read its last row and are not staged): a load under a branch makes the
    // compiler wait for every load in flight before the next one.
    constexpr int kChunksPerRow = D / 4;
    constexpr int kStage = 2 * kAttnKTile * kLd; // floats of one K+V stage
    f32x4 kst[Shape::kPerThread], vst[Shape::kPerThread];
    auto chunk_row = [&](int i) {
        const int r = (threadIdx.x + i * Shape::kThreads) / kChunksPerRow;
        return r < kAttnKTile ? r : kAttnKTile - 1;
    };
    auto fetch = [&](int kt) {
#pragma unroll
        for (int i = 0; i < Shape::kPerThread; ++i) {
            const int key = kt * kAttnKTile + chunk_row(i);
            const int64_t row = int64_t(key < S ? key : S - 1) * D;
            const int d = ((threadIdx.x + i * Shape::kThreads) % kChunksPerRow) * 4;
            kst[i] = *reinterpret_cast<const f32x4 *>(kh + row + d);
            vst[i] = *reinterpret_cast<const f32x4 *>(vh + row + d);
        }
    };
    auto commit = [&](int buf, int kt) {
#pragma unroll
        for (int i = 0; i < Shape::kPerThread; ++i) {
            const int c = threadIdx.x + i * Shape::kThreads;
            const bool live = kt * kAttnKTile + chunk_row(i) < S;
            f32x4 kv, vv;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                kv[j] = live ? kst[i][j] : 0.f;
                vv[j] = live ? vst[i][j] : 0.f;
            }
            if (Shape::kChunks % Shape::kThreads == 0 || c < Shape::kChunks) {
                const int row = c / kChunksPerRow, d = (c % kChunksPerRow) * 4;
                if constexpr (kX6) {
                    // K parts row-major; V parts transposed, keys at their x6_key_slot
                    uint16_t *Kx = lds16 + buf * Shape::kStageX6;
                    uint16_t *Vx = Kx + 3 * kAttnKTile * Shape::kRowK;
                    uint32_t kw[2][3], vw[2][3]; // [value pair][part]
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        split3x2(kv[2 * j], kv[2 * j + 1], kw[j][0], kw[j][1], kw[j][2]);
                    const int kofs = row * Shape::kRowK + 8 * x6_k_chunk<D>(d / 8, row) + d % 8;
#pragma unroll
                    for (int pp = 0; pp < 3; ++pp)
                        *reinterpret_cast<uint2 *>(Kx + pp * kAttnKTile * Shape::kRowK + kofs) =
                            make_uint2(kw[0][pp], kw[1][pp]);
                    if constexpr (kChunksPerRow == 16) {
                        // Lanes l16 + 16 q of a wave hold keys 4 w + q, dims 4 l16 .. + 3. A 4 x 4
                        // transpose over (q, element) (permlane32_swap exchanges bit 1 of q with bit 1
                        // of the element, permlane16_swap bit 0 with bit 0) leaves lane (l16, q) with
                        // keys 4 w .. 4 w + 3 of dim 4 l16 + q: four adjacent V^T slots, one 8-byte
                        // write per part.
                        uint32_t e[4] = {__float_as_uint(vv[0]), __float_as_uint(vv[1]), __float_as_uint(vv[2]),
                                         __float_as_uint(vv[3])};
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            const auto sw = __builtin_amdgcn_permlane32_swap(e[j], e[2 + j], false, false);
                            e[j] = sw[0];
                            e[2 + j] = sw[1];
                        }
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            const auto sw = __builtin_amdgcn_permlane16_swap(e[2 * j], e[2 * j + 1], false, false);
                            e[2 * j] = sw[0];
                            e[2 * j + 1] = sw[1];
                        }
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            split3x2(__uint_as_float(e[2 * j]), __uint_as_float(e[2 * j + 1]), vw[j][0], vw[j][1],
                                     vw[j][2]);
                        const int lane_q = (threadIdx.x % kWaveSize) / 16;
                        const int key0 = row - lane_q, vd = d + lane_q; // keys key0 .. key0 + 3 of dim vd
                        const int slot = x6_key_slot(key0);
                        const int vofs = vd * Shape::kRowV + 8 * x6_v_chunk(slot / 8, vd) + slot % 8;
#pragma unroll
                        for (int pp = 0; pp < 3; ++pp)
                            *reinterpret_cast<uint2 *>(Vx + pp * D * Shape::kRowV + vofs) =
                                make_uint2(vw[0][pp], vw[1][pp]);
                    } else {
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            split3x2(vv[2 * j], vv[2 * j + 1], vw[j][0], vw[j][1], vw[j][2]);
                        const int slot = x6_key_slot(row);
                        auto vpos = [&](int dd) { return dd * Shape::kRowV + 8 * x6_v_chunk(slot / 8, dd) + slot % 8; };
#pragma unroll
                        for (int pp = 0; pp < 3; ++pp)
#pragma unroll
                            for (int j = 0; j < 2; ++j) {
                                Vx[pp * D * Shape::kRowV + vpos(d + 2 * j)] = static_cast<uint16_t>(vw[j][pp]);
                                Vx[pp * D * Shape::kRowV + vpos(d + 2 * j + 1)] = static_cast<uint16_t>(vw[j][pp] >> 16);
                            }
                    }
                } else {
                    float *Ks = lds + buf * kStage;
                    float *Vs = Ks + kAttnKTile * kLd;
                    const int off = row * kLd + d;
                    *reinterpret_cast<f32x4 *>(Ks + off) = kv;
                    *reinterpret_cast<f32x4 *>(Vs + off) = vv;
                }
            }
        }
    };

    f32x4 oacc[kDT];
#pragma unroll
    for (int t = 0; t < kDT; ++t)
        oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = kNegInf, l_part = 0.f; // l_part: this lane's share of the row sum

    fetch(kt_begin);
    commit(0, kt_begin);
    __syncthreads();
    for (int kt = kt_begin; kt < ntiles; ++kt) {
        const int buf = (kt - kt_begin) & 1;
        fetch(kt + 1); // in flight during this tile's MFMAs (all zeros past the last tile)
        __builtin_amdgcn_sched_barrier(0); // keep the loads at the top
        const float *Ks = lds + buf * kStage;
        const float *Vs = Ks + kAttnKTile * kLd;
        const uint16_t *Kx = lds16 + buf * Shape::kStageX6;
        const uint16_t *Vx = Kx + 3 * kAttnKTile * Shape::kRowK;

        if (kt < my_ntiles) { // wave-uniform: the group's shorter tile skips its last K/V tile
            f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
            float vf[kX6 ? 1 : 2][4][kDT];
            if constexpr (kX6) {
                // S^T blocks on 16x16x32 products: lane (l16, g) supplies K[16u + l16][32c + 8g + j]
                // (A) and Q[q][32c + 8g + j] (B); sacc[u][r] is again key 16u + 4g + r.
#pragma unroll
                for (int c = 0; c < kDT / 2; ++c) {
                    bf16x8v kf[2][3];
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int pp = 0; pp < 3; ++pp)
                            kf[u][pp] = __builtin_bit_cast(
                                bf16x8v, *reinterpret_cast<const u32x4 *>(
                                             Kx + (pp * kAttnKTile + 16 * u + l16) * Shape::kRowK +
                                             8 * x6_k_chunk<D>(4 * c + g, 16 * u + l16)));
                    // the two blocks' chains alternate, so consecutive MFMAs are independent
#pragma unroll
                    for (int term = 0; term < 6; ++term)
#pragma unroll
                        for (int u = 0; u < 2; ++u)
                            sacc[u] = mfma_x6_term(term, kf[u], qx[c], sacc[u]);
                }
            } else {
                // Operands first: the K fragments of both 16-key blocks and the V^T operands of the
                // P V chain, so one LDS latency covers the tile.
                f32x4 kf[2][kQ / 4];
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int c = 0; c < kQ / 4; ++c)
                        kf[u][c] = *reinterpret_cast<const f32x4 *>(Ks + (16 * u + l16) * kLd + kQ * g + 4 * c);
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int t = 0; t < kDT; ++t)
                            vf[u][s][t] = Vs[(16 * u + 4 * g + s) * kLd + 16 * t + l16];

                // S^T[key][q] = sum_d K[key][d] Q[q][d] for the two 16-key blocks u; at step s lane
                // group g supplies reduction index kQ*g + s to both operands, and sacc[u][r] is key
                // 16u + 4g + r. The blocks' chains alternate so consecutive MFMAs are independent.
#pragma unroll
                for (int c = 0; c < kQ / 4; ++c)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int u = 0; u < 2; ++u)
                            sacc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[u][c][j], qreg[4 * c + j], sacc[u], 0,
                                                                           0, 0);
            }

            // Causal mask, only on tiles that reach past the tile's first query position (a
            // wave-uniform branch: the mask's VALU work sits on the wave's critical path).
            if (kt * kAttnKTile + kAttnKTile - 1 > q_offset + q0) {
                const int key0 = kt * kAttnKTile + 4 * g;
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        sacc[u][r] = key0 + 16 * u + r > lim ? kNegInf : sacc[u][r];
            }
            // Online softmax in base 2. Key 0 is in every row's first tile, so m_new is finite.
            float tmax = kNegInf;
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    tmax = fmaxf(tmax, sacc[u][r]);
            tmax = column_combine(tmax, wave::Max{});
            const float m_new = fmaxf(m_run, tmax);
            const float corr = __builtin_amdgcn_exp2f(m_run - m_new); // 0 on the first tile
            float psum = 0.f;
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float p = __builtin_amdgcn_exp2f(sacc[u][r] - m_new);
                    sacc[u][r] = p;
                    psum += p;
                }
            l_part = l_part * corr + psum;
            m_run = m_new;
#pragma unroll
            for (int t = 0; t < kDT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    oacc[t][r] *= corr;
            if constexpr (kX6) {
                // O^T[d][q] += V^T P^T over the tile's 32 keys in one 16x16x32 product per head-dim
                // tile: lane (l16, g) supplies slots 8g + j, i.e. keys 16 (j / 4) + 4g + j % 4, whose
                // probabilities are its own sacc[j / 4][j % 4].
                const float pv[8] = {sacc[0][0], sacc[0][1], sacc[0][2], sacc[0][3],
                                     sacc[1][0], sacc[1][1], sacc[1][2], sacc[1][3]};
                bf16x8v px[3];
                split3x8(pv, px);
#pragma unroll
                for (int t0 = 0; t0 < kDT; t0 += 2) {
                    bf16x8v vx[2][3];
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int pp = 0; pp < 3; ++pp)
                            vx[t][pp] = __builtin_bit_cast(
                                bf16x8v, *reinterpret_cast<const u32x4 *>(
                                             Vx + (pp * D + 16 * (t0 + t) + l16) * Shape::kRowV +
                                             8 * x6_v_chunk(g, 16 * (t0 + t) + l16)));
#pragma unroll
                    for (int term = 0; term < 6; ++term)
#pragma unroll
                        for (int t = 0; t < 2; ++t)
                            oacc[t0 + t] = mfma_x6_term(term, vx[t], px, oacc[t0 + t]);
                }
            } else {
                // O^T[d][q] += sum_key V[key][d] P^T[key][q]: at step s of block u lane group g
                // supplies key 16u + 4g + s, which is its own S^T register sacc[u][s].
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int t = 0; t < kDT; ++t)
                            oacc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[u][s][t], sacc[u][s], oacc[t], 0, 0, 0);
            }
        }
        // Stage the next tile into the other buffer (last read before the previous barrier);
        // the fence keeps the staging, which waits for the loads, at the end.
        __builtin_amdgcn_sched_barrier(0);
        commit(buf ^ 1, kt + 1);
        __syncthreads();
    }

    // oacc[t][r] = O^T[16t + 4g + r][q]: four consecutive head-dim values of row q.
    float l = column_combine(l_part, wave::Add{});
    if constexpr (kSplit) {
        if (half >= 0) {
            // Both halves write their (m, l, O) records with agent-coherent stores (through the
            // XCD's L2), wait for them, and count in; the second to arrive merges in the fixed
            // order half 0, half 1 and resets the counter. No workgroup waits on another.
            constexpr int kRec = 2 + 4 * kDT, kThr = Shape::kThreads;
            const int pair = slot * per_tile + static_cast<int>(blockIdx.x) % per_tile;
            float *mine = sp.rec + (int64_t(pair) * 2 + half) * kRec * kThr + threadIdx.x;
            const float *other = sp.rec + (int64_t(pair) * 2 + (1 - half)) * kRec * kThr + threadIdx.x;
            record_store<true>(mine, m_run);
            record_store<true>(mine + kThr, l);
#pragma unroll
            for (int t = 0; t < kDT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    record_store<true>(mine + (2 + 4 * t + r) * kThr, oacc[t][r]);
            __shared__ int last;
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0); // the record stores have completed
            __syncthreads();
            int *counter = sp.counters + int64_t(pair) * kAttnCounterStride;
            if (threadIdx.x == 0)
                last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1;
            __syncthreads();
            if (!last)
                return;
            const float m_o = record_load<true>(other), l_o = record_load<true>(other + kThr);
            f32x4 o_o[kDT];
#pragma unroll
            for (int t = 0; t < kDT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    o_o[t][r] = record_load<true>(other + (2 + 4 * t + r) * kThr);
            const float m0 = half == 0 ? m_run : m_o, m1 = half == 0 ? m_o : m_run;
            const float l0 = half == 0 ? l : l_o, l1 = half == 0 ? l_o : l;
            const float M = fmaxf(m0, m1);
            const float c0 = m0 == kNegInf ? 0.f : __builtin_amdgcn_exp2f(m0 - M);
            const float c1 = m1 == kNegInf ? 0.f : __builtin_amdgcn_exp2f(m1 - M);
            l = l0 * c0 + l1 * c1;
#pragma unroll
            for (int t = 0; t < kDT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float a0 = half == 0 ? oacc[t][r] : o_o[t][r], a1 = half == 0 ? o_o[t][r] : oacc[t][r];
                    oacc[t][r] = a0 * c0 + a1 * c1;
                }
            if (threadIdx.x == 0)
                __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (head_ok && tile_ok && q < T) {
        const int64_t orow = int64_t(h) * ol.head_stride + int64_t(q) * ol.row_stride;
#pragma unroll
        for (int t = 0; t < kDT; ++t) {
            f32x4 o;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                o[r] = oacc[t][r] * inv;
            if (ol.bf16) // uniform
                *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(out) + orow + 16 * t + 4 * g) =
                    uint2{uint32_t(float_to_bf16_rne(o[0])) | (uint32_t(float_to_bf16_rne(o[1])) << 16),
                          uint32_t(float_to_bf16_rne(o[2])) | (uint32_t(float_to_bf16_rne(o[3])) << 16)};
            else
                *reinterpret_cast<f32x4 *>(out + orow + 16 * t + 4 * g) = o;
        }
    }
}

// Caller memory of the workspace form: the split units' records and their arrival counters
// (zero before the first call; every call leaves them at zero). thr < 0 picks the split
// threshold automatically.
struct PrefillWorkspaceArgs {
    float *rec = nullptr;
    int64_t rec_floats = 0;
    int *counters = nullptr;
    int64_t counter_ints = 0;
    int thr = -1;
    bool merged_heads = false; // output [T][qh * D] instead of [qh][T][D]
    bool out_bf16 = false;     // output rounded to bf16 (nearest-even)
};

// Workspace form on the host: the threshold, how many groups split, and what that needs.
struct PrefillSplitPlan {
    int thr = 0, nsplit = 0;
    int alternate = 0; // units in alternating passes (one-tile grids) or in descending order
    int64_t rec_floats = 0, counter_ints = 0;
};

// Automatic threshold, from sweeps of thresholds and orders at 32 q / 8 kv heads, D = 64:
//  * one-tile grids (at most 3 workgroups per CU): every group past 2 K/V tiles splits and the
//    units go out in alternating passes, so a CU holds heavy and light halves (bf16x6 products:
//    T = 512 24.3 -> 18.0 us, T = 1024 44.2 -> 41.4 us);
//  * two-tile grids do not split. In one round (T = 2048, config 4: 512 workgroups, two per CU)
//    the alternating passes already pair each heavy group with a light one on its CU, and every
//    split form measured slower (fp32 products: 155 against 162-175 us). Over several rounds the
//    split paid with fp32 products (T = 4096 603 -> 570 us) but not with bf16x6 ones (T = 4096
//    381 against 387 us, T = 8192 1416 against 1431).
// The threshold then rises until the records and counters fit the caller's memory.
template <int kDT, int kWaves, int kTiles>
inline PrefillSplitPlan prefill_split_plan(int T, int S, int q_offset, int kv_rep, int kvh, int thr_req,
                                           int64_t rec_cap, int64_t counter_cap) {
    using Shape = PrefillShape<kDT, kWaves, kTiles>;
    const int per_tile = kvh * ((kv_rep + kWaves - 1) / kWaves);
    const int ntq = static_cast<int>(blocks_for64(T, kAttnQTile));
    const int ngroups = (ntq + kTiles - 1) / kTiles;
    const PrefillGeom geo{kTiles, ntq, S, q_offset};
    PrefillSplitPlan p;
    p.alternate = kTiles == 1;
    if (thr_req >= 0) {
        p.thr = thr_req;
    } else {
        p.thr = kTiles == 2 ? INT32_MAX : 2;
    }
    const int64_t rec_per_group = int64_t(per_tile) * 2 * (2 + 4 * kDT) * Shape::kThreads;
    const int64_t ctr_per_group = int64_t(per_tile) * kAttnCounterStride;
    for (;;) {
        const int gs = geo.first_split(ngroups, p.thr);
        p.nsplit = ngroups - gs;
        p.rec_floats = p.nsplit * rec_per_group;
        p.counter_ints = p.nsplit * ctr_per_group;
        if (p.nsplit == 0 || (p.rec_floats <= rec_cap && p.counter_ints <= counter_cap))
            return p;
        p.thr = geo.tiles(gs); // that group no longer splits
    }
}

template <int kDT, int kWaves, int kTiles, bool kX6>
inline void attention_prefill_launch(const float *q, const float *k, const float *v, float *out, int T, int S,
                                     int q_offset, int kv_rep, int kvh, int cap, float scale, hipStream_t stream,
                                     const PrefillWorkspaceArgs *ws) {
    using Shape = PrefillShape<kDT, kWaves, kTiles, kX6>;
    const int slices = (kv_rep + kWaves - 1) / kWaves;
    const int per_tile = kvh * slices;
    const int64_t ngroups = blocks_for64(blocks_for64(T, kAttnQTile), kTiles);
    require(ngroups * per_tile <= INT32_MAX, "attention_prefill: grid too large");
    const int pass_width = cu_count() / per_tile > 0 ? cu_count() / per_tile : 1;
    const int D = 16 * kDT, qh = kvh * kv_rep;
    const PrefillOut ol = ws && ws->merged_heads ? PrefillOut{D, int64_t(qh) * D, ws->out_bf16 ? 1 : 0}
                                                 : PrefillOut{int64_t(T) * D, D, ws && ws->out_bf16 ? 1 : 0};
    if (ws) {
        const PrefillSplitPlan p = prefill_split_plan<kDT, kWaves, kTiles>(T, S, q_offset, kv_rep, kvh, ws->thr,
                                                                           ws->rec_floats, ws->counter_ints);
        if (p.nsplit > 0) {
            require((ngroups + p.nsplit) * per_tile <= INT32_MAX, "attention_prefill: grid too large");
            launch_async_lds(stream, Shape::kLdsBytes, attention_prefill_kernel<kDT, kWaves, kTiles, true, kX6>,
                             static_cast<int>((ngroups + p.nsplit) * per_tile), Shape::kThreads, q, k, v, out, T, S,
                             q_offset, kv_rep, kvh, cap, scale * kLog2e, pass_width,
                             PrefillSplit{ws->rec, ws->counters, p.thr, p.alternate}, ol);
            return;
        }
    }
    launch_async_lds(stream, Shape::kLdsBytes, attention_prefill_kernel<kDT, kWaves, kTiles, false, kX6>,
                     static_cast<int>(ngroups * per_tile), Shape::kThreads, q, k, v, out, T, S, q_offset, kv_rep, kvh,
                     cap, scale * kLog2e, pass_width, PrefillSplit{nullptr, nullptr, 0, 0}, ol);
}

// Two query tiles per workgroup when the one-tile grid would fill every CU's four
// workgroup slots (measured on near-uniform work: 76 -> 79.5% of the MFMA peak); one
// otherwise, so short prompts still spread over all CUs.
template <int kDT, int kWaves> inline bool prefill_two_tiles(int T, int kv_rep, int kvh) {
    const int64_t wgs = blocks_for64(T, kAttnQTile) * kvh * ((kv_rep + kWaves - 1) / kWaves);
    return wgs >= 4 * int64_t(cu_count());
}

template <int kDT, int kWaves>
inline void attention_prefill_tiles(const float *q, const float *k, const float *v, float *out, int T, int S,
                                    int q_offset, int kv_rep, int kvh, int cap, float scale, hipStream_t stream,
                                    const PrefillWorkspaceArgs *ws) {
    // head_dim 32 or 64 takes the bf16x6 products (config 4 154 -> 109 us; T = 512 20.8 -> 18.0
    // us and T = 4096 569 -> 377 us in the workspace form); 16 and 48 keep fp32 MFMAs.
    constexpr bool kX6 = kDT % 2 == 0;
    if (prefill_two_tiles<kDT, kWaves>(T, kv_rep, kvh))
        attention_prefill_launch<kDT, kWaves, 2, kX6>(q, k, v, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream, ws);
    else
        attention_prefill_launch<kDT, kWaves, 1, kX6>(q, k, v, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream, ws);
}

template <int kDT>
inline void attention_prefill_dispatch(const float *q, const float *k, const float *v, float *out, int T, int S,
                                       int q_offset, int kv_rep, int kvh, int cap, float scale, hipStream_t stream,
                                       const PrefillWorkspaceArgs *ws = nullptr) {
    if (kv_rep == 1)
        attention_prefill_tiles<kDT, 1>(q, k, v, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream, ws);
    else if (kv_rep == 2)
        attention_prefill_tiles<kDT, 2>(q, k, v, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream, ws);
    else if (kv_rep <= 4)
        attention_prefill_tiles<kDT, 4>(q, k, v, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream, ws);
    else
        attention_prefill_tiles<kDT, 8>(q, k, v, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream, ws);
}

// What the workspace form needs for this shape at threshold thr (< 0: automatic), unbounded.
template <int kDT>
inline PrefillSplitPlan prefill_split_need(int T, int S, int q_offset, int kv_rep, int kvh, int thr) {
    constexpr int64_t kNoCap = INT64_MAX;
    auto by_waves = [&](auto waves) {
        constexpr int kW = decltype(waves)::value;
        return prefill_two_tiles<kDT, kW>(T, kv_rep, kvh)
                   ? prefill_split_plan<kDT, kW, 2>(T, S, q_offset, kv_rep, kvh, thr, kNoCap, kNoCap)
                   : prefill_split_plan<kDT, kW, 1>(T, S, q_offset, kv_rep, kvh, thr, kNoCap, kNoCap);
    };
    if (kv_rep == 1)
        return by_waves(std::integral_constant<int, 1>{});
    if (kv_rep == 2)
        return by_waves(std::integral_constant<int, 2>{});
    if (kv_rep <= 4)
        return by_waves(std::integral_constant<int, 4>{});
    return by_waves(std::integral_constant<int, 8>{});
}

// ---------------------------------------------------------------- decode
constexpr int kAttnChunk = 64;       // keys per decode workgroup
constexpr int kAttnDecodeMaxLen = 8192;
constexpr int kAttnMaxChunks = kAttnDecodeMaxLen / kAttnChunk;

// Partial record per (q head, chunk): [0] max, [1] sum, [2..2+D) unnormalised output.
inline int attention_decode_workspace_floats(int num_q_heads, int max_len, int head_dim) {
    const int chunks = (max_len + kAttnChunk - 1) / kAttnChunk;
    return num_q_heads * chunks * (head_dim + 2);
}

// Split-KV decode ("flash-decoding"): one workgroup per (kv head, chunk of
// kAttnChunk keys) stages the chunk's K/V rows in LDS with 16-byte loads
// (all issued before the LDS stores); wave w handles q head kvh * kv_rep + w:
// lane = key for the scores (four partial dot products), then lane = head-dim
// element for P V. Each chunk leaves a record (max, sum, unnormalised
// output[D]); the combine kernel (one wave per q head) merges a head's
// records in chunk order: M = max m_c, L = sum l_c e^(m_c - M),
// out = sum acc_c e^(m_c - M) / L, loading 16 chunk rows per round trip.
// The length is a host value or, for graph replay, read on the device.
//
// Fused form (counters set): the partial kernel also merges. Records are
// written with agent-coherent stores (relaxed agent-scope atomics, which
// write through the XCD's L2), each workgroup waits for its stores to
// complete and then counts itself in on counters[kvh]; the workgroup that
// arrives last reads its kv head's records with agent-coherent loads, merges
// them as the combine kernel does, and resets the counter to zero for the next
// launch. No workgroup waits on another, and no cache-wide writeback or
// invalidate is needed. The counters (kv head k's at counters[k *
// kAttnCounterStride]) must be zero before the first launch.
struct DecodeAttnArgs {
    const float *q;               // [qh][D]
    const float *kcache, *vcache; // [kvh][cap][D]
    float *out;                   // [qh][D]
    float *partial;               // [qh][max_chunks][D + 2]
    const int *len_ptr;           // if set, length = *len_ptr + len_bias
    int *counters;                // [kvh * kAttnCounterStride], zero between launches; null: combine kernel
    int len, len_bias;
    int kv_rep, D, cap, max_chunks;
    int chunks_per_record;        // 1, or 2: a workgroup computes two adjacent chunks and leaves one record
    float scale;
};

// Records of a kv head: one per chunk, or per pair of chunks.
__device__ __forceinline__ int decode_records(const DecodeAttnArgs &a, int nchunks) {
    return (nchunks + a.chunks_per_record - 1) / a.chunks_per_record;
}


// One wave merges q head h's records in chunk order: M = max m_c,
// L = sum l_c e^(m_c - M), out = sum acc_c e^(m_c - M) / L, 16 chunk rows per
// round trip.
template <bool kCoherent>
__device__ __forceinline__ void decode_combine_head(const DecodeAttnArgs &a, int h, int nchunks, int lane) {
    const int D = a.D;
    const float *base = a.partial + int64_t(h) * a.max_chunks * (D + 2);
    float m0 = kNegInf, l0 = 0.f, m1 = kNegInf, l1 = 0.f;
    if (lane < nchunks) {
        m0 = record_load<kCoherent>(base + int64_t(lane) * (D + 2));
        l0 = record_load<kCoherent>(base + int64_t(lane) * (D + 2) + 1);
    }
    if (lane + kWaveSize < nchunks) {
        m1 = record_load<kCoherent>(base + int64_t(lane + kWaveSize) * (D + 2));
        l1 = record_load<kCoherent>(base + int64_t(lane + kWaveSize) * (D + 2) + 1);
    }
    // The first batch of output rows is loaded together with the (max, sum) pairs, so a
    // merge of up to kBatch chunks (1024 keys) costs one memory round trip (32 measured slower).
    // Rows 16..63 (up to three more batches, long contexts) are issued right behind it, so they
    // share that round trip instead of taking one each; past 64 rows, one batch per trip.
    constexpr int kBatch = 16, kAhead = 3;
    float v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
        v[j] = j < nchunks && lane < D ? record_load<kCoherent>(base + int64_t(j) * (D + 2) + 2 + lane) : 0.f;
    // Uniform branches on the record count, and row and lane indices clamped (the extra values
    // are multiplied by nothing), so no load sits under a per-lane condition.
    float u[kAhead][kBatch];
    const int dl = lane < D ? lane : D - 1;
#pragma unroll
    for (int b = 0; b < kAhead; ++b) {
        if (nchunks > kBatch * (b + 1)) {
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int c = kBatch * (b + 1) + j < nchunks ? kBatch * (b + 1) + j : nchunks - 1;
                u[b][j] = record_load<kCoherent>(base + int64_t(c) * (D + 2) + 2 + dl);
            }
        } else {
#pragma unroll
            for (int j = 0; j < kBatch; ++j)
                u[b][j] = 0.f;
        }
    }
    const float M = wave::max(fmaxf(m0, m1));
    const float w0 = lane < nchunks ? expf(m0 - M) : 0.f;
    const float w1 = lane + kWaveSize < nchunks ? expf(m1 - M) : 0.f;
    const float L = wave::sum(l0 * w0 + l1 * w1);
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
        const float wc = wave::readlane(w0, j);
        acc = j < nchunks ? fmaf(v[j], wc, acc) : acc;
    }
#pragma unroll
    for (int b = 0; b < kAhead; ++b)
        if (nchunks > kBatch * (b + 1)) {
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int c = kBatch * (b + 1) + j;
                const float wc = wave::readlane(w0, c);
                acc = c < nchunks ? fmaf(u[b][j], wc, acc) : acc;
            }
        }
    for (int c0 = kBatch * (kAhead + 1); c0 < nchunks; c0 += kBatch) {
        {
#pragma unroll
            for (int j = 0; j < kBatch; ++j)
                v[j] = c0 + j < nchunks && lane < D
                           ? record_load<kCoherent>(base + int64_t(c0 + j) * (D + 2) + 2 + lane)
                           : 0.f;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int c = c0 + j;
            const float wc = wave::readlane(c < kWaveSize ? w0 : w1, c % kWaveSize);
            acc = c < nchunks ? fmaf(v[j], wc, acc) : acc;
        }
    }
    if (lane < D)
        record_store<kCoherent>(a.out + int64_t(h) * D + lane, L > 0.f ? acc / L : 0.f);
}

__device__ __forceinline__ int decode_len(const DecodeAttnArgs &a) {
    int len = a.len_ptr ? *a.len_ptr + a.len_bias : a.len;
    len = len < a.cap ? len : a.cap;
    return len < a.max_chunks * kAttnChunk ? len : a.max_chunks * kAttnChunk;
}

// Fused form, after a chunk workgroup has issued its records: count in once they are
// complete; the last workgroup of the kv head merges the head group's records into the
// output, then resets the counter. Returns true in that workgroup (its merged outputs,
// written with agent-coherent stores, have completed).
__device__ __forceinline__ bool decode_count_in_and_merge(const DecodeAttnArgs &a, int kvh, int nchunks, int h,
                                                          bool head_ok, int lane) {
    __shared__ int last;
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0); // the record stores have completed
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(a.counters + kvh * kAttnCounterStride, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == nchunks - 1;
    __syncthreads();
    if (!last)
        return false;
    if (head_ok)
        decode_combine_head<true>(a, h, nchunks, lane);
    if (threadIdx.x == 0)
        __hip_atomic_store(a.counters + kvh * kAttnCounterStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0); // the merged outputs have completed
    __syncthreads();
    return true;
}

// A chunk's record (m, l, acc[D]) of q head h: agent-coherent stores in the fused form.
__device__ __forceinline__ float *decode_record(const DecodeAttnArgs &a, int h, int chunk) {
    return a.partial + (int64_t(h) * a.max_chunks + chunk) * (a.D + 2);
}

// Register-blocked (kv head, record) workgroup for kWaves <= 8 waves per chunk (kv_rep <= 8 q
// heads), computing kSub adjacent chunks (1, or 2 with two groups of kWaves waves) and leaving one
// record. In each group, thread t holds key slots i < kPer = 16 / kWaves: key t/16 + (kWaves * 4) * i,
// head-dim pack dq = t % 16 of it (the row padded to 16 packs; packs >= D/4 and keys past the
// length are zero), loaded straight from HBM into registers with the q packs of every head of the
// group, so K and V never pass through LDS and no wave re-reads the chunk:
//  * scores: the thread's kPer x kWaves partial dot products (always 16) are summed over the 16
//    lanes of its row by a DPP reduce-scatter (row_ror 8, row_half_mirror, quad_perm ^2, ^1: each
//    step keeps half the values and adds the partner lane's other half), after which lane dq of
//    the row holds value dq, i.e. head dq % kWaves of slot dq / kWaves;
//  * softmax: wave h of the group reads head h's 64 scores from LDS (lane = key);
//  * P V: each thread accumulates its slots' V packs for every head (kWaves packs of 4),
//    reduce-scatters them over the wave's four rows with v_permlane32_swap then
//    v_permlane16_swap, and the waves' partial outputs are summed through LDS.
// With kSub = 2 the two chunks' (m, l, acc) are then combined in the workgroup (M = max, each
// rescaled by e^(m - M)), so a kv head has half as many records to merge; a second chunk past
// the length contributes nothing. About 10 KB of LDS traffic per chunk, against the 128 KB of
// the one-head-per-wave form. The records and their merge are those of decode_attention_chunk.
template <int kWaves, int kSub>
__device__ __forceinline__ bool decode_attention_chunk_rb(const DecodeAttnArgs &a, int kvh, int rec) {
    static_assert(kWaves >= 1 && kWaves <= 8 && (kWaves & (kWaves - 1)) == 0, "1, 2, 4 or 8 waves");
    static_assert(kSub == 1 || kSub == 2, "one or two chunks per record");
    constexpr int C = kAttnChunk;
    constexpr int TH = kWaves * kWaveSize;    // threads per chunk
    constexpr int kRowStep = TH / 16;         // keys between a thread's slots
    constexpr int kPer = 16 / kWaves;         // key slots per thread
    constexpr int kOut = 4 * kWaves;          // P V values per thread: kWaves heads x 4 dims
    constexpr int kOStride = kOut + 4;        // floats per dq column of a wave's partial outputs (kOut used)
    static_assert(kPer * kWaves == 16, "16 partial scores per thread");
    const int len = decode_len(a);
    const int nchunks = (len + C - 1) / C;
    const int nrec = (nchunks + kSub - 1) / kSub;
    if (rec >= nrec)
        return false;
    const int sub = threadIdx.x / TH, t = threadIdx.x % TH; // chunk of this thread's group, thread in it
    const int k0 = (rec * kSub + sub) * C;
    const int n = len - k0 < 0 ? 0 : (len - k0 < C ? len - k0 : C); // 0: a second chunk past the length
    const int D = a.D, P = D / 4, rep = a.kv_rep;
    const int wave = t / kWaveSize, lane = t % kWaveSize;
    const int dq = t % 16, row = t / 16, row4 = lane / 16;
    const bool dq_ok = dq < P;
    const f32x4 *kh = reinterpret_cast<const f32x4 *>(a.kcache + (int64_t(kvh) * a.cap + k0) * D);
    const f32x4 *vh = reinterpret_cast<const f32x4 *>(a.vcache + (int64_t(kvh) * a.cap + k0) * D);
    const f32x4 *q4 = reinterpret_cast<const f32x4 *>(a.q + int64_t(kvh) * rep * D);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    // q, then K, then V: the scores wait for q and K only, and V keeps arriving through the
    // scores and the softmax (their barriers order LDS only). Every load is issued, from a valid
    // clamped address (the cache row len - 1, the last pack of a row, head 0 of the group), and
    // what lies outside is zeroed afterwards: a load under a per-lane branch would make the
    // compiler wait for all of them before the first score.
    f32x4 kv[kPer], vv[kPer], qv[kWaves];
    const int dqc = dq_ok ? dq : P - 1;
#pragma unroll
    for (int h = 0; h < kWaves; ++h) {
        const f32x4 x = q4[(h < rep ? h : 0) * P + dqc];
        qv[h] = dq_ok && h < rep ? x : zero;
    }
    auto clamped = [&](int key) { return (k0 + key < len ? key : len - 1 - k0) * P + dqc; };
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int key = row + kRowStep * i;
        const f32x4 x = kh[clamped(key)];
        kv[i] = dq_ok && key < n ? x : zero;
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int key = row + kRowStep * i;
        const f32x4 x = vh[clamped(key)];
        vv[i] = dq_ok && key < n ? x : zero;
    }
    __builtin_amdgcn_sched_barrier(0);
    __shared__ float Ss[kSub][kWaves][C];                        // scaled scores, [head][key]
    __shared__ __attribute__((aligned(16))) float Ps[kSub][C][kWaves]; // probabilities, [key][head]
    __shared__ __attribute__((aligned(16))) float Os[kSub][kWaves][16 * kOStride]; // per-wave P V partials
    // scores: 16 partial dot products, then the row reduce-scatter
    float v[16];
#pragma unroll
    for (int i = 0; i < kPer; ++i)
#pragma unroll
        for (int h = 0; h < kWaves; ++h) {
            const f32x4 x = kv[i] * qv[h];
            v[i * kWaves + h] = (x[0] + x[1]) + (x[2] + x[3]);
        }
    {
        const bool b3 = dq & 8, b2 = dq & 4, b1 = dq & 2, b0 = dq & 1;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float keep = b3 ? v[k + 8] : v[k], send = b3 ? v[k] : v[k + 8];
            v[k] = keep + wave::dpp<0x128>(send, send); // row_ror:8, lane ^ 8
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float keep = b2 ? v[k + 4] : v[k], send = b2 ? v[k] : v[k + 4];
            v[k] = keep + wave::dpp<wave::kRowHalfMirror>(send, send); // lane 7 - p in each half row
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float keep = b1 ? v[k + 2] : v[k], send = b1 ? v[k] : v[k + 2];
            v[k] = keep + wave::dpp<wave::kQuadSwap2>(send, send);
        }
        const float keep = b0 ? v[1] : v[0], send = b0 ? v[0] : v[1];
        v[0] = keep + wave::dpp<wave::kQuadSwap1>(send, send);
    }
    {
        const int h = dq % kWaves, key = row + kRowStep * (dq / kWaves);
        if (h < rep)
            Ss[sub][h][key] = key < n ? v[0] * a.scale : kNegInf;
    }
    lds_barrier();
    // softmax of head `wave` over the chunk's keys (lane = key); an empty chunk leaves m = -inf
    const bool head_ok = wave < rep;
    const int h = kvh * rep + (head_ok ? wave : 0);
    float m = kNegInf, l = 0.f;
    if (head_ok) {
        float pr = 0.f;
        if (n > 0) {
            const float sc = Ss[sub][wave][lane];
            m = wave::max(sc);
            pr = lane < n ? expf(sc - m) : 0.f;
            l = wave::sum(pr);
        }
        Ps[sub][lane][wave] = pr;
    }
    lds_barrier();
    // P V: this thread's slots for every head of the group
    float o[kOut];
#pragma unroll
    for (int k = 0; k < kOut; ++k)
        o[k] = 0.f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int key = row + kRowStep * i;
#pragma unroll
        for (int hh = 0; hh < kWaves; ++hh) {
            const float pr = Ps[sub][key][hh];
#pragma unroll
            for (int c = 0; c < 4; ++c)
                o[4 * hh + c] = fmaf(pr, vv[i][c], o[4 * hh + c]);
        }
    }
    // reduce-scatter over the wave's four rows: rows 0-1 keep values [0, 2kW), rows 2-3 the
    // rest (permlane32_swap), then even rows the first kW of their half (permlane16_swap);
    // row r4 ends with values [r4 * kW, (r4 + 1) * kW), each summed over the four rows
#pragma unroll
    for (int k = 0; k < 2 * kWaves; ++k) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(o[k]), __float_as_uint(o[k + 2 * kWaves]),
                                                         false, false);
        o[k] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
        const auto sw =
            __builtin_amdgcn_permlane16_swap(__float_as_uint(o[k]), __float_as_uint(o[k + kWaves]), false, false);
        o[k] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
#pragma unroll
    for (int k = 0; k < kWaves; ++k)
        Os[sub][wave][dq * kOStride + row4 * kWaves + k] = o[k];
    __syncthreads();
    // wave = head, lane = head-dim element d: value 4 * head + d % 4 of column d / 4
    float acc = 0.f;
    if (head_ok && lane < D) {
        const int j = 4 * wave + lane % 4, col = lane / 4;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
            acc += Os[sub][w][col * kOStride + j];
    }
    if constexpr (kSub == 2) { // combine the two chunks into the record of group 0
        __shared__ float Ah[kWaves][kAttnMaxD], Mh[kWaves], Lh[kWaves];
        if (sub == 1 && head_ok) {
            if (lane < D)
                Ah[wave][lane] = acc;
            if (lane == 0) {
                Mh[wave] = m;
                Lh[wave] = l;
            }
        }
        __syncthreads();
        if (sub == 0 && head_ok) {
            const float m1 = Mh[wave], M = fmaxf(m, m1);
            const float a0 = expf(m - M), a1 = m1 == kNegInf ? 0.f : expf(m1 - M);
            l = l * a0 + Lh[wave] * a1;
            if (lane < D)
                acc = acc * a0 + Ah[wave][lane] * a1;
            m = M;
        }
    }
    const bool writer = sub == 0 && head_ok;
    if (writer && lane < D) {
        float *r = a.partial + (int64_t(h) * a.max_chunks + rec) * (D + 2);
        if (a.counters) {
            if (lane == 0) {
                record_store<true>(r, m);
                record_store<true>(r + 1, l);
            }
            record_store<true>(r + 2 + lane, acc);
        } else {
            if (lane == 0) {
                r[0] = m;
                r[1] = l;
            }
            r[2 + lane] = acc;
        }
    }
    return a.counters && decode_count_in_and_merge(a, kvh, nrec, h, writer, lane);
}

// One (kv head, chunk) workgroup of the decode attention with one wave per q head, for
// groups of more than 8 q heads. Returns true in the workgroup that merged its kv head's
// records (fused form only; the merged outputs were written with agent-coherent stores and
// have completed).
template <int kWaves>
__device__ __forceinline__ bool decode_attention_chunk(const DecodeAttnArgs &a, int kvh, int chunk) {
    constexpr int C = kAttnChunk;
    const int len = decode_len(a);
    const int nchunks = (len + C - 1) / C;
    if (chunk >= nchunks)
        return false;
    const int k0 = chunk * C;
    const int n = len - k0 < C ? len - k0 : C;
    const int D = a.D;
    __shared__ __attribute__((aligned(16))) float Ks[C][kAttnMaxD + 4];
    __shared__ __attribute__((aligned(16))) float Vs[C][kAttnMaxD];
    __shared__ __attribute__((aligned(16))) float Qs[kWaves][kAttnMaxD];
    __shared__ __attribute__((aligned(16))) float Ps[kWaves][C];
    const float *kh = a.kcache + (int64_t(kvh) * a.cap + k0) * D;
    const float *vh = a.vcache + (int64_t(kvh) * a.cap + k0) * D;
    const int wave = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    const bool head_ok = wave < a.kv_rep;
    const int h = kvh * a.kv_rep + (head_ok ? wave : 0);
    {
        constexpr int kMaxPer = C * kAttnMaxD / 4 / (kWaves * kWaveSize);
        constexpr int nthreads = kWaves * kWaveSize;
        const int packs = C * D / 4;
        f32x4 kv[kMaxPer], vv[kMaxPer];
#pragma unroll
        for (int i = 0; i < kMaxPer; ++i) {
            const int c = threadIdx.x + i * nthreads;
            const int r = (4 * c) / D;
            kv[i] = vv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (c < packs && r < n) {
                kv[i] = reinterpret_cast<const f32x4 *>(kh)[c];
                vv[i] = reinterpret_cast<const f32x4 *>(vh)[c];
            }
        }
#pragma unroll
        for (int i = 0; i < kMaxPer; ++i) {
            const int c = threadIdx.x + i * nthreads;
            if (c < packs) {
                const int r = (4 * c) / D, d = (4 * c) % D;
                *reinterpret_cast<f32x4 *>(&Ks[r][d]) = kv[i];
                *reinterpret_cast<f32x4 *>(&Vs[r][d]) = vv[i];
            }
        }
    }
    if (lane < D)
        Qs[wave][lane] = a.q[int64_t(h) * D + lane];
    __syncthreads();
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    for (int d = 0; d < D; d += 4) {
        const f32x4 kq = *reinterpret_cast<const f32x4 *>(&Ks[lane][d]);
        const f32x4 qv = *reinterpret_cast<const f32x4 *>(&Qs[wave][d]);
        s0 = fmaf(qv[0], kq[0], s0);
        s1 = fmaf(qv[1], kq[1], s1);
        s2 = fmaf(qv[2], kq[2], s2);
        s3 = fmaf(qv[3], kq[3], s3);
    }
    const float s = lane < n ? ((s0 + s1) + (s2 + s3)) * a.scale : kNegInf;
    const float m = wave::max(s);
    const float p = lane < n ? expf(s - m) : 0.f;
    const float l = wave::sum(p);
    Ps[wave][lane] = p;
    __builtin_amdgcn_wave_barrier();
    // lane = head-dim element; keys past n have p = 0 and zero V rows
    if (lane < D) {
        float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll 4
        for (int key = 0; key < C; key += 4) {
            const f32x4 pv = *reinterpret_cast<const f32x4 *>(&Ps[wave][key]);
            o0 = fmaf(pv[0], Vs[key][lane], o0);
            o1 = fmaf(pv[1], Vs[key + 1][lane], o1);
            o2 = fmaf(pv[2], Vs[key + 2][lane], o2);
            o3 = fmaf(pv[3], Vs[key + 3][lane], o3);
        }
        if (head_ok) {
            float *rec = a.partial + (int64_t(h) * a.max_chunks + chunk) * (D + 2);
            const float o = (o0 + o1) + (o2 + o3);
            if (a.counters) {
                if (lane == 0) {
                    record_store<true>(rec, m);
                    record_store<true>(rec + 1, l);
                }
                record_store<true>(rec + 2 + lane, o);
            } else {
                if (lane == 0) {
                    rec[0] = m;
                    rec[1] = l;
                }
                rec[2 + lane] = o;
            }
        }
    }
    return a.counters && decode_count_in_and_merge(a, kvh, nchunks, h, head_ok, lane);
}

template <int kWaves, int kSub>
__global__ __launch_bounds__(kSub *kWaves *kWaveSize) void attention_decode_partial_kernel(DecodeAttnArgs a) {
    if constexpr (kWaves <= 8)
        decode_attention_chunk_rb<kWaves, kSub>(a, blockIdx.x, blockIdx.y);
    else
        decode_attention_chunk<kWaves>(a, blockIdx.x, blockIdx.y);
}

// grid kvh, block kv_rep waves; wave w merges q head kvh * kv_rep + w. Workgroup k runs on the
// same XCD as the chunk workgroups of kv head k (blockIdx.x of the partial grid) under the
// round-robin dispatch, so their records are still in its L2: one wave per q head over 32
// workgroups measured slower (2048 keys: 8.34 against 7.90 us per call).
__global__ __launch_bounds__(kAttnMaxRep *kWaveSize) static void attention_decode_combine_kernel(DecodeAttnArgs a) {
    const int len = decode_len(a);
    const int nrec = decode_records(a, (len + kAttnChunk - 1) / kAttnChunk); // <= max_chunks <= 2 * kWaveSize
    const int wave = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    decode_combine_head<false>(a, blockIdx.x * a.kv_rep + wave, nrec, lane);
}

// ---- decode, scratch-free form (the reference signature) -----------------------------------
// ops::attention_decode keeps the reference's contract (include/ops/attention_decode.cuh:98-109):
// no workspace and no allocation, any head_dim <= 64, q and caches at any 4-byte alignment, any
// kv_rep, and num_q_heads need not be a multiple of kv_rep (q head h reads kv head h / kv_rep).
// With no scratch there is nowhere to leave split-KV records, so one workgroup owns a q head, as
// in the reference's grid. Its kSingleWaves waves take kSingleKeys-key chunks round robin, each
// wave with its own online-softmax state (m, l, unnormalised acc), and the wave states are merged
// in wave order at the end. A chunk is a contiguous run of n * D floats of the cache: K and V are
// read together with coalesced 4-byte buffer loads (one memory round trip per chunk; lanes past
// the chunk read zeros from the descriptor's range check) and staged in the wave's own LDS rows
// of kAttnMaxD + 1 floats, an odd stride, so the lane = key reads of the score loop hit distinct
// banks. Scores are the d-ascending fmaf chain of the reference's dot product; P V (lane = d) is
// key-ascending within a chunk.
// Workgroup b serves q head (b % 8) * (qh / 8) + b / 8 when 8 divides qh: under the round-robin
// dispatch of workgroups to the 8 XCDs, consecutive q heads, which share a kv head, then run on
// one XCD and read their K/V through the same L2.
constexpr int kSingleWaves = 8;
constexpr int kSingleKeys = 32;
constexpr int kSingleStride = kAttnMaxD + 1;
constexpr int kSinglePer = kSingleKeys * kAttnMaxD / kWaveSize; // chunk floats per lane at most

__global__ __launch_bounds__(kSingleWaves *kWaveSize) static void attention_decode_single_kernel(
    const float *__restrict__ q, const float *__restrict__ kcache, const float *__restrict__ vcache,
    float *__restrict__ out, int num_q_heads, int kv_rep, int D, int len, int max_seq, float scale) {
    __shared__ float Qs[kAttnMaxD];
    __shared__ float Ks[kSingleWaves][kSingleKeys * kSingleStride];
    __shared__ float Vs[kSingleWaves][kSingleKeys * kSingleStride];
    __shared__ float Ps[kSingleWaves][kSingleKeys];
    __shared__ float Wm[kSingleWaves], Wl[kSingleWaves];
    __shared__ float Wacc[kSingleWaves][kAttnMaxD];
    const int b = blockIdx.x;
    const int h = num_q_heads % 8 == 0 ? (b % 8) * (num_q_heads / 8) + b / 8 : b;
    const int wave = threadIdx.x / kWaveSize, lane = threadIdx.x % kWaveSize;
    const int64_t kv_base = int64_t(h / kv_rep) * max_seq * D;
    if (threadIdx.x < D)
        Qs[threadIdx.x] = q[int64_t(h) * D + threadIdx.x];
    __syncthreads();
    // element e = lane + 64 i of a chunk is key e / D, dimension e % D; stepped without division
    const int key0 = lane / D, d0 = lane % D, key_step = kWaveSize / D, d_step = kWaveSize % D;
    const int per = (kSingleKeys * D + kWaveSize - 1) / kWaveSize; // loads per lane per chunk
    float *ks = Ks[wave], *vs = Vs[wave];
    float m = kNegInf, l = 0.f, acc = 0.f;
    for (int c0 = wave * kSingleKeys; c0 < len; c0 += kSingleWaves * kSingleKeys) {
        const int n = len - c0 < kSingleKeys ? len - c0 : kSingleKeys;
        const int64_t off = kv_base + int64_t(c0) * D;
        const __amdgpu_buffer_rsrc_t ksrc = operand_rsrc(kcache + off, int64_t(n) * D * 4);
        const __amdgpu_buffer_rsrc_t vsrc = operand_rsrc(vcache + off, int64_t(n) * D * 4);
        float kr[kSinglePer], vr[kSinglePer];
#pragma unroll
        for (int i = 0; i < kSinglePer; ++i) {
            if (i < per) {
                kr[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ksrc, 4 * lane, 4 * kWaveSize * i, 0));
                vr[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vsrc, 4 * lane, 4 * kWaveSize * i, 0));
            }
        }
        {
            int key = key0, d = d0;
#pragma unroll
            for (int i = 0; i < kSinglePer; ++i) {
                if (i < per && key < n) {
                    ks[key * kSingleStride + d] = kr[i];
                    vs[key * kSingleStride + d] = vr[i];
                }
                key += key_step;
                d += d_step;
                if (d >= D) {
                    d -= D;
                    ++key;
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float s = 0.f;
        if (lane < n)
            for (int d = 0; d < D; ++d)
                s = fmaf(Qs[d], ks[lane * kSingleStride + d], s);
        const float sc = lane < n ? s * scale : kNegInf;
        const float mn = fmaxf(m, wave::max(sc)); // finite: the chunk has at least one key
        const float corr = m == kNegInf ? 0.f : expf(m - mn);
        const float p = lane < n ? expf(sc - mn) : 0.f;
        l = l * corr + wave::sum(p);
        m = mn;
        if (lane < kSingleKeys)
            Ps[wave][lane] = p;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < D) {
            float o = acc * corr;
            for (int k = 0; k < n; ++k)
                o = fmaf(Ps[wave][k], vs[k * kSingleStride + lane], o);
            acc = o;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (lane < D)
        Wacc[wave][lane] = acc;
    if (lane == 0) {
        Wm[wave] = m;
        Wl[wave] = l;
    }
    __syncthreads();
    if (wave != 0 || lane >= D)
        return;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kSingleWaves; ++w)
        M = fmaxf(M, Wm[w]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kSingleWaves; ++w) {
        const float f = Wm[w] == kNegInf ? 0.f : expf(Wm[w] - M); // a wave past the length holds nothing
        L = fmaf(Wl[w], f, L);
        o = fmaf(Wacc[w][lane], f, o);
    }
    out[int64_t(h) * D + lane] = o / L;
}

// Enqueues the partial and combine kernels (or the fused partial kernel alone
// when a.counters is set): grid (kvh, max_chunks) with kv_rep rounded up to a
// power of two waves per workgroup.
// Chunks per record: two when a kv head would otherwise have more than 16 records, so the merge
// reads at most 16 per head in one batch (2048 keys: 7.3 -> 6.x us per fused call); the load
// phase of 128 workgroups x 64 KB measured 3.0 against 2.7 us for 256 x 32 KB. Groups of more
// than 8 q heads keep one chunk per workgroup (their one-wave-per-head form).
inline int decode_chunks_per_record(int kv_rep, int max_chunks) { return kv_rep <= 8 && max_chunks > 16 ? 2 : 1; }

template <int kSub> inline void attention_decode_launch_sub(const DecodeAttnArgs &a, int kvh, hipStream_t stream) {
    const dim3 grid(kvh, (a.max_chunks + kSub - 1) / kSub);
    const int rep = a.kv_rep;
    if (rep <= 1)
        launch_async(stream, attention_decode_partial_kernel<1, kSub>, grid, kSub * kWaveSize, a);
    else if (rep <= 2)
        launch_async(stream, attention_decode_partial_kernel<2, kSub>, grid, kSub * 2 * kWaveSize, a);
    else if (rep <= 4)
        launch_async(stream, attention_decode_partial_kernel<4, kSub>, grid, kSub * 4 * kWaveSize, a);
    else if (rep <= 8)
        launch_async(stream, attention_decode_partial_kernel<8, kSub>, grid, kSub * 8 * kWaveSize, a);
    else if constexpr (kSub == 1)
        launch_async(stream, attention_decode_partial_kernel<16, 1>, grid, 16 * kWaveSize, a);
    else
        throw std::invalid_argument("attention_decode: chunk pairs need at most 8 q heads per kv head");
}

inline void attention_decode_launch(const DecodeAttnArgs &a, int kvh, hipStream_t stream) {
    require(a.chunks_per_record == decode_chunks_per_record(a.kv_rep, a.max_chunks),
            "attention_decode: chunks per record must follow decode_chunks_per_record");
    if (a.chunks_per_record == 2)
        attention_decode_launch_sub<2>(a, kvh, stream);
    else
        attention_decode_launch_sub<1>(a, kvh, stream);
    if (!a.counters)
        launch_async(stream, attention_decode_combine_kernel, kvh, a.kv_rep * kWaveSize, a);
}

} // namespace opworks::detail

namespace opworks::ops {

// Flash-style causal prefill over the cache (reference:
// ops::attention_prefill_chunked, include/ops/attention_prefill.cuh:164-177).
inline void attention_prefill(const float *q_heads, const float *kcache, const float *vcache, float *out, int T,
                              int S, int q_offset, int num_q_heads, int kv_rep, int head_dim, int cap,
                              hipStream_t stream = nullptr) {
    detail::require(T > 0 && S >= T && q_offset == S - T, "attention_prefill: bad shape/offset");
    detail::require(num_q_heads > 0 && kv_rep > 0 && num_q_heads % kv_rep == 0, "attention_prefill: bad head shape");
    detail::require(head_dim > 0 && head_dim <= detail::kAttnMaxD && head_dim % 16 == 0,
                    "attention_prefill supports head_dim in {16,32,48,64}");
    detail::require(cap >= S, "attention_prefill: length exceeds cache capacity");
    detail::require(q_heads && kcache && vcache && out, "attention_prefill requires non-null pointers");
    const float scale = 1.f / std::sqrt(static_cast<float>(head_dim));
    const int kvh = num_q_heads / kv_rep;
    switch (head_dim / 16) {
    case 1: detail::attention_prefill_dispatch<1>(q_heads, kcache, vcache, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream); break;
    case 2: detail::attention_prefill_dispatch<2>(q_heads, kcache, vcache, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream); break;
    case 3: detail::attention_prefill_dispatch<3>(q_heads, kcache, vcache, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream); break;
    default: detail::attention_prefill_dispatch<4>(q_heads, kcache, vcache, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream); break;
    }
}

// Floats and ints the workspace form needs for this shape (thr < 0: the automatic
// threshold), so the caller can size its memory; both 0 when nothing would split.
inline void attention_prefill_workspace_size(int T, int S, int q_offset, int num_q_heads, int kv_rep, int head_dim,
                                             int thr, int64_t *rec_floats, int64_t *counter_ints) {
    detail::require(T > 0 && S >= T && q_offset == S - T, "attention_prefill: bad shape/offset");
    detail::require(num_q_heads > 0 && kv_rep > 0 && num_q_heads % kv_rep == 0, "attention_prefill: bad head shape");
    detail::require(head_dim > 0 && head_dim <= detail::kAttnMaxD && head_dim % 16 == 0,
                    "attention_prefill supports head_dim in {16,32,48,64}");
    const int kvh = num_q_heads / kv_rep;
    detail::PrefillSplitPlan p;
    switch (head_dim / 16) {
    case 1: p = detail::prefill_split_need<1>(T, S, q_offset, kv_rep, kvh, thr); break;
    case 2: p = detail::prefill_split_need<2>(T, S, q_offset, kv_rep, kvh, thr); break;
    case 3: p = detail::prefill_split_need<3>(T, S, q_offset, kv_rep, kvh, thr); break;
    default: p = detail::prefill_split_need<4>(T, S, q_offset, kv_rep, kvh, thr); break;
    }
    *rec_floats = p.rec_floats;
    *counter_ints = p.counter_ints;
}

// Workspace form of attention_prefill, same results to rounding: the query-tile groups with the
// longest K/V ranges run as two workgroups over the halves of the range, merged by the one that
// finishes last, so no CU ends the grid running one long causal range alone. `rec` (rec_floats) needs no
// initialisation; `counters` (counter_ints) must be zero before the first call, and every call
// leaves them at zero. Calls that share a workspace must not overlap. When the memory holds less
// than attention_prefill_workspace_size asks, fewer groups split (none: the plain kernel).
inline void attention_prefill_ws(const float *q_heads, const float *kcache, const float *vcache, float *out, int T,
                                 int S, int q_offset, int num_q_heads, int kv_rep, int head_dim, int cap, float *rec,
                                 int64_t rec_floats, int *counters, int64_t counter_ints, int thr = -1,
                                 hipStream_t stream = nullptr, bool merged_heads = false, bool out_bf16 = false) {
    detail::require(T > 0 && S >= T && q_offset == S - T, "attention_prefill: bad shape/offset");
    detail::require(num_q_heads > 0 && kv_rep > 0 && num_q_heads % kv_rep == 0, "attention_prefill: bad head shape");
    detail::require(head_dim > 0 && head_dim <= detail::kAttnMaxD && head_dim % 16 == 0,
                    "attention_prefill supports head_dim in {16,32,48,64}");
    detail::require(cap >= S, "attention_prefill: length exceeds cache capacity");
    detail::require(q_heads && kcache && vcache && out, "attention_prefill requires non-null pointers");
    detail::require(rec_floats >= 0 && counter_ints >= 0 && (rec || rec_floats == 0) && (counters || counter_ints == 0),
                    "attention_prefill_ws: bad workspace");
    const float scale = 1.f / std::sqrt(static_cast<float>(head_dim));
    const int kvh = num_q_heads / kv_rep;
    detail::require(!(merged_heads || out_bf16) || reinterpret_cast<uintptr_t>(out) % 8 == 0,
                    "attention_prefill_ws: merged or bf16 output needs 8-byte alignment");
    const detail::PrefillWorkspaceArgs ws{rec, rec_floats, counters, counter_ints, thr, merged_heads, out_bf16};
    switch (head_dim / 16) {
    case 1: detail::attention_prefill_dispatch<1>(q_heads, kcache, vcache, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream, &ws); break;
    case 2: detail::attention_prefill_dispatch<2>(q_heads, kcache, vcache, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream, &ws); break;
    case 3: detail::attention_prefill_dispatch<3>(q_heads, kcache, vcache, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream, &ws); break;
    default: detail::attention_prefill_dispatch<4>(q_heads, kcache, vcache, out, T, S, q_offset, kv_rep, kvh, cap, scale, stream, &ws); break;
    }
}

// Same contract as the reference's chunked prefill (name kept for drop-in callers).
inline void attention_prefill_chunked(const float *q_heads, const float *kcache, const float *vcache, float *out,
                                      int T, int S, int q_offset, int num_q_heads, int kv_rep, int head_dim, int cap,
                                      hipStream_t stream = nullptr) {
    attention_prefill(q_heads, kcache, vcache, out, T, S, q_offset, num_q_heads, kv_rep, head_dim, cap, stream);
}

inline int attention_decode_workspace_size(int num_q_heads, int max_len, int head_dim) {
    return detail::attention_decode_workspace_floats(num_q_heads, max_len, head_dim);
}

// ints of arrival counters attention_decode_fused needs: one 256-byte line per kv head.
inline int attention_decode_counters_size(int num_q_heads, int kv_rep) {
    detail::require(num_q_heads > 0 && kv_rep > 0 && num_q_heads % kv_rep == 0,
                    "attention_decode requires positive head shape");
    return num_q_heads / kv_rep * detail::kAttnCounterStride;
}

} // namespace opworks::ops

namespace opworks::detail {

inline void attention_decode_enqueue(const float *q, const float *kcache, const float *vcache, float *out,
                                     int num_q_heads, int kv_rep, int head_dim, int len, int max_seq,
                                     float *workspace, int workspace_size, const int *len_ptr, int len_bias,
                                     int max_len, int *counters, hipStream_t stream) {
    require(num_q_heads > 0 && kv_rep > 0 && head_dim > 0 && num_q_heads % kv_rep == 0,
            "attention_decode requires positive head shape");
    require(kv_rep <= kAttnMaxRep, "attention_decode supports at most 16 q heads per kv head");
    require(head_dim <= 64, "attention_decode supports head_dim <= 64");
    const int bound = len_ptr ? max_len : len;
    require(bound > 0 && bound <= max_seq, "attention_decode length outside the cache capacity");
    require(bound <= kAttnDecodeMaxLen, "attention_decode length exceeds 8192");
    require(q && kcache && vcache && out && workspace, "attention_decode requires non-null pointers");
    const int max_chunks = (bound + kAttnChunk - 1) / kAttnChunk;
    require(workspace_size >= num_q_heads * max_chunks * (head_dim + 2), "attention_decode workspace is too small");
    require(head_dim % 4 == 0, "attention_decode needs head_dim to be a multiple of 4");
    require(aligned16(q) && aligned16(kcache) && aligned16(vcache), "attention_decode needs 16-byte aligned q and caches");
    DecodeAttnArgs a{};
    a.q = q;
    a.kcache = kcache;
    a.vcache = vcache;
    a.out = out;
    a.partial = workspace;
    a.len_ptr = len_ptr;
    a.counters = counters;
    a.len = len;
    a.len_bias = len_bias;
    a.kv_rep = kv_rep;
    a.D = head_dim;
    a.cap = max_seq;
    a.max_chunks = max_chunks;
    a.chunks_per_record = decode_chunks_per_record(kv_rep, max_chunks);
    a.scale = 1.f / std::sqrt(static_cast<float>(head_dim));
    attention_decode_launch(a, num_q_heads / kv_rep, stream);
}

} // namespace opworks::detail

namespace opworks::ops {

// Single-query GQA attention over the first len cache entries, workspace form
// (no allocation; graph-capturable). If len_ptr is non-null the length is
// *len_ptr + len_bias, read on the device, and max_len bounds it.
inline void attention_decode_ws(const float *q, const float *kcache, const float *vcache, float *out,
                                int num_q_heads, int kv_rep, int head_dim, int len, int max_seq, float *workspace,
                                int workspace_size, const int *len_ptr = nullptr, int len_bias = 0,
                                int max_len = 0, hipStream_t stream = nullptr) {
    detail::attention_decode_enqueue(q, kcache, vcache, out, num_q_heads, kv_rep, head_dim, len, max_seq, workspace,
                                     workspace_size, len_ptr, len_bias, max_len, nullptr, stream);
}

// The same in one launch: the last chunk workgroup of each kv head to finish
// merges that head group's records. `counters` holds
// attention_decode_counters_size(num_q_heads, kv_rep) ints that are zero
// before the call and are zero again when it completes; calls that share
// counters must not overlap.
inline void attention_decode_fused(const float *q, const float *kcache, const float *vcache, float *out,
                                   int num_q_heads, int kv_rep, int head_dim, int len, int max_seq, float *workspace,
                                   int workspace_size, int *counters, hipStream_t stream = nullptr) {
    detail::require(counters != nullptr, "attention_decode_fused needs its arrival counters");
    detail::attention_decode_enqueue(q, kcache, vcache, out, num_q_heads, kv_rep, head_dim, len, max_seq, workspace,
                                     workspace_size, nullptr, 0, 0, counters, stream);
}

// Reference signature and contract (include/ops/attention_decode.cuh:98-109): one
// scratch-free launch that allocates nothing, so it can be captured in a graph;
// accepts any head_dim in [1, 64], any 4-byte alignment of q and the caches, and
// any kv_rep (q head h reads kv head h / kv_rep). The caches hold
// ceil(num_q_heads / kv_rep) kv heads of max_seq rows.
inline void attention_decode(const float *q, const float *kcache, const float *vcache, float *out, int num_q_heads,
                             int kv_rep, int head_dim, int len, int max_seq, hipStream_t stream = nullptr) {
    detail::require(num_q_heads > 0 && kv_rep > 0 && head_dim > 0, "attention_decode: head counts and head_dim must be positive");
    detail::require(head_dim <= detail::kAttnMaxD, "attention_decode: head_dim must be at most 64");
    detail::require(len > 0 && len <= max_seq, "attention_decode: len must be in [1, max_seq]");
    detail::require(len <= detail::kAttnDecodeMaxLen, "attention_decode: len must be at most 8192");
    detail::require(q && kcache && vcache && out, "attention_decode: null pointer");
    const float scale = 1.f / std::sqrt(static_cast<float>(head_dim));
    launch_async(stream, detail::attention_decode_single_kernel, num_q_heads, detail::kSingleWaves * kWaveSize,
                         q, kcache, vcache, out, num_q_heads, kv_rep, head_dim, len, max_seq, scale);
}

} // namespace opworks::ops

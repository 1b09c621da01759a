#pragma once

// bf16 GEMM with fp32 accumulation on the CDNA4 matrix cores:
//   C[m][n] = epi(sum_k bf16(A[m][k]) * W[n][k] + bias[n]),   W bf16 [N][K] (HF layout).
// A is either fp32 (rounded to bf16, nearest-even, while it is staged into LDS —
// the reference's ops::linear_mma_bf16 contract, include/ops/linear_mma.cuh:24-93)
// or already bf16.
//
// Kernel shape (gfx950):
//  * workgroup tile 256 x 256, 512 threads = 8 waves in 2 x 4; each wave owns
//    128 x 64 outputs (128 accumulator registers);
//  * K tile 64 (128 KB of LDS with bf16 A, 144 KB with fp32 A; one workgroup
//    per CU);
//  * an MFMA operand is 8 consecutive k of one row per lane, so both operands
//    keep their k-contiguous global layout in LDS; the reads of 16
//    consecutive rows fall on disjoint bank groups, by XOR-swizzled 16-byte
//    chunks (chunk c of row r in slot c ^ ((r >> 1) & 7)) where loads go
//    straight to LDS and by 16 bytes of row padding where they are staged in
//    registers;
//  * with bf16 A both operands go from global memory straight into LDS
//    (gfx950 global_load_lds_dwordx4, no register staging) and the wave tile
//    is 8 x 4 v_mfma_f32_16x16x32_bf16 tiles, two MFMA steps per K tile. The
//    workgroup syncs once per K tile, before the last step's MFMAs, whose
//    operands are already in registers: the next tile's first fragments are
//    read while those MFMAs run, so no step waits on the barrier's LDS reads;
//  * with fp32 A both operands are loaded into registers (A raw, rounded when
//    written to LDS) and stored halfway through the current tile's MFMAs, on
//    4 x 2 v_mfma_f32_32x32x16_bf16 tiles (the 16x16 form's fragments would
//    not fit beside the staging registers);
//  * LDS double buffered, the next tile's loads issued before the current
//    tile's MFMAs; inside a tile the next MFMA step's fragments are read while
//    the current step's MFMAs run; same XCD-banded tile order as the fp32
//    kernel.
// On 4096^3 uniformly random bf16 operands the 16x16x32 and 32x32x16 forms gave
// bit-identical outputs (measured on gfx950); the tests hold both to the oracle.

#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "../core/bf16.hpp"
#include "../core/lds_direct.hpp"
#include "../core/hip_utils.hpp"
#include "elementwise.hpp"
#include "gemm_f32.hpp"

namespace opworks::detail {

using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

constexpr int kBfBM = 256, kBfBN = 256;
constexpr int kBfBK = 32; // K granularity of split-K planning (the smaller of the two K tiles)
constexpr int kBfThreads = 512;

// Workgroup tile shapes. Big: 256 x 256 outputs, 8 waves in 2 x 4 (128 x 64 each), one
// workgroup per CU. Small: 128 x 128, 4 waves in 2 x 2 (64 x 64 each), 64 KB of LDS so two
// workgroups share a CU; for short-M products (prefill projections at a few hundred rows), where
// 256 x 256 tiles leave CUs idle or force deep split-K. The small shape exists on the direct
// path only (bf16 A, 16-byte aligned operands).
struct BfBig {
    static constexpr int BM = 256, BN = 256, kThreads = 512, WM = 2, WN = 4, kStages = 2;
};
struct BfSmall {
    static constexpr int BM = 128, BN = 128, kThreads = 256, WM = 2, WN = 2, kStages = 2;
};
// Tall: 128 x 256 outputs, 8 waves in 2 x 4 (64 x 64 each), three LDS stages (144 KB, one
// workgroup per CU), so two K tiles are in flight while one is multiplied. For short-M products
// from 256 rows (the prefill projections). At 512 rows, against two 128 x 128 workgroups per CU
// on two stages (same outputs, bit for bit): gate/up 56-60 -> 43-45 us, down (8 splits) 28-33 ->
// 25-26, qkv 16.0-16.2 -> 14.2-14.9, o_proj 13.9-14.3 -> 13.4-13.6. The third stage is what pays:
// a 256 x 128 tile on two stages ran as slowly as the small tiles (57-59 us for gate/up), on three
// 44-49 us.
struct BfTall {
    static constexpr int BM = 128, BN = 256, kThreads = 512, WM = 2, WN = 4, kStages = 3;
};

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return static_cast<uint32_t>(float_to_bf16_rne(lo)) | (static_cast<uint32_t>(float_to_bf16_rne(hi)) << 16);
}

template <typename TA, bool kVec, typename Epi, GemmStore kStore = GemmStore::store, typename Shape = BfBig>
__global__ __launch_bounds__(Shape::kThreads) void gemm_bf16_mfma_kernel(const TA *__restrict__ A,
                                                                    const uint16_t *__restrict__ W,
                                                                    const float *__restrict__ bias,
                                                                    float *__restrict__ C, int M, int N, int K,
                                                                    Epi epi) {
    static_assert(std::is_same_v<TA, float> || std::is_same_v<TA, uint16_t>, "A is fp32 or bf16 bits");
    constexpr bool kF32A = std::is_same_v<TA, float>;
    constexpr int BK = 64; // against 32: 945 -> 1013-1030 TFLOP/s (bf16 A), 512-token bf16 TTFT 4.5 -> 4.05 ms
    // Both operands go straight from global memory into LDS (gfx950 global_load_lds_dwordx4)
    // on the vector path with bf16 A. With fp32 A, which is rounded on the way in registers,
    // and on the scalar path both are staged through registers.
    constexpr bool kDirect = kVec && !kF32A;
    constexpr int kBM = Shape::BM, kBN = Shape::BN, kT = Shape::kThreads;
    constexpr int kWTM = kBM / Shape::WM, kWTN = kBN / Shape::WN; // outputs per wave
    static_assert(std::is_same_v<Shape, BfBig> || kDirect, "the small and tall tiles run on the direct path only");
    static_assert(kBM == kBN || kDirect, "register staging: both operands stage the same rows per thread");
    constexpr int kStages = Shape::kStages;
    static_assert(kStages == 2 || kDirect, "register staging is double buffered");
    // LDS rows: a direct load writes 1 KB of consecutive bytes, so its rows are unpadded, with
    // chunk c of row r in slot c ^ ((r >> 1) & 7). The LDS serves 256 bytes a cycle, 16 lanes of
    // a 16-byte read, and the reads of 16 consecutive rows at one k then fall on 16 different
    // 16-byte bank groups (with c ^ (r & 7) they fell on 8, two lanes each). Register staging
    // pads each row by 16 bytes instead (a 144-byte stride), which does the same and keeps every
    // read offset a compile-time constant (the swizzle took the fp32-A kernel past 256 registers).
    constexpr int kRowE = kDirect ? BK : BK + 8;       // bf16 elements per LDS row
    constexpr int kCPR = BK / 8;                       // 16-byte chunks (8 k) per tile row
    constexpr int kPer = kBM * kCPR / kT;              // chunks per thread of A (and of B when square)
    constexpr int kPerB = kBN * kCPR / kT;             // chunks per thread of B
    constexpr int kStage = (kBM + kBN) * kRowE;        // uint16 elements per stage
    __shared__ __attribute__((aligned(16))) uint16_t lds[kStages * kStage];

    const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
    int tm, tn;
    gemm_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * kBM, n0 = tn * kBN;
    const int tid = threadIdx.x, lane = tid % kWaveSize;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWaveSize); // uniform: LDS targets in scalar registers
    const int wm = wave / Shape::WN, wn = wave % Shape::WN;
    const int l32 = lane % 32, half = lane / 32;
    const int l16 = lane % 16, quad = lane / 16;
    // The compiler does not count direct loads as writes to the array: without a store it may
    // treat the array as never written and drop the reads. This one never runs (M >= 0).
    if (kDirect && M < 0)
        lds[tid] = 0;

    auto swz = [](int row, int chunk) {
        return row * kRowE + ((kDirect ? chunk ^ ((row >> 1) & 7) : chunk) << 3);
    };

    // Register staging: chunk tid + kT * i of each operand tile (kBM or kBN rows x BK k),
    // row (tid + kT * i) / kCPR. The vector path loads unconditionally from clamped
    // addresses into raw registers (fp32 A is rounded to bf16 only when staged): a load under
    // a branch makes the compiler wait for every load in flight before the next one. Rows past
    // M or N then hold copies of the last row, which only feed outputs that are not stored; the
    // K tail is zeroed when staged.
    using AStage = std::conditional_t<kF32A, f32x4, u32x4>;
    constexpr int kAParts = kF32A ? 2 : 1;
    constexpr int kPerMax = kPer > kPerB ? kPer : kPerB; // chunks i < kPer of A, i < kPerB of B
    AStage ra[kPer][kAParts];
    u32x4 rb[kPerB];
    auto chunk_row = [&](int i) { return (tid + kT * i) / kCPR; };
    auto chunk_k = [&](int i) { return ((tid + kT * i) % kCPR) * 8; };
    auto load_chunk_bf16 = [&](const uint16_t *src, int row, int rows_total, int k) -> u32x4 {
        uint16_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            e[j] = (row < rows_total && k + j < K) ? src[int64_t(row) * K + k + j] : uint16_t(0);
        return u32x4{e[0] | (uint32_t(e[1]) << 16), e[2] | (uint32_t(e[3]) << 16), e[4] | (uint32_t(e[5]) << 16),
                     e[6] | (uint32_t(e[7]) << 16)};
    };
    // Register loads of tile kt: operand A unless with_a is false, operand B if with_b.
    auto global_load = [&](int kt, bool with_a, bool with_b) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < kPerMax; ++i) {
            const int r = chunk_row(i), k = k0 + chunk_k(i);
            if constexpr (kVec) {
                const int ar = m0 + r < M ? m0 + r : M - 1, br = n0 + r < N ? n0 + r : N - 1;
                const int kc = k < K ? k : K - 8;
                if (with_a && i < kPer) {
#pragma unroll
                    for (int p = 0; p < kAParts; ++p)
                        ra[i][p] = *reinterpret_cast<const AStage *>(A + int64_t(ar) * K + kc + 4 * p);
                }
                if (with_b && i < kPerB)
                    rb[i] = *reinterpret_cast<const u32x4 *>(W + int64_t(br) * K + kc);
            } else {
                if (with_a && i < kPer) {
                    if constexpr (kF32A) {
#pragma unroll
                        for (int p = 0; p < 2; ++p)
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const int kk = k + 4 * p + j;
                                ra[i][p][j] = (m0 + r < M && kk < K) ? A[int64_t(m0 + r) * K + kk] : 0.f;
                            }
                    } else {
                        ra[i][0] = load_chunk_bf16(A, m0 + r, M, k);
                    }
                }
                if (with_b && i < kPerB)
                    rb[i] = load_chunk_bf16(W, n0 + r, N, k);
            }
        }
    };
    auto lds_store = [&](int buf, int kt, bool zero_tail, bool with_a, bool with_b) {
        uint16_t *As = lds + buf * kStage;
        uint16_t *Bs = As + kBM * kRowE;
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < kPerMax; ++i) {
            const int k = k0 + chunk_k(i);
            const int ia = i < kPer ? i : 0, ib = i < kPerB ? i : 0; // in range; unused when i is past
            u32x4 av, bv = rb[ib];
            if constexpr (kF32A)
                av = u32x4{pack_bf16x2(ra[ia][0][0], ra[ia][0][1]), pack_bf16x2(ra[ia][0][2], ra[ia][0][3]),
                           pack_bf16x2(ra[ia][1][0], ra[ia][1][1]), pack_bf16x2(ra[ia][1][2], ra[ia][1][3])};
            else
                av = ra[ia][0];
            if (zero_tail) { // the partial last K tile only: k >= K contributes nothing
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    av[j] = k < K ? av[j] : 0u;
                    bv[j] = k < K ? bv[j] : 0u;
                }
            }
            const int off = swz(chunk_row(i), chunk_k(i) / 8);
            if (with_a && i < kPer)
                *reinterpret_cast<u32x4 *>(As + off) = av;
            if (with_b && i < kPerB)
                *reinterpret_cast<u32x4 *>(Bs + off) = bv;
        }
    };
    // Direct loads of tile kt (full K tiles of the vector path): the wave's instruction i
    // writes the 1 KB block of rows 8 * wave + 8 * waves * i .. + 7, lane l at byte 16 l, i.e.
    // row r = block + l / 8, slot l % 8, which holds chunk (l % 8) ^ ((r >> 1) & 7) of that row;
    // (r >> 1) & 7 = (4 (wave & 1) + l / 16) & 7 for every i (8 * waves is a multiple of 16).
    const int d_row = lane >> 3, d_chunk = (lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7);
    auto direct_load = [&](int buf, int kt) {
        const int k0 = kt * BK + 8 * d_chunk;
        uint16_t *As = lds + buf * kStage;
        uint16_t *Bs = As + kBM * kRowE;
#pragma unroll
        for (int i = 0; i < (kPer > kPerB ? kPer : kPerB); ++i) {
            const int block = 8 * wave + (kT / 8) * i, r = block + d_row;
            const int ar = m0 + r < M ? m0 + r : M - 1, br = n0 + r < N ? n0 + r : N - 1;
            if (i < kPer)
                load_lds16(A + int64_t(ar) * K + k0, As + block * kRowE);
            if (i < kPerB)
                load_lds16(W + int64_t(br) * K + k0, Bs + block * kRowE);
        }
    };
    // s_waitcnt operand for vmcnt(n), expcnt and lgkmcnt at their maxima (gfx9: vmcnt bits 3:0
    // and 15:14): waits until at most n of the wave's vector memory accesses are outstanding.
    constexpr int kLoadsPerStage = kPer + kPerB; // direct loads per thread per stage
    constexpr int kInFlight = (kStages - 2) * kLoadsPerStage;
    static_assert(kInFlight < 64, "vmcnt holds 6 bits");
    constexpr int kWaitOlderStages = kWaitVmcnt0Only | (kInFlight & 15) | ((kInFlight >> 4) << 14);
    // __syncthreads() waits for every outstanding direct load (the compiler's workgroup fence
    // drains vmcnt), which would take the younger stages' loads out of flight. With more than two
    // stages the loop syncs with a bare barrier instead, after this wave's older stages landed
    // (vmcnt) and its LDS reads returned (lgkmcnt(0): no wave overwrites a stage another wave may
    // still be reading). The sched_barrier fences keep the compiler from moving LDS accesses
    // across it.
    auto stage_sync = [] {
        if constexpr (kStages == 2) {
            __syncthreads();
        } else {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(kWaitOlderStages & ~0x0F00); // the same vmcnt, lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Accumulators: 16x16 tiles (4 registers each) on the direct path, 32x32 tiles (16) otherwise.
    constexpr int kTile = kDirect ? 16 : 32;
    constexpr int FM = kWTM / kTile, FN = kWTN / kTile;
    using Acc = std::conditional_t<kDirect, f32x4, f32x16>;
    Acc acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
            acc[i][j] = Acc{};

    // Direct path, 16x16x32 MFMAs: fragment set p holds step s's operands, lane l reading row
    // l % 16 of each 16-row tile at k 32 s + 8 (l / 16) .. + 7 (chunk 4 s + l / 16).
    bf16x8 fa[2][FM], fb[2][FN];
    auto read16 = [&](int buf, int s, int p) {
        const uint16_t *As = lds + buf * kStage;
        const uint16_t *Bs = As + kBM * kRowE;
        const int ch = 4 * s + quad;
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
            fa[p][bm] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(
                                                       As + swz(wm * kWTM + bm * 16 + l16, ch)));
#pragma unroll
        for (int bn = 0; bn < FN; ++bn)
            fb[p][bn] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(
                                                       Bs + swz(wn * kWTN + bn * 16 + l16, ch)));
    };
    auto mfma16 = [&](int p) {
        if constexpr (kDirect) {
#pragma unroll
            for (int bm = 0; bm < FM; ++bm)
#pragma unroll
                for (int bn = 0; bn < FN; ++bn)
                    acc[bm][bn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[p][bm], fb[p][bn], acc[bm][bn], 0, 0, 0);
        }
    };
    // The fragment reads issued with a step (FM + FN of them) go one per MFMA at its start.
    auto interleave16 = [] {
#pragma unroll
        for (int j = 0; j < FM + FN; ++j) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // one fragment read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // one MFMA
        }
        __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - FM - FN, 0);
    };

    // One K tile of the register-staged paths: BK / 16 MFMA steps on 32x32x16 tiles. The
    // fragments are double buffered across steps: the next step's six reads are interleaved
    // one per MFMA with the current step's first six MFMAs, so they arrive while the matrix
    // core runs. stage_next() (the next tile's LDS stores, into the other buffer) runs halfway,
    // so its wait for the global loads and its LDS writes overlap the second half's MFMAs
    // (against staging after the last step: 990-999 -> 1019-1025 TFLOP/s).
    auto compute = [&](int buf, auto &&stage_next) {
        const uint16_t *As = lds + buf * kStage;
        const uint16_t *Bs = As + kBM * kRowE;
        constexpr int kSteps = BK / 16;
        bf16x8 a[2][4], b[2][2];
        auto read = [&](int s, bf16x8 (&fa)[4], bf16x8 (&fb)[2]) {
            const int ch = 2 * s + half; // k 16 s + 8 half .. + 7
#pragma unroll
            for (int bm = 0; bm < 4; ++bm)
                fa[bm] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(
                                                        As + swz(wm * kWTM + bm * 32 + l32, ch)));
#pragma unroll
            for (int bn = 0; bn < 2; ++bn)
                fb[bn] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(
                                                        Bs + swz(wn * kWTN + bn * 32 + l32, ch)));
        };
        read(0, a[0], b[0]);
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            if (s + 1 < kSteps)
                read(s + 1, a[(s + 1) & 1], b[(s + 1) & 1]);
            if (s == kSteps / 2)
                stage_next();
            if constexpr (!kDirect) {
#pragma unroll
                for (int bm = 0; bm < 4; ++bm)
#pragma unroll
                    for (int bn = 0; bn < 2; ++bn)
                        acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s & 1][bm], b[s & 1][bn],
                                                                              acc[bm][bn], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 6, 0); // step 0's reads
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            if (s + 1 < kSteps) {
#pragma unroll
                for (int j = 0; j < 6; ++j) {
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // one of step s + 1's reads
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // one of step s's MFMAs
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            } else {
                __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
            }
        }
    };

    // K tiles of this workgroup: all of them, or split blockIdx.y's contiguous share
    const int ktiles_all = (K + BK - 1) / BK;
    const int per_split = (ktiles_all + gridDim.y - 1) / gridDim.y;
    const int kt_begin = blockIdx.y * per_split;
    const int kt_end = kt_begin + per_split < ktiles_all ? kt_begin + per_split : ktiles_all;
    // The vector path pipelines its full K tiles and runs a partial last tile (K not a multiple
    // of the K tile) after the loop, with the tail zeroed; the scalar path bounds every element.
    const int kt_full = kVec ? (K / BK < kt_end ? (K / BK > kt_begin ? K / BK : kt_begin) : kt_end) : kt_end;
    if constexpr (kDirect) {
      if (kt_begin < kt_full) {
        // Per K tile: the next tile's direct loads into the idle stage, step 0's MFMAs with step
        // 1's fragments read in between, then (every wave's loads landed, every read of this tile
        // done) one barrier, and step 1's MFMAs with the next tile's step-0 fragments read in
        // between. The idle stage was last read before the previous tile's barrier.
        // (4096^3, bf16 A, on one box: 123-126 us with a barrier at the end of each tile on
        // 32x32x16 tiles, 112-114 us with this barrier, 102.5-104 us on 16x16x32 tiles.)
        // With kStages stages the loads run kStages - 1 tiles ahead: tile kt + kStages - 1 goes
        // into the stage tile kt - 1 used, which no wave reads after the previous barrier, and
        // the wait before each barrier leaves the younger tiles' loads (kInFlight) outstanding.
        for (int s = 0; s + 1 < kStages; ++s)
            direct_load(s, kt_begin + s < kt_full ? kt_begin + s : kt_full - 1);
        __builtin_amdgcn_s_waitcnt(kWaitOlderStages);
        stage_sync();
        read16(0, 0, 0);
        for (int kt = kt_begin; kt < kt_full; ++kt) {
            const int j = kt - kt_begin;
            const int buf = kStages == 2 ? (j & 1) : j % kStages;
            const int nbuf = kStages == 2 ? (buf ^ 1) : (buf + 1 == kStages ? 0 : buf + 1);
            const int lbuf = kStages == 2 ? (buf ^ 1) : (buf == 0 ? kStages - 1 : buf - 1);
            // past the last tile: a reload of a valid tile into the idle stage, never read (a
            // peeled last tile without it took the residual epilogue into spills)
            const int next = kt + kStages - 1 < kt_full ? kt + kStages - 1 : kt_full - 1;
            direct_load(lbuf, next);
            __builtin_amdgcn_sched_barrier(0); // the loads stay at the top, in flight during the MFMAs
            read16(buf, 1, 1);
            mfma16(0);
            interleave16();
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(kWaitOlderStages); // this wave's loads of the next tile landed
            stage_sync();
            __builtin_amdgcn_sched_barrier(0);
            read16(nbuf, 0, 0);
            mfma16(1);
            interleave16();
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (kInFlight > 0) // the reloads past the end land before the stages are reused
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0Only);
      }
    } else if (kt_begin < kt_full) {
        // Each K tile: the next tile's loads are issued first into registers, stored halfway
        // through the MFMA steps, then the workgroup syncs once.
        global_load(kt_begin, true, true);
        lds_store(0, kt_begin, false, true, true);
        __syncthreads();
        for (int kt = kt_begin; kt < kt_full; ++kt) {
            const int buf = (kt - kt_begin) & 1;
            const int next = kt + 1 < kt_full ? kt + 1 : kt;
            global_load(next, true, true);
            __builtin_amdgcn_sched_barrier(0);
            compute(buf, [&] { lds_store(buf ^ 1, next, false, true, true); });
            __syncthreads();
        }
    }
    if (kt_full < kt_end) { // the partial last K tile (vector path), staged through registers
        __syncthreads(); // every wave is done with the stages (the direct path's last reads)
        global_load(kt_full, true, true);
        lds_store(0, kt_full, true, true, true);
        __syncthreads();
        if constexpr (kDirect) {
            read16(0, 0, 0);
            read16(0, 1, 1);
            mfma16(0);
            mfma16(1);
        } else {
            compute(0, [] {});
        }
    }
    if constexpr (kStore == GemmStore::partial)
        C += int64_t(blockIdx.y) * M * N;

    // Accumulator register r of a 16x16 tile holds row 4 (l / 16) + r, column l % 16; of a 32x32
    // tile, row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32. A tile inside C on both axes stores
    // without bounds tests (each test compiled to an exec-mask branch per store).
    auto store_tile = [&](auto checked_t) {
        constexpr bool checked = decltype(checked_t)::value;
        constexpr int kRegs = kDirect ? 4 : 16; // accumulator registers per tile
        // A store counts in vmcnt like a load, so a load issued after stores waits for them too:
        // every bias value is loaded before the first store, and the residual C values of a
        // batch of tiles before its stores (one drain per batch, not one per element).
        float bv[FN];
#pragma unroll
        for (int bn = 0; bn < FN; ++bn)
            bv[bn] = 0.f;
        if (kStore != GemmStore::partial && bias != nullptr) { // one uniform test for every column
#pragma unroll
            for (int bn = 0; bn < FN; ++bn) {
                const int col = n0 + wn * kWTN + bn * kTile + (kDirect ? l16 : l32);
                bv[bn] = (!checked || col < N) ? bias[col] : 0.f;
            }
        }
        auto row_of = [&](int bm, int r) {
            return kDirect ? m0 + wm * kWTM + bm * 16 + 4 * quad + r
                           : m0 + wm * kWTM + bm * 32 + 8 * (r / 4) + 4 * half + (r % 4);
        };
        // residual loads per batch of 16 values: four 16x16 tiles or one 32x32 tile (larger batches
        // pushed both paths into spills)
        constexpr int kBatch = kDirect ? 4 : 1;
#pragma unroll
        for (int bn = 0; bn < FN; ++bn) {
            const int col = n0 + wn * kWTN + bn * kTile + (kDirect ? l16 : l32);
            const bool col_ok = !checked || col < N;
#pragma unroll
            for (int bm0 = 0; bm0 < FM; bm0 += kBatch) {
                float prev[kBatch][kRegs];
                if constexpr (kStore == GemmStore::residual) {
#pragma unroll
                    for (int i = 0; i < kBatch; ++i)
#pragma unroll
                        for (int r = 0; r < kRegs; ++r) {
                            const int row = row_of(bm0 + i, r);
                            prev[i][r] = (!checked || (row < M && col_ok)) ? C[int64_t(row) * N + col] : 0.f;
                        }
                }
#pragma unroll
                for (int i = 0; i < kBatch; ++i) {
                    const int bm = bm0 + i;
#pragma unroll
                    for (int r = 0; r < kRegs; ++r) {
                        const int row = row_of(bm, r);
                        const bool ok = !checked || (row < M && col_ok);
                        if constexpr (kStore == GemmStore::partial) {
                            if (ok)
                                C[int64_t(row) * N + col] = acc[bm][bn][r];
                            continue;
                        }
                        const float v = epi(acc[bm][bn][r] + bv[bn]);
                        if constexpr (kStore == GemmStore::swiglu || kStore == GemmStore::swiglu_bf16) {
                            const float partner = __shfl_xor(v, 1); // lane l ^ 1 holds column col ^ 1
                            if ((col & 1) == 0 && (!checked || (row < M && col + 1 < N))) {
                                const float y = v / (1.f + expf(-v)) * partner;
                                if constexpr (kStore == GemmStore::swiglu)
                                    C[int64_t(row) * (N / 2) + col / 2] = y;
                                else
                                    reinterpret_cast<uint16_t *>(C)[int64_t(row) * (N / 2) + col / 2] =
                                        float_to_bf16_rne(y);
                            }
                        } else if constexpr (kStore == GemmStore::residual) {
                            if (ok)
                                C[int64_t(row) * N + col] = prev[i][r] + v;
                        } else {
                            if (ok)
                                C[int64_t(row) * N + col] = v;
                        }
                    }
                }
            }
        }
    };
    // The register-staged paths keep the checked form only: a second copy pushed them into spills.
    if constexpr (kDirect) {
        if (m0 + kBM <= M && n0 + kBN <= N)
            store_tile(std::false_type{});
        else
            store_tile(std::true_type{});
    } else {
        store_tile(std::true_type{});
    }
}

// C written per kStore (see GemmStore): store, += (residual), or SwiGLU of
// interleaved (gate, up) column pairs into C[M][N / 2].
template <typename TA, typename Epi, GemmStore kStore = GemmStore::store>
void gemm_bf16_launch(const TA *A, const uint16_t *W, const float *bias, float *C, int M, int N, int K, Epi epi,
                      hipStream_t stream, int splits = 1) {
    require((kStore != GemmStore::swiglu && kStore != GemmStore::swiglu_bf16) || N % 2 == 0,
            "swiglu epilogue needs an even number of columns");
    const int tiles = static_cast<int>(blocks_for64(M, kBfBM) * blocks_for64(N, kBfBN));
    const dim3 grid(tiles, splits);
    const bool vec = aligned16(A) && aligned16(W) && K % 8 == 0;
    if (vec)
        launch_async(stream, gemm_bf16_mfma_kernel<TA, true, Epi, kStore>, grid, kBfThreads, A, W, bias, C, M, N, K,
                     epi);
    else
        launch_async(stream, gemm_bf16_mfma_kernel<TA, false, Epi, kStore>, grid, kBfThreads, A, W, bias, C, M, N, K,
                     epi);
}

// Floats of split-K workspace any launch planned by splitk_factor(tiles, ., 256) needs (the
// small- and tall-tile plans below stay within it: splits x tiles <= 512 tiles of a quarter the
// size, or <= 256 of half).
constexpr int64_t kSplitKWorkspaceBf16 = int64_t(256) * kBfBM * kBfBN;

// Split-K form of gemm_bf16_launch for store / residual outputs (see
// gemm_f32_launch_splitk); 256-wide tiles, so one round of 256 workgroups.
template <typename TA, typename Epi, GemmStore kStore>
void gemm_bf16_launch_splitk(const TA *A, const uint16_t *W, const float *bias, float *C, int M, int N, int K,
                             Epi epi, float *ws, int64_t ws_floats, hipStream_t stream) {
    const int tiles = static_cast<int>(blocks_for64(M, kBfBM) * blocks_for64(N, kBfBN));
    const int splits = splitk_factor(tiles, static_cast<int>(blocks_for64(K, kBfBK)), 256);
    if (splits == 1 || N % 4 != 0 || !ws || int64_t(splits) * M * N > ws_floats || !aligned16(C) ||
        (bias && !aligned16(bias))) {
        gemm_bf16_launch<TA, Epi, kStore>(A, W, bias, C, M, N, K, epi, stream);
        return;
    }
    gemm_bf16_launch<TA, IdentityEpilogue, GemmStore::partial>(A, W, nullptr, ws, M, N, K, IdentityEpilogue{}, stream,
                                                               splits);
    launch_async(stream, splitk_reduce_kernel<Epi, kStore>, stream_grid(int64_t(M) * N / 4), 256, ws, splits, bias, C,
                 M, N, epi);
}

// bf16 A on the direct path (both operands straight into LDS), for any M: 256 x 256 tiles when
// they fill the GPU's 256 CUs, else 128 x 256 three-stage tiles from 256 rows (one workgroup per
// CU) and 128 x 128 tiles below (two per CU), and for store / residual outputs K split across
// workgroups toward one round of the GPU, at least 8 K tiles of 64 per split, the partial tiles
// summed in split order by splitk_reduce_kernel. At M = 512 (a 512-token prefill) the 256 x 256
// tiles gave gate/up 128 workgroups and qkv, o_proj and down 8-way splits on 16-24 tiles.
// `reduce` as in gemm_f32_launch_splitk: called as reduce(ws, splits) in place of the reduction
// kernel when K is split (small and tall tiles only). Returns true when it was.
template <typename Epi, GemmStore kStore, typename Reduce = std::nullptr_t>
bool gemm_bf16_launch_direct(const uint16_t *A, const uint16_t *W, const float *bias, float *C, int M, int N, int K,
                             Epi epi, float *ws, int64_t ws_floats, hipStream_t stream, Reduce reduce = nullptr) {
    const bool vec = aligned16(A) && aligned16(W) && K % 8 == 0;
    const int big_tiles = static_cast<int>(blocks_for64(M, kBfBM) * blocks_for64(N, kBfBN));
    constexpr bool kSwiglu = kStore == GemmStore::swiglu || kStore == GemmStore::swiglu_bf16;
    require(!kSwiglu || N % 2 == 0, "swiglu epilogue needs an even number of columns");
    if (!vec || big_tiles >= 256) {
        if constexpr (kSwiglu)
            gemm_bf16_launch<uint16_t, Epi, kStore>(A, W, bias, C, M, N, K, epi, stream);
        else
            gemm_bf16_launch_splitk<uint16_t, Epi, kStore>(A, W, bias, C, M, N, K, epi, ws, ws_floats, stream);
        return false;
    }
    // One workgroup per CU for the tall tiles, two for the small ones: split toward that many.
    auto run = [&](auto shape, int target) {
        using S = decltype(shape);
        const int tiles = static_cast<int>(blocks_for64(M, S::BM) * blocks_for64(N, S::BN));
        int splits = 1;
        if constexpr (!kSwiglu) {
            splits = splitk_factor(tiles, static_cast<int>(blocks_for64(K, 64)), target);
            if (N % 4 != 0 || !ws || int64_t(splits) * M * N > ws_floats || !aligned16(C) ||
                (bias && !aligned16(bias)))
                splits = 1;
        }
        if (splits == 1)
            launch_async(stream, gemm_bf16_mfma_kernel<uint16_t, true, Epi, kStore, S>, dim3(tiles, 1), S::kThreads,
                         A, W, bias, C, M, N, K, epi);
        else
            launch_async(stream, gemm_bf16_mfma_kernel<uint16_t, true, IdentityEpilogue, GemmStore::partial, S>,
                         dim3(tiles, splits), S::kThreads, A, W, static_cast<const float *>(nullptr), ws, M, N, K,
                         IdentityEpilogue{});
        return splits;
    };
    const int splits = M >= 256 ? run(BfTall{}, 256) : run(BfSmall{}, 512);
    if (splits == 1)
        return false;
    if constexpr (!kSwiglu) {
        if constexpr (std::is_same_v<Reduce, std::nullptr_t>)
            launch_async(stream, splitk_reduce_kernel<Epi, kStore>, stream_grid(int64_t(M) * N / 4), 256, ws, splits,
                         bias, C, M, N, epi);
        else
            reduce(ws, splits);
    }
    return true;
}

} // namespace opworks::detail

#pragma once

// fp32 GEMM on bf16 MFMAs with three-part operands ("bf16x6", core/bf16x6.hpp):
//   C[m][n] = epi(sum_k A[m][k] B(k, n) + bias[n]),   A fp32 [M][K] k-contiguous, and B either
// W [N][K] (nk, the HF weight layout) or B [K][N] (kn, the reference's mat_mul); 16-byte aligned,
// K a multiple of 8, and N a multiple of 4 for kn. Every fp32 operand value splits
// exactly into three bf16 parts and each product keeps the six terms x_i y_j with i + j <= 2,
// accumulated in fp32 by the MFMA: the products carry fp32's error (each dropped term is at most
// 2^-24 of |x y|, 2^-23 together), on 16-cycle 16x16x32 bf16 MFMAs. Per 16x16x32 block of
// products that is 6 x 16 = 96 matrix-core cycles against 8 x 32 = 256 on 16x16x4 fp32 MFMAs.
//
// Kernel shape (gfx950): 128 x 256 outputs per workgroup, 512 lanes as 2 x 4 waves of 64 x 64
// (4 x 4 16x16 accumulator tiles); K steps of 32. Each step's fp32 tiles are loaded into
// registers one step ahead, split, and written as three bf16 planes per operand into the idle
// LDS stage (72 KB per stage, two stages, one workgroup per CU); a kn-layout B is transposed on the
// way (each thread holds 4 k x 4 n and writes 8-byte pieces of n-major rows). Plane rows are 64 bytes with
// their 16-byte chunks swizzled (x6_k_chunk<32>, measured conflict-free for these reads). A
// wave reads its 3 x (4 + 4) fragments of a step and issues 6 x 16 MFMAs, smallest terms first,
// with the next step's split and LDS writes interleaved with the last two terms' MFMAs.

// Included by gemm_f32.hpp ahead of its launchers, which send fp32 products here; it
// uses that header's GemmStore, gemm_tile_of and IdentityEpilogue. Include gemm_f32.hpp, not this.

#include <cstdint>
#include <type_traits>

#include "../core/bf16x6.hpp"
#include "../core/hip_utils.hpp"

namespace opworks::detail {

struct GemmX6Shape {
    static constexpr int BM = 128, BN = 256, BK = 32, kThreads = 512, WM = 2, WN = 4;
};

template <BLayout kB, typename Epi, GemmStore kStore>
__global__ __launch_bounds__(GemmX6Shape::kThreads) void gemm_x6_kernel(const float *__restrict__ A,
                                                                       const float *__restrict__ W,
                                                                       const float *__restrict__ bias,
                                                                       float *__restrict__ C, int M, int N, int K,
                                                                       Epi epi) {
    using S = GemmX6Shape;
    constexpr int BM = S::BM, BN = S::BN, BK = S::BK, kT = S::kThreads;
    constexpr int kWTM = BM / S::WM, kWTN = BN / S::WN; // 64 x 64 outputs per wave
    constexpr int FM = kWTM / 16, FN = kWTN / 16;
    constexpr int kPlaneA = BM * BK, kPlaneB = BN * BK; // bf16 elements per plane
    constexpr int kStage = 3 * (kPlaneA + kPlaneB);
    static_assert(BM * BK / 8 == kT && BN * BK / 8 == 2 * kT, "one A chunk and two B chunks of 8 k per thread");
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStage];

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    gemm_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid % kWaveSize;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWaveSize);
    const int wm = wave / S::WN, wn = wave % S::WN;
    const int l16 = lane % 16, quad = lane / 16;

    // Staging: 8 consecutive k of one row per chunk; A chunk tid is row tid / 4, B chunks tid and
    // tid + kT rows tid / 4 and tid / 4 + 128, all at k 8 (tid % 4) of the step. Rows past M or N
    // read the last row (those outputs are not stored) and chunks past K read a valid chunk and
    // are zeroed, so every load is issued unconditionally.
    const int kc = tid % 4, srow = tid / 4;
    const float *arow = A + int64_t(m0 + srow < M ? m0 + srow : M - 1) * K;
    // nk: B rows srow and srow + 128 of the tile. kn: thread (q, o) = (tid % 64, tid / 64) holds
    // columns 4q .. 4q + 3 of the tile at k 4o .. 4o + 3 (a wave reads 1 KB of one k row per load);
    // columns past N read the last four (N % 4 == 0), rows past K read row K - 1 and are zeroed.
    const float *brow0 = W + (kB == BLayout::nk ? int64_t(n0 + srow < N ? n0 + srow : N - 1) * K : 0);
    const float *brow1 = W + (kB == BLayout::nk ? int64_t(n0 + srow + 128 < N ? n0 + srow + 128 : N - 1) * K : 0);
    const int bq = tid % 64, bo = tid / 64;
    const int bcol = n0 + 4 * bq + 3 < N ? n0 + 4 * bq : N - 4;
    f32x4 ra[2], rb[2][2], rk[4];
    bool kin = true;
    int kin_rows = 0; // kn: bit i set when row k 4o + i of the step lies inside K
    auto gload = [&](int kt) {
        const int k = kt * BK + 8 * kc;
        kin = k < K;
        const int kl = kin ? k : K - 8;
        ra[0] = *reinterpret_cast<const f32x4 *>(arow + kl);
        ra[1] = *reinterpret_cast<const f32x4 *>(arow + kl + 4);
        if constexpr (kB == BLayout::nk) {
            rb[0][0] = *reinterpret_cast<const f32x4 *>(brow0 + kl);
            rb[0][1] = *reinterpret_cast<const f32x4 *>(brow0 + kl + 4);
            rb[1][0] = *reinterpret_cast<const f32x4 *>(brow1 + kl);
            rb[1][1] = *reinterpret_cast<const f32x4 *>(brow1 + kl + 4);
        } else {
            kin_rows = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kr = kt * BK + 4 * bo + i;
                kin_rows |= (kr < K ? 1 : 0) << i;
                rk[i] = *reinterpret_cast<const f32x4 *>(W + int64_t(kr < K ? kr : K - 1) * N + bcol);
            }
        }
    };
    auto slot = [](int row, int chunk) { return row * BK + 8 * x6_k_chunk<32>(chunk, row); };
    auto put = [&](uint16_t *plane0, int plane_elems, int row, const f32x4 (&x)[2]) {
        const float v[8] = {x[0][0], x[0][1], x[0][2], x[0][3], x[1][0], x[1][1], x[1][2], x[1][3]};
        float z[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            z[j] = kin ? v[j] : 0.f;
        bf16x8v part[3];
        split3x8(z, part);
        const int off = slot(row, kc);
#pragma unroll
        for (int p = 0; p < 3; ++p)
            *reinterpret_cast<bf16x8v *>(plane0 + p * plane_elems + off) = part[p];
    };
    auto commit = [&](int buf) {
        uint16_t *st = lds + buf * kStage;
        put(st, kPlaneA, srow, ra);
        if constexpr (kB == BLayout::nk) {
            put(st + 3 * kPlaneA, kPlaneB, srow, rb[0]);
            put(st + 3 * kPlaneA, kPlaneB, srow + 128, rb[1]);
        } else { // column 4q + j: its four k values, split, as 8-byte pieces of the n-major rows
            uint16_t *pb = st + 3 * kPlaneA;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    v[i] = (kin_rows >> i) & 1 ? rk[i][j] : 0.f;
                uint32_t w[3][2];
                split3x2(v[0], v[1], w[0][0], w[1][0], w[2][0]);
                split3x2(v[2], v[3], w[0][1], w[1][1], w[2][1]);
                const int row = 4 * bq + j;
                const int off = row * BK + 8 * x6_k_chunk<32>(bo / 2, row) + 4 * (bo % 2);
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    *reinterpret_cast<uint2 *>(pb + p * kPlaneB + off) = uint2{w[p][0], w[p][1]};
            }
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
            acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // One K step from stage buf: B part 0 and A part 2 first (the first term's operands), then
    // the rest in the order the terms use them. `mid` runs before the fifth of the six terms: the
    // next step's split and LDS writes, whose VALU work then overlaps the last two terms' MFMAs
    // (against after the sixth, on one box: 4096^3 kn 651 -> 636 us, 512 x 16384 x 2048 166 ->
    // 158 us, 4096^3 nk unchanged; same outputs).
    auto step = [&](int buf, auto &&mid) {
        const uint16_t *st = lds + buf * kStage;
        const uint16_t *pa = st, *pb = st + 3 * kPlaneA;
        bf16x8v fa[3][FM], fb[3][FN];
        auto ra16 = [&](int p, int bm) {
            const int row = wm * kWTM + 16 * bm + l16;
            fa[p][bm] = *reinterpret_cast<const bf16x8v *>(pa + p * kPlaneA + slot(row, quad));
        };
        auto rb16 = [&](int p, int bn) {
            const int row = wn * kWTN + 16 * bn + l16;
            fb[p][bn] = *reinterpret_cast<const bf16x8v *>(pb + p * kPlaneB + slot(row, quad));
        };
#pragma unroll
        for (int bn = 0; bn < FN; ++bn)
            rb16(0, bn);
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
            ra16(2, bm);
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
            ra16(1, bm);
#pragma unroll
        for (int bn = 0; bn < FN; ++bn)
            rb16(1, bn);
#pragma unroll
        for (int bm = 0; bm < FM; ++bm)
            ra16(0, bm);
#pragma unroll
        for (int bn = 0; bn < FN; ++bn)
            rb16(2, bn);
        auto terms = [&](int t0, int t1) {
#pragma unroll
            for (int term = t0; term < t1; ++term)
#pragma unroll
                for (int bm = 0; bm < FM; ++bm)
#pragma unroll
                    for (int bn = 0; bn < FN; ++bn) {
                        const bf16x8v a[3] = {fa[0][bm], fa[1][bm], fa[2][bm]};
                        const bf16x8v b[3] = {fb[0][bn], fb[1][bn], fb[2][bn]};
                        acc[bm][bn] = mfma_x6_term(term, a, b, acc[bm][bn]);
                    }
        };
        terms(0, 4);
        // The last two terms' 2 x 16 MFMAs interleaved with `mid`'s split (VALU) and LDS writes:
        // a wave issues in order, so without this its MFMAs wait behind the whole split (4096^3:
        // kn 209 -> 218-220 TFLOP/s, nk 223 -> 230; the same from the fourth term on).
        __builtin_amdgcn_sched_barrier(0);
        mid();
        terms(4, 6);
#pragma unroll
        for (int i = 0; i < 2 * FM * FN; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0); // up to five VALU
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0); // up to one LDS write
        }
    };

    // K steps of this workgroup: all, or blockIdx.y's contiguous share when K is split
    const int ksteps = (K + BK - 1) / BK;
    const int per_split = (ksteps + gridDim.y - 1) / gridDim.y;
    const int kt_begin = blockIdx.y * per_split;
    const int kt_end = kt_begin + per_split < ksteps ? kt_begin + per_split : ksteps;
    if (kt_begin < kt_end) {
        gload(kt_begin);
        commit(0);
        __syncthreads();
        for (int kt = kt_begin; kt < kt_end; ++kt) {
            const int buf = (kt - kt_begin) & 1;
            gload(kt + 1 < kt_end ? kt + 1 : kt); // past the end: a valid step again, never read
            __builtin_amdgcn_sched_barrier(0);    // the loads go out before the step's MFMAs
            step(buf, [&] { commit(buf ^ 1); });  // the idle stage, last read before the previous barrier
            __syncthreads();
        }
    }
    if constexpr (kStore == GemmStore::partial)
        C += int64_t(blockIdx.y) * M * N;

    // Accumulator register r of tile (bm, bn) holds row 4 quad + r, column l16 of the tile.
    auto store_tile = [&](auto checked_t) {
        constexpr bool checked = decltype(checked_t)::value;
        float bv[FN];
#pragma unroll
        for (int bn = 0; bn < FN; ++bn) {
            const int col = n0 + wn * kWTN + 16 * bn + l16;
            bv[bn] = (kStore != GemmStore::partial && bias != nullptr && (!checked || col < N)) ? bias[col] : 0.f;
        }
#pragma unroll
        for (int bn = 0; bn < FN; ++bn) {
            const int col = n0 + wn * kWTN + 16 * bn + l16;
            const bool col_ok = !checked || col < N;
#pragma unroll
            for (int bm = 0; bm < FM; ++bm) {
                float prev[4] = {0.f, 0.f, 0.f, 0.f};
                if constexpr (kStore == GemmStore::residual) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int row = m0 + wm * kWTM + 16 * bm + 4 * quad + r;
                        prev[r] = (!checked || (row < M && col_ok)) ? C[int64_t(row) * N + col] : 0.f;
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + wm * kWTM + 16 * bm + 4 * quad + r;
                    const bool ok = !checked || (row < M && col_ok);
                    if constexpr (kStore == GemmStore::partial) {
                        if (ok)
                            C[int64_t(row) * N + col] = acc[bm][bn][r];
                    } else {
                        const float v = epi(acc[bm][bn][r] + bv[bn]);
                        if constexpr (kStore == GemmStore::swiglu) {
                            const float partner = __shfl_xor(v, 1); // lane l ^ 1 holds column col ^ 1
                            if ((col & 1) == 0 && (!checked || (row < M && col + 1 < N)))
                                C[int64_t(row) * (N / 2) + col / 2] = v / (1.f + expf(-v)) * partner;
                        } else if constexpr (kStore == GemmStore::residual) {
                            if (ok)
                                C[int64_t(row) * N + col] = prev[r] + v;
                        } else {
                            if (ok)
                                C[int64_t(row) * N + col] = v;
                        }
                    }
                }
            }
        }
    };
    if (m0 + BM <= M && n0 + BN <= N)
        store_tile(std::false_type{});
    else
        store_tile(std::true_type{});
}

// Whether the bf16x6 kernel takes this product: both operands 16-byte aligned, A's rows in chunks
// of 8 k, and for a kn-layout B whole groups of 4 columns.
template <BLayout kB> inline bool gemm_x6_ok(const float *A, const float *B, int N, int K) {
    return aligned16(A) && aligned16(B) && K % 8 == 0 && K > 0 && (kB == BLayout::nk || (N % 4 == 0 && N >= 4));
}

template <BLayout kB, typename Epi, GemmStore kStore>
void gemm_x6_launch(const float *A, const float *B, const float *bias, float *C, int M, int N, int K, Epi epi,
                    hipStream_t stream, int splits = 1) {
    static_assert(kStore != GemmStore::swiglu_bf16, "the bf16x6 GEMM stores fp32");
    require((kStore != GemmStore::swiglu) || N % 2 == 0, "swiglu epilogue needs an even number of columns");
    require(gemm_x6_ok<kB>(A, B, N, K), "gemm_x6: operands must be 16-byte aligned with K a multiple of 8 "
                                        "(and N a multiple of 4 for a kn-layout B)");
    using S = GemmX6Shape;
    const int64_t tiles = blocks_for64(M, S::BM) * blocks_for64(N, S::BN);
    require(tiles <= INT32_MAX && splits >= 1, "gemm_x6: grid too large");
    launch_async(stream, gemm_x6_kernel<kB, Epi, kStore>, dim3(static_cast<unsigned>(tiles), splits), S::kThreads, A,
                 B, bias, C, M, N, K, epi);
}

} // namespace opworks::detail

#pragma once

// fp32 GEMM on the CDNA4 matrix cores: C[m][n] = epi(sum_k A[m][k] * B(k, n) + bias[n]).
//
// A comes in two layouts: ALayout::mk — A[m][k], k contiguous (the usual
// row-major operand) — and ALayout::km — A[k][m], m contiguous (a transposed
// operand, MatmulBuilder::transpose_a), staged like the kn-layout B.
// B comes in two layouts:
//  * BLayout::kn — B[k][n], n contiguous: ops::mat_mul (reference
//    include/ops/matmul.cuh:11-91, where the reduction dim is called N);
//  * BLayout::nk — B[n][k], k contiguous: ops::linear's Y = X W^T with HF
//    [out, in] weights (reference include/ops/linear.cuh:18-73).
//
// Kernel shapes (gfx950), all on v_mfma_f32_16x16x4_f32 with K tiles of 16:
//  * GemmBig: workgroup tile 256 x 256, 512 threads = 8 waves in 4 x 2, each
//    wave owns 64 x 128 = 4 x 8 MFMA tiles (128 accumulator registers); used
//    when the output has at least 256 such tiles (one per CU) and K is not
//    split, e.g. the 4096^3 GEMM;
//  * GemmMid: 256 x 128, 512 threads = 8 waves in 4 x 2, each 64 x 64; when
//    fewer than 256 GemmBig tiles but at least 256 of these cover the output;
//  * GemmSmall: 128 x 128, 256 threads = 4 waves in 2 x 2, each 64 x 64; for
//    smaller outputs and the split-K partial tiles.
// Measured on 4096^3 fp32: 256 x 256 / 8 waves / 16x16x4 at 126-128 TFLOP/s,
// against 117-120 for every 128 x 128 variant of 32x32x2 or 16x16x4 MFMA, K
// tile 16 or 32, and one or two register staging sets.
//  * operands are staged through LDS, double buffered, one barrier per K tile,
//    before its last MFMA step; the next tile's global loads are issued before
//    the current tile's MFMAs and its first fragments read during that step;
//  * K is permuted per 16-lane group: in a K tile, MFMA step j of lane group g
//    (lanes 16g .. 16g + 15) uses k = 4g + j. A product sum does not depend on
//    the order of k, and this order lets a k-contiguous operand (A, and B in
//    the nk layout) keep its global layout in LDS (rows padded to 20 floats,
//    so 16 consecutive rows fall on disjoint bank groups) and deliver four
//    MFMA steps with one ds_read_b128; the kn-layout B is read one float per
//    step from rows padded to BN + 4 floats, which puts the four lane groups
//    (4 rows apart) on disjoint banks;
//  * workgroup ids are remapped so each XCD (its own L2) works on a
//    contiguous band of tiles, then grouped 8 tile-rows at a time.
// Accumulation is fp32 on the matrix core; the result differs from a
// k-ascending fmaf chain only by summation order.

#include <cstddef>
#include <cstdlib>
#include <cstdint>
#include <type_traits>

#include "../core/hip_utils.hpp"
#include "elementwise.hpp"

namespace opworks::detail {

enum class BLayout { kn, nk };
enum class ALayout { mk, km };

using f32x16 = float __attribute__((ext_vector_type(16)));

template <int kBM, int kBN, int kWM, int kWN, int kBK = 16> struct GemmF32Shape {
    static constexpr int BM = kBM, BN = kBN, BK = kBK, WM = kWM, WN = kWN;
    static_assert(BK % 16 == 0, "a K tile is a whole number of 16-k MFMA groups");
    static constexpr int kThreads = WM * WN * kWaveSize;
    static constexpr int TM = BM / WM, TN = BN / WN;   // wave tile
    static constexpr int FM = TM / 16, FN = TN / 16;   // 16 x 16 MFMA tiles per wave
    static constexpr int LdK = BK + 4;                 // padded row of a k-contiguous tile
    static constexpr int LdN = BN + 4;                 // padded row of the kn-layout B tile
    static constexpr int LdM = BM + 4;                 // padded row of the km-layout A tile
    static constexpr int CA = BM * BK / 4 / kThreads;  // 16-byte A chunks per thread per K tile
    static constexpr int CB = BN * BK / 4 / kThreads;  // 16-byte B chunks per thread per K tile
    static_assert(CA * kThreads * 4 == BM * BK && CB * kThreads * 4 == BN * BK, "tile / thread mismatch");
};
using GemmSmall = GemmF32Shape<128, 128, 2, 2>;
using GemmBig = GemmF32Shape<256, 256, 4, 2>; // a K tile of 32 measured 132.4 against 133.5 TFLOP/s
using GemmMid = GemmF32Shape<256, 128, 4, 2>; // 8 waves of 64 x 64
constexpr int kGemmBK = 16;
constexpr int kNumXcd = 8;

struct IdentityEpilogue {
    __device__ float operator()(float x) const { return x; }
};

// How the epilogue writes C (all modes apply epi(acc + bias[col]) first):
//  store    C[row][col] = v
//  residual C[row][col] += v                     (C holds the residual stream)
//  swiglu   columns (2i, 2i+1) hold (gate_i, up_i): C[row][i] = silu(gate) * up,
//           C is N/2 wide; silu(g) = g / (1 + expf(-g)).
//  partial  raw accumulators of K split gridDim.y into C[blockIdx.y][M][N]
//           (split-K; splitk_reduce_kernel sums the splits in order and
//           applies bias, epilogue and the final store)
//  swiglu_bf16  (bf16 GEMM only) swiglu, each product rounded to bf16 bits
//           (nearest-even) into C read as a uint16_t [M][N / 2] array: the
//           input of the next bf16 GEMM, which would round it on load anyway
enum class GemmStore { store, residual, swiglu, partial, swiglu_bf16 };

// Maps the dispatch-order workgroup id to a (tile_m, tile_n) pair: a band of
// consecutive tiles per XCD (dispatch is round-robin over XCDs), then
// group-of-8-rows ordering inside the band.
__device__ __forceinline__ void gemm_tile_of(int bid, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int total = tiles_m * tiles_n;
    int t = bid;
    if (total % kNumXcd == 0)
        t = (bid % kNumXcd) * (total / kNumXcd) + bid / kNumXcd;
    constexpr int G = 8;
    const int per_group = G * tiles_n;
    const int group = t / per_group;
    const int first_m = group * G;
    const int gsize = tiles_m - first_m < G ? tiles_m - first_m : G;
    const int in_group = t % per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// Buffer loads of the nk vector path: a descriptor over the rest of the operand from a uniform
// base (moved to each K tile's first element), and a 32-bit byte offset per lane. A load at or
// past num_records reads zeros, so an out-of-range chunk (a row past the edge, the K tail) takes
// offset kBufOob instead of a branch around its load; num_records is capped below kBufOob. The
// per-lane offsets stay below 2^31 because gemm_vec_ok sends larger operands to the scalar path.
constexpr uint32_t kBufOob = 0x7FFFFFF0u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t operand_rsrc(const void *base, int64_t bytes) {
    const uint32_t n = bytes <= 0 ? 0u : (bytes >= int64_t(kBufOob) ? kBufOob : static_cast<uint32_t>(bytes));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, n, 0x00020000); // raw, dword data
}
__device__ __forceinline__ f32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// TB: float, or uint16_t for bf16 weights in the nk layout, widened exactly to
// fp32 (bits << 16) while staged, so the products are fp32 x fp32 on the
// matrix core (the reference's rows 2..15 path for bf16 weights).
template <typename Shape, BLayout kB, bool kVec, typename Epi, GemmStore kStore = GemmStore::store,
          typename TB = float, ALayout kAL = ALayout::mk>
__global__ __launch_bounds__(Shape::kThreads) void gemm_f32_mfma_kernel(const float *__restrict__ A,
                                                                        const TB *__restrict__ B,
                                                                        const float *__restrict__ bias,
                                                                        float *__restrict__ C, int M, int N, int K,
                                                                        Epi epi) {
    constexpr int BM = Shape::BM, BN = Shape::BN, BK = Shape::BK, T_ = Shape::kThreads;
    constexpr int TM = Shape::TM, TN = Shape::TN, FM = Shape::FM, FN = Shape::FN;
    constexpr int LdK = Shape::LdK, LdN = Shape::LdN, LdM = Shape::LdM, CA = Shape::CA, CB = Shape::CB;
    constexpr int kA = kAL == ALayout::mk ? BM * LdK : BK * LdM;    // floats of the A stage
    constexpr int kStage = kA + (kB == BLayout::kn ? BK * LdN : BN * LdK);
    __shared__ __attribute__((aligned(16))) float lds[2 * kStage];
    // nk GEMMs (both operands k-contiguous) load through buffer descriptors, which freed the
    // registers their split-barrier pipeline needed (4096^3 nk: 1032 -> 977-980 us); the kn and
    // km layouts keep plain loads (buffer loads measured 1.3% slower on the kn config).
    constexpr bool kBufLoads = kB == BLayout::nk && kAL == ALayout::mk;

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    gemm_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid % kWaveSize, wave = tid / kWaveSize;
    const int wm = wave / Shape::WN, wn = wave % Shape::WN;
    const int l16 = lane % 16, grp = lane / 16;

    // ---- global -> register staging: chunk idx = tid + T i of a tile whose
    // rows hold BK (k-contiguous) or BN (kn-layout B) floats
    f32x4 ra[CA], rb[CB];
    static_assert(std::is_same_v<TB, float> || (std::is_same_v<TB, uint16_t> && kB == BLayout::nk),
                  "bf16 B is supported in the nk layout");
    // 4 consecutive k of one row: 16 bytes of fp32 or 8 bytes of bf16 (widened)
    auto load_rows_k = [&](const auto *src, int row0, int rows_total, int k0, f32x4 *dst, auto count) {
        using T = std::remove_cv_t<std::remove_pointer_t<decltype(src)>>;
        const T *base = src + int64_t(row0) * K + k0; // this tile's first element of the operand
        [[maybe_unused]] const auto rsrc =
            operand_rsrc(base, (int64_t(rows_total - row0) * K - k0) * int64_t(sizeof(T)));
#pragma unroll
        for (int i = 0; i < decltype(count)::value; ++i) {
            const int idx = tid + T_ * i;
            const int r = idx / (BK / 4), c = (idx % (BK / 4)) * 4;
            const int gr = row0 + r, gk = k0 + c;
            const bool in = gr < rows_total;
            if constexpr (kVec && !kBufLoads) {
                dst[i] = (in && gk < K) ? *reinterpret_cast<const f32x4 *>(src + int64_t(gr) * K + gk)
                                        : f32x4{0.f, 0.f, 0.f, 0.f};
            } else if constexpr (kVec) {
                const uint32_t off = (in && gk < K) ? uint32_t(r * K + c) * uint32_t(sizeof(T)) : kBufOob;
                if constexpr (std::is_same_v<T, float>) {
                    dst[i] = buf_load16(rsrc, off);
                } else {
                    using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
                    const u32x2 b = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, off, 0, 0));
                    dst[i] = f32x4{__builtin_bit_cast(float, b[0] << 16), __builtin_bit_cast(float, b[0] & 0xffff0000u),
                                   __builtin_bit_cast(float, b[1] << 16), __builtin_bit_cast(float, b[1] & 0xffff0000u)};
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (std::is_same_v<T, float>)
                        dst[i][j] = (in && gk + j < K) ? src[int64_t(gr) * K + gk + j] : 0.f;
                    else
                        dst[i][j] = (in && gk + j < K)
                                        ? __builtin_bit_cast(float, uint32_t(src[int64_t(gr) * K + gk + j]) << 16)
                                        : 0.f;
                }
            }
        }
    };
    auto load_b_kn = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int idx = tid + T_ * i;
            const int r = idx / (BN / 4), c = (idx % (BN / 4)) * 4;
            const int gk = k0 + r, gn = n0 + c;
            if constexpr (kVec) {
                rb[i] = (gk < K && gn < N) ? *reinterpret_cast<const f32x4 *>(B + int64_t(gk) * N + gn)
                                           : f32x4{0.f, 0.f, 0.f, 0.f};
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    rb[i][j] = (gk < K && gn + j < N) ? B[int64_t(gk) * N + gn + j] : 0.f;
            }
        }
    };
    auto load_a_km = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int idx = tid + T_ * i;
            const int r = idx / (BM / 4), c = (idx % (BM / 4)) * 4;
            const int gk = k0 + r, gm = m0 + c;
            if constexpr (kVec) {
                ra[i] = (gk < K && gm < M) ? *reinterpret_cast<const f32x4 *>(A + int64_t(gk) * M + gm)
                                           : f32x4{0.f, 0.f, 0.f, 0.f};
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    ra[i][j] = (gk < K && gm + j < M) ? A[int64_t(gk) * M + gm + j] : 0.f;
            }
        }
    };
    auto global_load = [&](int kt) {
        const int k0 = kt * BK;
        if constexpr (kAL == ALayout::mk)
            load_rows_k(A, m0, M, k0, ra, std::integral_constant<int, CA>{});
        else
            load_a_km(k0);
        if constexpr (kB == BLayout::kn)
            load_b_kn(k0);
        else
            load_rows_k(B, n0, N, k0, rb, std::integral_constant<int, CB>{});
    };
    auto lds_store = [&](int buf) {
        float *As = lds + buf * kStage;
        float *Bs = As + kA;
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int idx = tid + T_ * i;
            if constexpr (kAL == ALayout::mk)
                *reinterpret_cast<f32x4 *>(As + (idx / (BK / 4)) * LdK + (idx % (BK / 4)) * 4) = ra[i];
            else
                *reinterpret_cast<f32x4 *>(As + (idx / (BM / 4)) * LdM + (idx % (BM / 4)) * 4) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int idx = tid + T_ * i;
            if constexpr (kB == BLayout::kn)
                *reinterpret_cast<f32x4 *>(Bs + (idx / (BN / 4)) * LdN + (idx % (BN / 4)) * 4) = rb[i];
            else
                *reinterpret_cast<f32x4 *>(Bs + (idx / (BK / 4)) * LdK + (idx % (BK / 4)) * 4) = rb[i];
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
            acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // A K tile is one 16-k group = four MFMA steps; lane group g supplies k = 4g + e at step e.
    // Fragments are held per step ([set][e][tile]), so a step's values die with it.
    static_assert(BK == 16, "one 16-k group per K tile");
    float fa[2][4][FM], fb[2][4][FN];
    auto read_frags = [&](int buf, int p) {
        const float *As = lds + buf * kStage;
        const float *Bs = As + kA;
        const int kk = 4 * grp;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            if constexpr (kAL == ALayout::mk) {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(As + (wm * TM + i * 16 + l16) * LdK + kk);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    fa[p][e][i] = v[e];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    fa[p][e][i] = As[(kk + e) * LdM + wm * TM + i * 16 + l16];
            }
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            if constexpr (kB == BLayout::kn) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    fb[p][e][j] = Bs[(kk + e) * LdN + wn * TN + j * 16 + l16];
            } else {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(Bs + (wn * TN + j * 16 + l16) * LdK + kk);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    fb[p][e][j] = v[e];
            }
        }
    };
    auto mfma_step = [&](int p, int e) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[p][e][i], fb[p][e][j], acc[i][j], 0, 0, 0);
    };

    // K tiles of this workgroup: all of them, or split blockIdx.y's contiguous share
    const int ktiles_all = (K + BK - 1) / BK;
    const int per_split = (ktiles_all + gridDim.y - 1) / gridDim.y;
    const int kt_begin = blockIdx.y * per_split;
    const int kt_end = kt_begin + per_split < ktiles_all ? kt_begin + per_split : ktiles_all;
    // Tile kt from fragment set p: the next tile's global loads first, its LDS stores after two
    // MFMA steps, one barrier before the last step (every store of the next tile done, every
    // read of the stage it fills long done), and the next tile's fragments read into set p ^ 1
    // while the last step's MFMAs run, so no step waits on a barrier's LDS reads. Past the last
    // tile the next tile is a reload of this one, never used. (4096^3 kn: 1023-1027 us with a
    // barrier at the end of each tile, 986-987 us with this one.)
    auto k_tile = [&](int kt, auto p_t) {
        constexpr int p = decltype(p_t)::value;
        const int buf = (kt - kt_begin) & 1;
        global_load(kt + 1 < kt_end ? kt + 1 : kt);
        __builtin_amdgcn_sched_barrier(0);
        mfma_step(p, 0);
        mfma_step(p, 1);
        __builtin_amdgcn_sched_barrier(0);
        lds_store(buf ^ 1);
        __builtin_amdgcn_sched_barrier(0);
        mfma_step(p, 2);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        read_frags(buf ^ 1, p ^ 1);
        mfma_step(p, 3);
        __builtin_amdgcn_sched_barrier(0);
    };
    // GemmBig in the nk layout keeps one barrier at the end of each tile: with two fragment sets
    // its load addresses spilled to scratch inside the K loop.
    constexpr bool kSplitBarrier = true;
    if (kSplitBarrier && kt_begin < kt_end) {
        global_load(kt_begin);
        lds_store(0);
        __syncthreads();
        read_frags(0, 0);
        int kt = kt_begin;
        for (; kt + 1 < kt_end; kt += 2) { // two tiles per trip: each fragment set keeps its registers
            k_tile(kt, std::integral_constant<int, 0>{});
            k_tile(kt + 1, std::integral_constant<int, 1>{});
        }
        if (kt < kt_end)
            k_tile(kt, std::integral_constant<int, 0>{});
    } else if (kt_begin < kt_end) {
        global_load(kt_begin);
        lds_store(0);
        __syncthreads();
        for (int kt = kt_begin; kt < kt_end; ++kt) {
            const int buf = (kt - kt_begin) & 1;
            if (kt + 1 < kt_end)
                global_load(kt + 1);
            read_frags(buf, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                mfma_step(0, e);
            if (kt + 1 < kt_end)
                lds_store(buf ^ 1);
            __syncthreads();
        }
    }
    if constexpr (kStore == GemmStore::partial)
        C += int64_t(blockIdx.y) * M * N;

    // ---- epilogue: accumulator register r of a 16 x 16 tile holds row
    // 4 * grp + r, column l16. A store counts in vmcnt like a load, so a load issued after stores
    // waits for them too: every bias value is loaded before the first store, and a column group's
    // residual C values before its stores (one drain per group, not one per element).
    float bv[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int col = n0 + wn * TN + j * 16 + l16;
        bv[j] = (bias != nullptr && col < N && kStore != GemmStore::partial) ? bias[col] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int col = n0 + wn * TN + j * 16 + l16;
        float prev[FM][4];
        if constexpr (kStore == GemmStore::residual) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + wm * TM + i * 16 + 4 * grp + r;
                    prev[i][r] = (row < M && col < N) ? C[int64_t(row) * N + col] : 0.f;
                }
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm * TM + i * 16 + 4 * grp + r;
                if constexpr (kStore == GemmStore::partial) {
                    if (row < M && col < N)
                        C[int64_t(row) * N + col] = acc[i][j][r];
                    continue;
                }
                const float v = epi(acc[i][j][r] + bv[j]);
                if constexpr (kStore == GemmStore::swiglu) {
                    const float partner = __shfl_xor(v, 1); // lane l ^ 1 holds column col ^ 1
                    if ((l16 & 1) == 0 && row < M && col + 1 < N)
                        C[int64_t(row) * (N / 2) + col / 2] = v / (1.f + expf(-v)) * partner;
                } else if constexpr (kStore == GemmStore::residual) {
                    if (row < M && col < N)
                        C[int64_t(row) * N + col] = prev[i][r] + v;
                } else {
                    if (row < M && col < N)
                        C[int64_t(row) * N + col] = v;
                }
            }
        }
    }
}

// Split-K epilogue: C = epi(sum_s part[s] + bias) (store) or C += ... (residual),
// the splits summed in order s = 0, 1, ...; one thread per 4 columns of a row.
template <typename Epi, GemmStore kStore>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ part, int splits,
                                                            const float *__restrict__ bias, float *__restrict__ C,
                                                            int M, int N, Epi epi) {
    static_assert(kStore == GemmStore::store || kStore == GemmStore::residual, "split-K stores or accumulates");
    const int64_t mn = int64_t(M) * N;
    OPWORKS_GRID_LOOP(i4, mn / 4) {
        const int64_t i = 4 * i4;
        f32x4 sum = *reinterpret_cast<const f32x4 *>(part + i);
        for (int sp = 1; sp < splits; ++sp) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(part + sp * mn + i);
            sum = sum + v;
        }
        const int col = static_cast<int>(i % N);
        f32x4 out;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            out[j] = epi(sum[j] + (bias ? bias[col + j] : 0.f));
        f32x4 *dst = reinterpret_cast<f32x4 *>(C + i);
        if constexpr (kStore == GemmStore::residual)
            *dst = *dst + out;
        else
            *dst = out;
    }
}

// Splits that bring a launch of `tiles` output tiles to about `target`
// workgroups: a power of two <= 8 with at least 8 K tiles per split (1 = no split).
inline int splitk_factor(int tiles, int ktiles, int target) {
    int s = 1;
    while (s < 8 && tiles * s * 2 <= target && ktiles / (s * 2) >= 8)
        s *= 2;
    return s;
}

// 16-byte loads need aligned operands and 4-element runs along each contiguous dimension.
// The nk vector path's buffer offsets reach 256 rows of a k-contiguous operand from a tile's
// base, in bytes below 2^31 (kBufOob).
inline bool gemm_vec_ok(const void *a, const void *b, int M, int K, int N, ALayout a_layout, BLayout b_layout) {
    const bool aligned = aligned16(a) && aligned16(b);
    const bool a_runs = a_layout == ALayout::mk ? K % 4 == 0 : M % 4 == 0;
    const bool b_runs = b_layout == BLayout::nk ? K % 4 == 0 : N % 4 == 0;
    const bool buffer_loads = a_layout == ALayout::mk && b_layout == BLayout::nk;
    const bool fits = !buffer_loads || int64_t(256) * K * 4 < int64_t(kBufOob);
    return aligned && a_runs && b_runs && fits;
}

template <typename Shape, BLayout kB, typename Epi, GemmStore kStore, typename TB = float,
          ALayout kAL = ALayout::mk>
void gemm_f32_launch_shape(const float *A, const TB *B, const float *bias, float *C, int M, int N, int K, Epi epi,
                           hipStream_t stream, int splits) {
    const int tiles = static_cast<int>(blocks_for64(M, Shape::BM) * blocks_for64(N, Shape::BN));
    const dim3 grid(tiles, splits);
    if (gemm_vec_ok(A, B, M, K, N, kAL, kB))
        launch_async(stream, gemm_f32_mfma_kernel<Shape, kB, true, Epi, kStore, TB, kAL>, grid, Shape::kThreads, A, B,
                     bias, C, M, N, K, epi);
    else
        launch_async(stream, gemm_f32_mfma_kernel<Shape, kB, false, Epi, kStore, TB, kAL>, grid, Shape::kThreads, A,
                     B, bias, C, M, N, K, epi);
}

} // namespace opworks::detail

#include "gemm_x6.hpp"

namespace opworks::detail {

// The fp32 products that the bf16x6 kernel takes: fp32 operands, A row-major, 16-byte aligned,
// K a multiple of 8 (and N of 4 for a kn-layout B), and enough work to fill its 128 x 256 tiles
// (at 4096^3 nk: 1003 -> 673 us, 1.30 of the fp32 MFMA peak; 512 x 16384 x 2048: 279 -> 179 us), for plain
// and SwiGLU stores. Callers that need the fp32 MFMA kernels' summation pass allow_x6 = false; the
// split-K form never takes it. The Llama runtime, held to the oracle's logits at NRMSE 1e-5, takes
// it for the gate/up projection only: config 5's worst step read 9.27e-6 on fp32 MFMAs, 9.94e-6 with
// gate/up on bf16x6 (fp32 TTFT 9.57 -> 8.10 ms), 1.05e-5 with every projection on it.
// OPWORKS_GEMM_X6=0 in the environment keeps every product on the fp32 MFMA kernels.
inline bool gemm_x6_enabled() {
    static const bool enabled = [] {
        const char *v = std::getenv("OPWORKS_GEMM_X6");
        return !(v && v[0] == '0' && v[1] == '\0');
    }();
    return enabled;
}
template <BLayout kB, GemmStore kStore, typename TB, ALayout kAL>
inline bool gemm_use_x6(const float *A, const TB *B, int M, int N, int K) {
    if constexpr (std::is_same_v<TB, float> && kAL == ALayout::mk &&
                  (kStore == GemmStore::store || kStore == GemmStore::swiglu)) {
        return M >= 16 && int64_t(M) * N * K >= (int64_t(1) << 26) && gemm_x6_ok<kB>(A, B, N, K) &&
               gemm_x6_enabled();
    } else {
        return false;
    }
}

// Enqueues C[M][N] = epi(A[M][K] B + bias) (written per kStore). K == 0 writes epi(bias or 0).
// When K is not split: GemmBig when its tiles alone cover every CU, else GemmMid when its
// 256 x 128 tiles do (the prefill gate/up projection at 512 rows: 280 -> 262 us against
// GemmSmall); otherwise, and for split-K partials, GemmSmall.
template <BLayout kB, typename Epi, GemmStore kStore = GemmStore::store, typename TB = float,
          ALayout kAL = ALayout::mk>
void gemm_f32_launch(const float *A, const TB *B, const float *bias, float *C, int M, int N, int K, Epi epi,
                     hipStream_t stream, int splits = 1, bool allow_x6 = true) {
    require(kStore != GemmStore::swiglu || N % 2 == 0, "swiglu epilogue needs an even number of columns");
    if constexpr (std::is_same_v<TB, float> && kAL == ALayout::mk &&
                  (kStore == GemmStore::store || kStore == GemmStore::swiglu)) {
        if (allow_x6 && gemm_use_x6<kB, kStore, TB, kAL>(A, B, M, N, K)) {
            gemm_x6_launch<kB, Epi, kStore>(A, B, bias, C, M, N, K, epi, stream, splits);
            return;
        }
    }
    const int64_t big_tiles = blocks_for64(M, GemmBig::BM) * blocks_for64(N, GemmBig::BN);
    const int64_t mid_tiles = blocks_for64(M, GemmMid::BM) * blocks_for64(N, GemmMid::BN);
    if (splits == 1 && big_tiles >= 256)
        gemm_f32_launch_shape<GemmBig, kB, Epi, kStore, TB, kAL>(A, B, bias, C, M, N, K, epi, stream, splits);
    else if (splits == 1 && mid_tiles >= 256)
        gemm_f32_launch_shape<GemmMid, kB, Epi, kStore, TB, kAL>(A, B, bias, C, M, N, K, epi, stream, splits);
    else
        gemm_f32_launch_shape<GemmSmall, kB, Epi, kStore, TB, kAL>(A, B, bias, C, M, N, K, epi, stream, splits);
}

// Floats of split-K workspace any launch planned by splitk_factor(tiles, ., 512) needs.
constexpr int64_t kSplitKWorkspaceF32 = int64_t(512) * GemmSmall::BM * GemmSmall::BN;

// C (store or residual) = epi(A B + bias) with K split across `splits`
// workgroup rows when the output alone has too few tiles to fill the GPU;
// the partial tiles go to `ws` (splits * M * N floats) and are summed in order.
// `reduce` (optional): when K is split, called as reduce(ws, splits) in place of the reduction
// kernel, so a caller can fuse what follows the store into it. Returns true when K was split.
template <BLayout kB, typename Epi, GemmStore kStore, typename TB = float, typename Reduce = std::nullptr_t>
bool gemm_f32_launch_splitk(const float *A, const TB *B, const float *bias, float *C, int M, int N, int K, Epi epi,
                            float *ws, int64_t ws_floats, hipStream_t stream, Reduce reduce = nullptr) {
    // Partials on GemmMid tiles up to 256 workgroups when M fills its 256-row tiles and that splits
    // K at all, else on GemmSmall tiles up to 512 (prefill at 512 rows: qkv 86.2 -> 81.8 us, down
    // 152.5 -> 148.4 us, o_proj unchanged). Either plan needs at most 256 * 256 * 128 =
    // 512 * 128 * 128 floats.
    const int ktiles = static_cast<int>(blocks_for64(K, kGemmBK));
    const int mid_splits =
        M >= GemmMid::BM
            ? splitk_factor(static_cast<int>(blocks_for64(M, GemmMid::BM) * blocks_for64(N, GemmMid::BN)), ktiles, 256)
            : 1;
    const int splits = mid_splits > 1 ? mid_splits
                                      : splitk_factor(static_cast<int>(blocks_for64(M, GemmSmall::BM) *
                                                                       blocks_for64(N, GemmSmall::BN)),
                                                      ktiles, 512);
    if (splits == 1 || N % 4 != 0 || !ws || int64_t(splits) * M * N > ws_floats || !aligned16(C) ||
        (bias && !aligned16(bias))) {
        gemm_f32_launch<kB, Epi, kStore, TB>(A, B, bias, C, M, N, K, epi, stream, 1, false); // fp32 MFMA
        return false;
    }
    if (mid_splits > 1)
        gemm_f32_launch_shape<GemmMid, kB, IdentityEpilogue, GemmStore::partial, TB>(
            A, B, nullptr, ws, M, N, K, IdentityEpilogue{}, stream, splits);
    else
        gemm_f32_launch_shape<GemmSmall, kB, IdentityEpilogue, GemmStore::partial, TB>(
            A, B, nullptr, ws, M, N, K, IdentityEpilogue{}, stream, splits);
    if constexpr (std::is_same_v<Reduce, std::nullptr_t>)
        launch_async(stream, splitk_reduce_kernel<Epi, kStore>, stream_grid(int64_t(M) * N / 4), 256, ws, splits, bias,
                     C, M, N, epi);
    else
        reduce(ws, splits);
    return true;
}

} // namespace opworks::detail

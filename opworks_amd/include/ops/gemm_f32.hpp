#pragma once

// fp32 GEMM on the CDNA4 matrix cores: C[m][n] = epi(sum_k A[m][k] * B(k, n) + bias[n]).
//
// B comes in two layouts:
//  * BLayout::kn — B[k][n], n contiguous: ops::mat_mul (reference
//    include/ops/matmul.cuh:11-91, where the reduction dim is called N);
//  * BLayout::nk — B[n][k], k contiguous: ops::linear's Y = X W^T with HF
//    [out, in] weights (reference include/ops/linear.cuh:18-73).
//
// Kernel shape (gfx950):
//  * workgroup tile 128 x 128, K tile 32, 256 threads = 4 waves in 2 x 2,
//    each wave owns a 64 x 64 block = 2 x 2 v_mfma_f32_32x32x2_f32 tiles
//    (64 accumulator registers);
//  * operands are staged through LDS, double buffered, one barrier per K tile;
//    the next tile's global loads are issued before the current tile's MFMAs;
//  * K is permuted per lane half: inside a K tile, MFMA step s of lane half h
//    uses k = 8*(s/4) + 4*h + s%4. A product sum does not depend on the
//    order of k, and this order lets a k-contiguous operand (A, and B in the
//    nk layout) keep its global layout in LDS (rows padded to 36 floats) and
//    deliver four MFMA steps with one ds_read_b128; the kn-layout B is read
//    one float per step from rows padded to 136 floats, which keeps the two
//    lane halves (4 rows apart) on disjoint banks;
//  * workgroup ids are remapped so each XCD (its own L2) works on a
//    contiguous band of tiles, then grouped 8 tile-rows at a time.
// Accumulation is fp32 on the matrix core; the result differs from a
// k-ascending fmaf chain only by summation order.

#include <cstdint>

#include "../core/hip_utils.hpp"
#include "elementwise.hpp"

namespace opworks::detail {

enum class BLayout { kn, nk };

using f32x16 = float __attribute__((ext_vector_type(16)));

constexpr int kGemmBM = 128, kGemmBN = 128, kGemmBK = 32;
constexpr int kGemmThreads = 256;
constexpr int kGemmLdK = kGemmBK + 4;  // padded row of a k-contiguous tile
constexpr int kGemmLdN = kGemmBN + 8;  // padded row of the kn-layout B tile
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
enum class GemmStore { store, residual, swiglu, partial };

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

template <BLayout kB, bool kVec> struct GemmF32Tiles {
    // LDS stage sizes in floats
    static constexpr int kA = kGemmBM * kGemmLdK;
    static constexpr int kB_ = kB == BLayout::kn ? kGemmBK * kGemmLdN : kGemmBN * kGemmLdK;
    static constexpr int kStage = kA + kB_;
};

template <BLayout kB, bool kVec, typename Epi, GemmStore kStore = GemmStore::store>
__global__ __launch_bounds__(kGemmThreads) void gemm_f32_mfma_kernel(const float *__restrict__ A,
                                                                     const float *__restrict__ B,
                                                                     const float *__restrict__ bias,
                                                                     float *__restrict__ C, int M, int N, int K,
                                                                     Epi epi) {
    using Tiles = GemmF32Tiles<kB, kVec>;
    __shared__ __attribute__((aligned(16))) float lds[2 * Tiles::kStage];

    const int tiles_m = (M + kGemmBM - 1) / kGemmBM, tiles_n = (N + kGemmBN - 1) / kGemmBN;
    int tm, tn;
    gemm_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * kGemmBM, n0 = tn * kGemmBN;
    const int tid = threadIdx.x, lane = tid % kWaveSize, wave = tid / kWaveSize;
    const int wm = wave / 2, wn = wave % 2;
    const int l32 = lane % 32, half = lane / 32;

    // ---- global -> register staging (4 x 16 B per operand per thread)
    f32x4 ra[4], rb[4];
    auto load_rows_k = [&](const float *src, int row0, int rows_total, int k0, f32x4 *dst) {
        // tile of 128 rows x 32 k, k contiguous; thread covers float4 idx = tid + 256 i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + kGemmThreads * i;
            const int r = idx / 8, c = (idx % 8) * 4;
            const int gr = row0 + r, gk = k0 + c;
            if constexpr (kVec) {
                dst[i] = (gr < rows_total && gk < K) ? *reinterpret_cast<const f32x4 *>(src + int64_t(gr) * K + gk)
                                                     : f32x4{0.f, 0.f, 0.f, 0.f};
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    dst[i][j] = (gr < rows_total && gk + j < K) ? src[int64_t(gr) * K + gk + j] : 0.f;
            }
        }
    };
    auto load_b_kn = [&](int k0) {
        // tile of 32 k x 128 n, n contiguous
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + kGemmThreads * i;
            const int r = idx / 32, c = (idx % 32) * 4;
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
    auto global_load = [&](int kt) {
        const int k0 = kt * kGemmBK;
        load_rows_k(A, m0, M, k0, ra);
        if constexpr (kB == BLayout::kn)
            load_b_kn(k0);
        else
            load_rows_k(B, n0, N, k0, rb);
    };
    auto lds_store = [&](int buf) {
        float *As = lds + buf * Tiles::kStage;
        float *Bs = As + Tiles::kA;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + kGemmThreads * i;
            *reinterpret_cast<f32x4 *>(As + (idx / 8) * kGemmLdK + (idx % 8) * 4) = ra[i];
            if constexpr (kB == BLayout::kn)
                *reinterpret_cast<f32x4 *>(Bs + (idx / 32) * kGemmLdN + (idx % 32) * 4) = rb[i];
            else
                *reinterpret_cast<f32x4 *>(Bs + (idx / 8) * kGemmLdK + (idx % 8) * 4) = rb[i];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[i][j] = f32x16{};

    auto compute = [&](int buf) {
        const float *As = lds + buf * Tiles::kStage;
        const float *Bs = As + Tiles::kA;
#pragma unroll
        for (int g = 0; g < kGemmBK / 8; ++g) {
            const int kk = 8 * g + 4 * half;
            f32x4 a[2], b[2];
#pragma unroll
            for (int bm = 0; bm < 2; ++bm)
                a[bm] = *reinterpret_cast<const f32x4 *>(As + (wm * 64 + bm * 32 + l32) * kGemmLdK + kk);
#pragma unroll
            for (int bn = 0; bn < 2; ++bn) {
                if constexpr (kB == BLayout::kn) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        b[bn][j] = Bs[(kk + j) * kGemmLdN + wn * 64 + bn * 32 + l32];
                } else {
                    b[bn] = *reinterpret_cast<const f32x4 *>(Bs + (wn * 64 + bn * 32 + l32) * kGemmLdK + kk);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int bm = 0; bm < 2; ++bm)
#pragma unroll
                    for (int bn = 0; bn < 2; ++bn)
                        acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[bm][j], b[bn][j], acc[bm][bn], 0, 0, 0);
        }
    };

    // K tiles of this workgroup: all of them, or split blockIdx.y's contiguous share
    const int ktiles_all = (K + kGemmBK - 1) / kGemmBK;
    const int per_split = (ktiles_all + gridDim.y - 1) / gridDim.y;
    const int kt_begin = blockIdx.y * per_split;
    const int kt_end = kt_begin + per_split < ktiles_all ? kt_begin + per_split : ktiles_all;
    if (kt_begin < kt_end) {
        global_load(kt_begin);
        lds_store(0);
        __syncthreads();
        for (int kt = kt_begin; kt < kt_end; ++kt) {
            const int buf = (kt - kt_begin) & 1;
            if (kt + 1 < kt_end)
                global_load(kt + 1);
            compute(buf);
            if (kt + 1 < kt_end)
                lds_store(buf ^ 1);
            __syncthreads();
        }
    }
    if constexpr (kStore == GemmStore::partial)
        C += int64_t(blockIdx.y) * M * N;

    // ---- epilogue: accumulator register r of a 32x32 tile holds
    // row 8*(r/4) + 4*half + r%4, column l32.
#pragma unroll
    for (int bn = 0; bn < 2; ++bn) {
        const int col = n0 + wn * 64 + bn * 32 + l32;
        const float bv = (bias != nullptr && col < N && kStore != GemmStore::partial) ? bias[col] : 0.f;
#pragma unroll
        for (int bm = 0; bm < 2; ++bm) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * 64 + bm * 32 + 8 * (r / 4) + 4 * half + (r % 4);
                if constexpr (kStore == GemmStore::partial) {
                    if (row < M && col < N)
                        C[int64_t(row) * N + col] = acc[bm][bn][r];
                    continue;
                }
                const float v = epi(acc[bm][bn][r] + bv);
                if constexpr (kStore == GemmStore::swiglu) {
                    const float partner = __shfl_xor(v, 1); // lane l ^ 1 holds column col ^ 1
                    if ((l32 & 1) == 0 && row < M && col + 1 < N)
                        C[int64_t(row) * (N / 2) + col / 2] = v / (1.f + expf(-v)) * partner;
                } else if constexpr (kStore == GemmStore::residual) {
                    if (row < M && col < N)
                        C[int64_t(row) * N + col] += v;
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

inline bool gemm_vec_ok(const void *a, const void *b, int K, int N, BLayout layout) {
    const bool aligned = aligned16(a) && aligned16(b);
    return aligned && K % 4 == 0 && (layout == BLayout::nk || N % 4 == 0);
}

// Enqueues C[M][N] = epi(A[M][K] B + bias) (written per kStore). K == 0 writes epi(bias or 0).
template <BLayout kB, typename Epi, GemmStore kStore = GemmStore::store>
void gemm_f32_launch(const float *A, const float *B, const float *bias, float *C, int M, int N, int K, Epi epi,
                     hipStream_t stream, int splits = 1) {
    require(kStore != GemmStore::swiglu || N % 2 == 0, "swiglu epilogue needs an even number of columns");
    const int tiles = static_cast<int>(blocks_for64(M, kGemmBM) * blocks_for64(N, kGemmBN));
    const dim3 grid(tiles, splits);
    if (gemm_vec_ok(A, B, K, N, kB))
        launch_async(stream, gemm_f32_mfma_kernel<kB, true, Epi, kStore>, grid, kGemmThreads, A, B, bias, C, M, N, K,
                     epi);
    else
        launch_async(stream, gemm_f32_mfma_kernel<kB, false, Epi, kStore>, grid, kGemmThreads, A, B, bias, C, M, N,
                     K, epi);
}

// Floats of split-K workspace any launch planned by splitk_factor(tiles, ., 512) needs.
constexpr int64_t kSplitKWorkspaceF32 = int64_t(512) * kGemmBM * kGemmBN;

// C (store or residual) = epi(A B + bias) with K split across `splits`
// workgroup rows when the output alone has too few tiles to fill the GPU;
// the partial tiles go to `ws` (splits * M * N floats) and are summed in order.
template <BLayout kB, typename Epi, GemmStore kStore>
void gemm_f32_launch_splitk(const float *A, const float *B, const float *bias, float *C, int M, int N, int K, Epi epi,
                            float *ws, int64_t ws_floats, hipStream_t stream) {
    const int tiles = static_cast<int>(blocks_for64(M, kGemmBM) * blocks_for64(N, kGemmBN));
    const int splits = splitk_factor(tiles, static_cast<int>(blocks_for64(K, kGemmBK)), 512);
    if (splits == 1 || N % 4 != 0 || !ws || int64_t(splits) * M * N > ws_floats || !aligned16(C) ||
        (bias && !aligned16(bias))) {
        gemm_f32_launch<kB, Epi, kStore>(A, B, bias, C, M, N, K, epi, stream);
        return;
    }
    gemm_f32_launch<kB, IdentityEpilogue, GemmStore::partial>(A, B, nullptr, ws, M, N, K, IdentityEpilogue{}, stream,
                                                              splits);
    launch_async(stream, splitk_reduce_kernel<Epi, kStore>, stream_grid(int64_t(M) * N / 4), 256, ws, splits, bias, C,
                 M, N, epi);
}

} // namespace opworks::detail

#pragma once

// bf16 GEMM with fp32 accumulation on the CDNA4 matrix cores:
//   C[m][n] = epi(sum_k bf16(A[m][k]) * W[n][k] + bias[n]),   W bf16 [N][K] (HF layout).
// A is either fp32 (rounded to bf16, nearest-even, while it is staged into LDS —
// the reference's ops::linear_mma_bf16 contract, include/ops/linear_mma.cuh:24-93)
// or already bf16.
//
// Kernel shape (gfx950):
//  * workgroup tile 256 x 256, K tile 32, 512 threads = 8 waves in 2 x 4; each
//    wave owns 128 x 64 = 4 x 2 v_mfma_f32_32x32x16_bf16 tiles (128
//    accumulator registers);
//  * an MFMA operand is 8 consecutive k of one row per lane, so both operands
//    keep their k-contiguous global layout in LDS; rows are padded from 64 to
//    80 bytes, which puts the 16-byte reads of 16 consecutive rows on disjoint
//    bank groups;
//  * LDS double buffered, next tile's global loads issued before the current
//    tile's MFMAs, one barrier per K tile; same XCD-banded tile order as the
//    fp32 kernel.

#include <cstdint>

#include "../core/bf16.hpp"
#include "../core/hip_utils.hpp"
#include "elementwise.hpp"
#include "gemm_f32.hpp"

namespace opworks::detail {

using bf16x8 = __bf16 __attribute__((ext_vector_type(8)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

constexpr int kBfBM = 256, kBfBN = 256, kBfBK = 32;
constexpr int kBfThreads = 512;
constexpr int kBfLd = kBfBK + 8; // bf16 elements per padded LDS row (80 bytes)

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return static_cast<uint32_t>(float_to_bf16_rne(lo)) | (static_cast<uint32_t>(float_to_bf16_rne(hi)) << 16);
}

template <typename TA, bool kVec, typename Epi, GemmStore kStore = GemmStore::store>
__global__ __launch_bounds__(kBfThreads) void gemm_bf16_mfma_kernel(const TA *__restrict__ A,
                                                                    const uint16_t *__restrict__ W,
                                                                    const float *__restrict__ bias,
                                                                    float *__restrict__ C, int M, int N, int K,
                                                                    Epi epi) {
    static_assert(std::is_same_v<TA, float> || std::is_same_v<TA, uint16_t>, "A is fp32 or bf16 bits");
    constexpr int kStage = (kBfBM + kBfBN) * kBfLd; // uint16 elements per stage
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStage];

    const int tiles_m = (M + kBfBM - 1) / kBfBM, tiles_n = (N + kBfBN - 1) / kBfBN;
    int tm, tn;
    gemm_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * kBfBM, n0 = tn * kBfBN;
    const int tid = threadIdx.x, lane = tid % kWaveSize, wave = tid / kWaveSize;
    const int wm = wave / 4, wn = wave % 4; // 2 x 4 waves
    const int l32 = lane % 32, half = lane / 32;

    // Staging: each operand tile is 256 rows x 32 k = 1024 chunks of 8 k; 2 chunks per thread.
    u32x4 ra[2], rb[2];
    auto load_chunk_bf16 = [&](const uint16_t *src, int row, int rows_total, int k) -> u32x4 {
        if constexpr (kVec) {
            return (row < rows_total && k < K) ? *reinterpret_cast<const u32x4 *>(src + int64_t(row) * K + k)
                                               : u32x4{0u, 0u, 0u, 0u};
        } else {
            uint16_t e[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                e[j] = (row < rows_total && k + j < K) ? src[int64_t(row) * K + k + j] : uint16_t(0);
            return u32x4{e[0] | (uint32_t(e[1]) << 16), e[2] | (uint32_t(e[3]) << 16), e[4] | (uint32_t(e[5]) << 16),
                         e[6] | (uint32_t(e[7]) << 16)};
        }
    };
    auto load_chunk_f32 = [&](const float *src, int row, int k) -> u32x4 {
        float e[8];
        if constexpr (kVec) {
            if (row < M && k < K) {
                const f32x4 lo = *reinterpret_cast<const f32x4 *>(src + int64_t(row) * K + k);
                const f32x4 hi = *reinterpret_cast<const f32x4 *>(src + int64_t(row) * K + k + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    e[j] = lo[j];
                    e[4 + j] = hi[j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    e[j] = 0.f;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                e[j] = (row < M && k + j < K) ? src[int64_t(row) * K + k + j] : 0.f;
        }
        return u32x4{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3]), pack_bf16x2(e[4], e[5]),
                     pack_bf16x2(e[6], e[7])};
    };
    auto global_load = [&](int kt) {
        const int k0 = kt * kBfBK;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + kBfThreads * i;
            const int r = idx / 4, c = (idx % 4) * 8;
            if constexpr (std::is_same_v<TA, float>)
                ra[i] = load_chunk_f32(A, m0 + r, k0 + c);
            else
                ra[i] = load_chunk_bf16(A, m0 + r, M, k0 + c);
            rb[i] = load_chunk_bf16(W, n0 + r, N, k0 + c);
        }
    };
    auto lds_store = [&](int buf) {
        uint16_t *As = lds + buf * kStage;
        uint16_t *Bs = As + kBfBM * kBfLd;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + kBfThreads * i;
            const int off = (idx / 4) * kBfLd + (idx % 4) * 8;
            *reinterpret_cast<u32x4 *>(As + off) = ra[i];
            *reinterpret_cast<u32x4 *>(Bs + off) = rb[i];
        }
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[i][j] = f32x16{};

    auto compute = [&](int buf) {
        const uint16_t *As = lds + buf * kStage;
        const uint16_t *Bs = As + kBfBM * kBfLd;
#pragma unroll
        for (int s = 0; s < kBfBK / 16; ++s) {
            const int kk = 16 * s + 8 * half;
            bf16x8 a[4], b[2];
#pragma unroll
            for (int bm = 0; bm < 4; ++bm)
                a[bm] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(
                                                        As + (wm * 128 + bm * 32 + l32) * kBfLd + kk));
#pragma unroll
            for (int bn = 0; bn < 2; ++bn)
                b[bn] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(
                                                        Bs + (wn * 64 + bn * 32 + l32) * kBfLd + kk));
#pragma unroll
            for (int bm = 0; bm < 4; ++bm)
#pragma unroll
                for (int bn = 0; bn < 2; ++bn)
                    acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[bm], b[bn], acc[bm][bn], 0, 0, 0);
        }
    };

    // K tiles of this workgroup: all of them, or split blockIdx.y's contiguous share
    const int ktiles_all = (K + kBfBK - 1) / kBfBK;
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

#pragma unroll
    for (int bn = 0; bn < 2; ++bn) {
        const int col = n0 + wn * 64 + bn * 32 + l32;
        const float bv = (bias != nullptr && col < N && kStore != GemmStore::partial) ? bias[col] : 0.f;
#pragma unroll
        for (int bm = 0; bm < 4; ++bm) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * 128 + bm * 32 + 8 * (r / 4) + 4 * half + (r % 4);
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

// C written per kStore (see GemmStore): store, += (residual), or SwiGLU of
// interleaved (gate, up) column pairs into C[M][N / 2].
template <typename TA, typename Epi, GemmStore kStore = GemmStore::store>
void gemm_bf16_launch(const TA *A, const uint16_t *W, const float *bias, float *C, int M, int N, int K, Epi epi,
                      hipStream_t stream, int splits = 1) {
    require(kStore != GemmStore::swiglu || N % 2 == 0, "swiglu epilogue needs an even number of columns");
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

// Floats of split-K workspace any launch planned by splitk_factor(tiles, ., 256) needs.
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

} // namespace opworks::detail

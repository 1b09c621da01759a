#pragma once

// ops::transpose and ops::copy — the kernels behind TransformBuilder (the
// reference's builder carries rows, cols and the operation, include/builders/
// transform.cuh:7-30, and ships no kernel).
//
//   transpose: out[c][r] = in[r][c] for a row-major rows x cols input, so out
//              is cols x rows;
//   reshape, copy: out[i] = in[i] for i < rows * cols (a row-major reshape
//              keeps the element order, so both are a copy).
//
// Transpose on gfx950: one 512-lane workgroup per 128 x 128 tile staged in
// LDS (66 KB) with one word of padding per row (the column reads of the store
// phase fall on distinct banks). When both pointers are 16-byte aligned and
// rows and cols are multiples of 4, each lane moves 16-byte packs on both
// sides: a tile row is read by 32 lanes as 512 contiguous bytes and an output
// row written the same way. Measured on 8192 x 8192 against 64 x 64 tiles of
// 256 lanes: 5.7 vs 4.3 TB/s (a plain copy of the same bytes runs at 6.5).
// Otherwise every element goes through a bounds-checked scalar path. Tile
// rows past 65535 loop over blockIdx.y. Bytes are moved, never computed on,
// so results are bit-exact.

#include <cstdint>

#include "../core/hip_utils.hpp"
#include "elementwise.hpp" // f32x4, aligned16, map

namespace opworks::detail {

constexpr int kTransposeTile = 128;
constexpr int kTransposeThreads = 512;

template <bool kVec>
__global__ __launch_bounds__(kTransposeThreads) void transpose_kernel(const float *__restrict__ in,
                                                                      float *__restrict__ out, int rows, int cols) {
    constexpr int T = kTransposeTile;
    constexpr int kLanesPerRow = T / 4;                            // 16-byte packs per tile row
    constexpr int kRowsPerPass = kTransposeThreads / kLanesPerRow; // tile rows one pass covers
    __shared__ float tile[T][T + 1];
    const int tid = threadIdx.x, ty = tid / kLanesPerRow, tx = tid % kLanesPerRow;
    const int64_t c0 = int64_t(blockIdx.x) * T;
    const int tiles_r = (rows + T - 1) / T;
    for (int tr = blockIdx.y; tr < tiles_r; tr += gridDim.y) {
        const int64_t r0 = int64_t(tr) * T;
        if constexpr (kVec) {
            f32x4 v[T / kRowsPerPass];
#pragma unroll
            for (int k = 0; k < T / kRowsPerPass; ++k) {
                const int r = ty + kRowsPerPass * k;
                v[k] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (r0 + r < rows && c0 + 4 * tx < cols)
                    v[k] = *reinterpret_cast<const f32x4 *>(in + (r0 + r) * cols + c0 + 4 * tx);
            }
#pragma unroll
            for (int k = 0; k < T / kRowsPerPass; ++k)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    tile[ty + kRowsPerPass * k][4 * tx + e] = v[k][e];
        } else {
#pragma unroll 4
            for (int k = 0; k < T * T / kTransposeThreads; ++k) {
                const int idx = tid + kTransposeThreads * k, r = idx / T, c = idx % T;
                tile[r][c] = (r0 + r < rows && c0 + c < cols) ? in[(r0 + r) * cols + c0 + c] : 0.f;
            }
        }
        __syncthreads();
        if constexpr (kVec) {
#pragma unroll
            for (int k = 0; k < T / kRowsPerPass; ++k) {
                const int oc = ty + kRowsPerPass * k; // output row c0 + oc
                if (c0 + oc < cols && r0 + 4 * tx < rows) {
                    const f32x4 v = {tile[4 * tx][oc], tile[4 * tx + 1][oc], tile[4 * tx + 2][oc],
                                     tile[4 * tx + 3][oc]};
                    *reinterpret_cast<f32x4 *>(out + (c0 + oc) * rows + r0 + 4 * tx) = v;
                }
            }
        } else {
#pragma unroll 4
            for (int k = 0; k < T * T / kTransposeThreads; ++k) {
                const int idx = tid + kTransposeThreads * k, oc = idx / T, orow = idx % T;
                if (c0 + oc < cols && r0 + orow < rows)
                    out[(c0 + oc) * rows + r0 + orow] = tile[orow][oc];
            }
        }
        __syncthreads(); // the tile is reused by the next tile row
    }
}

struct CopyOp {
    __device__ float operator()(float x) const { return x; }
};

} // namespace opworks::detail

namespace opworks::ops {

// out (cols x rows) = transpose of in (rows x cols). Empty shapes submit no work.
inline void transpose(const float *in, float *out, int rows, int cols, hipStream_t stream = nullptr) {
    detail::validate_matrix(rows, cols);
    if (rows == 0 || cols == 0)
        return;
    detail::require(in && out, "transpose requires non-null pointers");
    detail::require(in != out, "transpose cannot run in place");
    constexpr int T = detail::kTransposeTile;
    const int tiles_c = static_cast<int>(detail::blocks_for64(cols, T));
    const int tiles_r = static_cast<int>(detail::blocks_for64(rows, T));
    const dim3 grid(tiles_c, tiles_r < 65535 ? tiles_r : 65535);
    const bool vec = detail::aligned16(in) && detail::aligned16(out) && rows % 4 == 0 && cols % 4 == 0;
    if (vec)
        launch_async(stream, detail::transpose_kernel<true>, grid, detail::kTransposeThreads, in, out, rows, cols);
    else
        launch_async(stream, detail::transpose_kernel<false>, grid, detail::kTransposeThreads, in, out, rows, cols);
}

// out[i] = in[i], i < n (16-byte packs when both pointers allow).
inline void copy(const float *in, float *out, int n, hipStream_t stream = nullptr) {
    map(in, out, n, detail::CopyOp{}, stream);
}

} // namespace opworks::ops

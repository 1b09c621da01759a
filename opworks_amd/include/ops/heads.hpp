#pragma once

// Token-major <-> head-major permutations and the embedding gather:
//   ops::embedding<WT>  out[t][:] = table[ids[t]][:] (fp32 or bf16 table, fp32 out)
//                                     (reference: include/ops/embedding.cuh:10-34)
//   ops::split_heads    out[h][off + t][d] = in[t][h*D + d]   (KV-cache append)
//   ops::merge_heads    out[t][h*D + d] = in[h][off + t][d]
//                                     (reference: include/ops/split_heads.cuh:9-66)
// Each lane moves four consecutive floats when the head (or row) width and
// the pointers allow 16-byte accesses, else one.

#include <limits>

#include "../core/bf16.hpp"
#include "../core/weight_pack.hpp"
#include "elementwise.hpp"

namespace opworks::detail {

// vocab bounds the ids; an id outside [0, vocab) produces a NaN row instead
// of reading outside the table.
template <typename WT, int kVec>
__global__ __launch_bounds__(kThreads) void embedding_kernel(const WT *__restrict__ table, int64_t vocab,
                                                             const int *__restrict__ ids, float *__restrict__ out,
                                                             int n, int hidden) {
    const int per_row = hidden / kVec;
    OPWORKS_GRID_LOOP(i, int64_t(n) * per_row) {
        const int t = static_cast<int>(i / per_row);
        const int c = kVec * static_cast<int>(i % per_row);
        const int id = ids[t];
        const bool ok = id >= 0 && id < vocab;
        const WT *src = table + (ok ? int64_t(id) * hidden : 0) + c;
        float *dst = out + int64_t(t) * hidden + c;
        if constexpr (kVec == 4 && std::is_same_v<WT, float>) {
            f32x4 v = *reinterpret_cast<const f32x4 *>(src);
            if (!ok)
                v = f32x4{NAN, NAN, NAN, NAN};
            *reinterpret_cast<f32x4 *>(dst) = v;
        } else {
#pragma unroll
            for (int k = 0; k < kVec; ++k)
                dst[k] = ok ? widen(src[k]) : NAN;
        }
    }
}

// kToHeads: token-major -> head-major. head-major rows live at row
// `off + t` of a slab of `stride` rows per head.
template <bool kToHeads, int kVec>
__global__ __launch_bounds__(kThreads) void permute_heads_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                                 int rows, int heads, int D, int stride, int off) {
    const int dv = D / kVec;
    OPWORKS_GRID_LOOP(i, int64_t(rows) * heads * dv) {
        const int d = kVec * static_cast<int>(i % dv);
        const int64_t th = i / dv; // t * heads + h
        const int h = static_cast<int>(th % heads);
        const int t = static_cast<int>(th / heads);
        const int64_t packed = th * D + d;
        const int64_t slab = (int64_t(h) * stride + off + t) * D + d;
        const float *src = in + (kToHeads ? packed : slab);
        float *dst = out + (kToHeads ? slab : packed);
        if constexpr (kVec == 4)
            *reinterpret_cast<f32x4 *>(dst) = *reinterpret_cast<const f32x4 *>(src);
        else
            *dst = *src;
    }
}

template <bool kToHeads>
inline void permute_heads(const float *in, float *out, int rows, int heads, int D, int stride, int off,
                          hipStream_t stream, const char *name) {
    validate_size(rows);
    if (rows == 0)
        return;
    require(heads > 0 && D > 0, kToHeads ? "split_heads requires positive head shape"
                                         : "merge_heads requires positive head shape");
    require(off >= 0 && stride >= off + rows, kToHeads ? "split_heads exceeds the output row stride"
                                                       : "merge_heads exceeds the input row stride");
    require(in && out, kToHeads ? "split_heads requires non-null pointers" : "merge_heads requires non-null pointers");
    const int64_t n = int64_t(rows) * heads * D;
    require(n <= std::numeric_limits<int>::max(), "head permutation exceeds INT_MAX elements");
    (void)name;
    if (D % 4 == 0 && aligned16(in) && aligned16(out))
        launch_async(stream, permute_heads_kernel<kToHeads, 4>, stream_grid(n / 4), kThreads, in, out, rows, heads, D,
                     stride, off);
    else
        launch_async(stream, permute_heads_kernel<kToHeads, 1>, stream_grid(n), kThreads, in, out, rows, heads, D,
                     stride, off);
}

} // namespace opworks::detail

namespace opworks::ops {

// vocab defaults to "unchecked" like the reference, whose callers validate ids.
template <typename WT>
inline void embedding(const WT *table, const int *ids, float *out, int n, int hidden, hipStream_t stream = nullptr,
                      int64_t vocab = std::numeric_limits<int64_t>::max()) {
    detail::validate_size(n);
    detail::validate_size(hidden);
    if (n == 0)
        return;
    detail::require(hidden > 0 && table && ids && out, "embedding requires positive width and non-null pointers");
    const bool vec = std::is_same_v<WT, float> && hidden % 4 == 0 && detail::aligned16(table) &&
                     detail::aligned16(out);
    if (vec)
        launch_async(stream, detail::embedding_kernel<WT, 4>, detail::stream_grid(int64_t(n) * hidden / 4), kThreads,
                     table, vocab, ids, out, n, hidden);
    else
        launch_async(stream, detail::embedding_kernel<WT, 1>, detail::stream_grid(int64_t(n) * hidden), kThreads,
                     table, vocab, ids, out, n, hidden);
}

inline void split_heads(const float *in, float *out, int rows, int heads, int head_dim, int out_row_stride,
                        int out_row_offset = 0, hipStream_t stream = nullptr) {
    detail::permute_heads<true>(in, out, rows, heads, head_dim, out_row_stride, out_row_offset, stream, "split_heads");
}

inline void merge_heads(const float *in, float *out, int rows, int heads, int head_dim, int in_row_stride,
                        int in_row_offset = 0, hipStream_t stream = nullptr) {
    detail::permute_heads<false>(in, out, rows, heads, head_dim, in_row_stride, in_row_offset, stream, "merge_heads");
}

} // namespace opworks::ops

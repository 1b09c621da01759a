#pragma once

// ops::rms_norm — row-wise RMSNorm (reference: include/ops/rms_norm.cuh:9-40).
// Per row: ss = sum(x^2); inv = rsqrtf(ss/cols + eps); out = x * inv * weight.

#include "../core/bf16.hpp"
#include "rowwise_kernels.hpp"

namespace opworks::detail {

// OT = float, or uint16_t: the output rounded to bf16 (nearest-even) as it is stored, for a
// bf16 GEMM that would round it on load anyway (the same bits, half the bytes, no extra pass).
template <int kW, int kV, bool kExact, typename OT = float>
__global__ __launch_bounds__(RowShape<kW>::kBlock) void rms_norm_reg_kernel(const float *__restrict__ x,
                                                                             const float *__restrict__ weight,
                                                                             OT *__restrict__ out, int rows,
                                                                             int cols, float eps) {
    const RowPos p = row_position<kW>(rows);
    const int n4 = cols / 4;
    const f32x4 *src = reinterpret_cast<const f32x4 *>(x + p.row * cols);
    f32x4 v[kV];
    float local = 0.f;
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int q = pack_index<kW>(p, k);
        if (p.active && (kExact || q < n4)) {
            v[k] = __builtin_nontemporal_load(src + q);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                local = fmaf(v[k][j], v[k][j], local);
        }
    }
    const float inv = rsqrtf(row_combine<kW>(wave::sum(local), p, wave::Add{}) / cols + eps);
    const f32x4 *w4 = reinterpret_cast<const f32x4 *>(weight);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int q = pack_index<kW>(p, k);
        if (p.active && (kExact || q < n4)) {
            const f32x4 w = w4[q];
            f32x4 r;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                r[j] = v[k][j] * inv * w[j];
            if constexpr (std::is_same_v<OT, float>) {
                __builtin_nontemporal_store(r, reinterpret_cast<f32x4 *>(out + p.row * cols) + q);
            } else {
                const uint2 b = make_uint2(uint32_t(float_to_bf16_rne(r[0])) | (uint32_t(float_to_bf16_rne(r[1])) << 16),
                                           uint32_t(float_to_bf16_rne(r[2])) | (uint32_t(float_to_bf16_rne(r[3])) << 16));
                reinterpret_cast<uint2 *>(out + p.row * cols)[q] = b;
            }
        }
    }
}

static __global__ void __launch_bounds__(kThreads)
    rms_norm_stream_kernel(const float *__restrict__ x, const float *__restrict__ weight, float *__restrict__ out,
                           int cols, float eps) {
    const float *row_in = x + static_cast<int64_t>(blockIdx.x) * cols;
    float *row_out = out + static_cast<int64_t>(blockIdx.x) * cols;
    float local = 0.f;
    OPWORKS_BLOCK_LOOP(j, cols) {
        const float v = row_in[j];
        local = fmaf(v, v, local);
    }
    const float inv = rsqrtf(block_reduce_all<ReduceSum>(local) / cols + eps);
    OPWORKS_BLOCK_LOOP(j, cols) { row_out[j] = row_in[j] * inv * weight[j]; }
}

} // namespace opworks::detail

namespace opworks::ops {

// RMSNorm over the last dim of a rows x cols matrix (no mean subtraction).
inline void rms_norm(const float *x, const float *weight, float *out, int rows, int cols, float eps,
                     hipStream_t stream = nullptr) {
    detail::validate_matrix(rows, cols);
    if (rows == 0)
        return;
    detail::require(cols > 0, "rms_norm requires positive columns for nonempty rows");
    detail::require(x && weight && out, "rms_norm requires non-null pointers");
    detail::require(eps > 0.f, "rms_norm epsilon must be positive");
    const bool packed = detail::aligned16(x) && detail::aligned16(weight) && detail::aligned16(out);
    const detail::RowPlan plan = detail::plan_row_for_rows(rows, cols, packed);
    if (plan.waves == 0) {
        launch_async(stream, detail::rms_norm_stream_kernel, rows, kThreads, x, weight, out, cols, eps);
        return;
    }
    detail::dispatch_row_plan_for_rows(plan, [&](auto w, auto v) {
        constexpr int kW = decltype(w)::value, kV = decltype(v)::value;
        auto *kernel = detail::row_plan_exact<kW, kV>(cols) ? detail::rms_norm_reg_kernel<kW, kV, true>
                                                              : detail::rms_norm_reg_kernel<kW, kV, false>;
        launch_async(stream, kernel, detail::row_grid<kW>(rows),
                     detail::RowShape<kW>::kBlock, x, weight, out, rows, cols, eps);
    });
}

} // namespace opworks::ops

namespace opworks::detail {

// The split-K reduction of a residual projection fused with the RMSNorm that reads its result:
// per row, hidden += sum of the splits' partial tiles (in split order, splitk_reduce_kernel's
// sums), then normed = RMSNorm(hidden) * weight in rms_norm_reg_kernel<kW, kV>'s pack order and
// reduction, written as OT (fp32, or bf16 bits for a bf16 GEMM's input). The same values as the
// reduction kernel followed by the row kernel, one launch and one pass over the rows fewer.
// Exact plans only (cols / 4 == kW * kV * 64): each lane owns whole packs of its row.
template <int kW, int kV, typename OT>
__global__ __launch_bounds__(RowShape<kW>::kBlock) void splitk_residual_rms_norm_kernel(
    const float *__restrict__ part, int splits, float *__restrict__ hidden, const float *__restrict__ weight,
    OT *__restrict__ out, int rows, int cols, float eps) {
    const RowPos p = row_position<kW>(rows);
    const int64_t mn = int64_t(rows) * cols;
    f32x4 v[kV];
    float local = 0.f;
    if (p.active) {
#pragma unroll
        for (int k = 0; k < kV; ++k) {
            const int64_t off = p.row * cols + 4 * int64_t(pack_index<kW>(p, k));
            f32x4 sum = *reinterpret_cast<const f32x4 *>(part + off);
            for (int sp = 1; sp < splits; ++sp)
                sum = sum + *reinterpret_cast<const f32x4 *>(part + sp * mn + off);
            f32x4 h = *reinterpret_cast<const f32x4 *>(hidden + off);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                h[j] = h[j] + (sum[j] + 0.f);
            *reinterpret_cast<f32x4 *>(hidden + off) = h;
            v[k] = h;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                local = fmaf(h[j], h[j], local);
        }
    }
    const float inv = rsqrtf(row_combine<kW>(wave::sum(local), p, wave::Add{}) / cols + eps);
    if (!p.active)
        return;
    const f32x4 *w4 = reinterpret_cast<const f32x4 *>(weight);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int q = pack_index<kW>(p, k);
        const f32x4 w = w4[q];
        f32x4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            r[j] = v[k][j] * inv * w[j];
        if constexpr (std::is_same_v<OT, float>) {
            __builtin_nontemporal_store(r, reinterpret_cast<f32x4 *>(out + p.row * cols) + q);
        } else {
            const uint2 b = make_uint2(uint32_t(float_to_bf16_rne(r[0])) | (uint32_t(float_to_bf16_rne(r[1])) << 16),
                                       uint32_t(float_to_bf16_rne(r[2])) | (uint32_t(float_to_bf16_rne(r[3])) << 16));
            reinterpret_cast<uint2 *>(out + p.row * cols)[q] = b;
        }
    }
}

// True when splitk_residual_rms_norm can run on this shape (an exact register plan, aligned rows).
inline bool splitk_residual_rms_norm_ok(int rows, int cols, const void *hidden, const void *weight, const void *out) {
    const RowPlan plan = plan_row_for_rows(rows, cols, aligned16(hidden) && aligned16(weight) && aligned16(out));
    return plan.waves != 0 && cols / 4 == plan.waves * plan.packs * kWaveSize;
}

template <typename OT>
inline void splitk_residual_rms_norm(const float *part, int splits, float *hidden, const float *weight, OT *out,
                                     int rows, int cols, float eps, hipStream_t stream) {
    require(splitk_residual_rms_norm_ok(rows, cols, hidden, weight, out) && splits >= 1 && eps > 0.f,
            "splitk_residual_rms_norm: unsupported shape");
    const RowPlan plan = plan_row_for_rows(rows, cols, true);
    dispatch_row_plan_for_rows(plan, [&](auto w, auto v) {
        constexpr int kW = decltype(w)::value, kV = decltype(v)::value;
        launch_async(stream, splitk_residual_rms_norm_kernel<kW, kV, OT>, row_grid<kW>(rows), RowShape<kW>::kBlock,
                     part, splits, hidden, weight, out, rows, cols, eps);
    });
}

// RMSNorm whose output is rounded to bf16 bits as it is stored (the input of a bf16 GEMM).
// Needs the register plan (16-byte aligned rows, cols a multiple of 4, at most 32768).
inline void rms_norm_to_bf16(const float *x, const float *weight, uint16_t *out, int rows, int cols, float eps,
                             hipStream_t stream) {
    validate_matrix(rows, cols);
    if (rows == 0)
        return;
    require(x && weight && out && eps > 0.f, "rms_norm_to_bf16: bad arguments");
    const RowPlan plan = plan_row_for_rows(rows, cols, aligned16(x) && aligned16(weight) && aligned16(out));
    require(plan.waves != 0, "rms_norm_to_bf16 needs aligned rows of a multiple of 4 columns");
    dispatch_row_plan_for_rows(plan, [&](auto w, auto v) {
        constexpr int kW = decltype(w)::value, kV = decltype(v)::value;
        auto *kernel = row_plan_exact<kW, kV>(cols) ? rms_norm_reg_kernel<kW, kV, true, uint16_t>
                                                     : rms_norm_reg_kernel<kW, kV, false, uint16_t>;
        launch_async(stream, kernel, row_grid<kW>(rows), RowShape<kW>::kBlock, x, weight, out, rows, cols, eps);
    });
}

} // namespace opworks::detail

#pragma once

// ops::softmax — row-wise softmax over the last dimension of a rows x cols
// fp32 matrix (reference: include/ops/softmax.cuh:10-43). Per row:
// m = max_j x_j, s = sum_j expf(x_j - m), out_j = expf(x_j - m) / s (the
// register-resident kernel multiplies by 1/s: within 1.5 ulp of the divide).
// Register-resident rows compute each expf once and read the row once.

#include "rowwise_kernels.hpp"

namespace opworks::detail {

template <int kW, int kV, bool kExact>
__global__ __launch_bounds__(RowShape<kW>::kBlock) void softmax_rows_reg_kernel(const float *__restrict__ in,
                                                                                 float *__restrict__ out, int rows,
                                                                                 int cols) {
    const RowPos p = row_position<kW>(rows);
    const int n4 = cols / 4;
    f32x4 x[kV];
    load_row_packs<kW, kV, kExact>(in, rows, cols, p, x);
    float local_max = kNegInf;
#pragma unroll
    for (int k = 0; k < kV; ++k)
        if (pack_valid<kW, kExact>(p, k, n4))
            local_max = fmaxf(local_max, fmaxf(fmaxf(x[k][0], x[k][1]), fmaxf(x[k][2], x[k][3])));
    const float m = row_combine<kW>(wave::max(local_max), p, wave::Max{});
    float local_sum = 0.f;
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        if (pack_valid<kW, kExact>(p, k, n4)) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[k][j] = expf(x[k][j] - m);
                local_sum += x[k][j];
            }
        }
    }
    const float s = row_combine<kW>(wave::sum(local_sum), p, wave::Add{});
    const float inv_s = 1.f / s; // one divide per row; each output is e * (1/s)
    f32x4 *dst = reinterpret_cast<f32x4 *>(out + p.row * cols);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int q = pack_index<kW>(p, k);
        if (p.active && (kExact || q < n4)) {
            f32x4 r;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                r[j] = x[k][j] * inv_s;
            __builtin_nontemporal_store(r, dst + q);
        }
    }
}

// One workgroup per row, three passes over the row (any cols, any alignment).
static __global__ void __launch_bounds__(kThreads) softmax_rows_stream_kernel(const float *__restrict__ in,
                                                                              float *__restrict__ out, int cols) {
    const float *row_in = in + static_cast<int64_t>(blockIdx.x) * cols;
    float *row_out = out + static_cast<int64_t>(blockIdx.x) * cols;
    float local_max = kNegInf;
    OPWORKS_BLOCK_LOOP(j, cols) { local_max = fmaxf(local_max, row_in[j]); }
    const float m = block_reduce_all<ReduceMax>(local_max);
    float local_sum = 0.f;
    OPWORKS_BLOCK_LOOP(j, cols) { local_sum += expf(row_in[j] - m); }
    const float s = block_reduce_all<ReduceSum>(local_sum);
    OPWORKS_BLOCK_LOOP(j, cols) { row_out[j] = expf(row_in[j] - m) / s; }
}

} // namespace opworks::detail

namespace opworks::ops {

// Softmax over the last dim of a rows x cols matrix. In-place (in == out) is allowed.
inline void softmax(const float *in, float *out, int rows, int cols, hipStream_t stream = nullptr) {
    detail::validate_matrix(rows, cols);
    if (rows == 0)
        return;
    detail::require(cols > 0, "softmax requires positive columns for nonempty rows");
    detail::require(in && out, "softmax requires non-null pointers");
    const detail::RowPlan plan = detail::plan_row(cols, detail::aligned16(in) && detail::aligned16(out));
    if (plan.waves == 0) {
        launch_async(stream, detail::softmax_rows_stream_kernel, rows, kThreads, in, out, cols);
        return;
    }
    detail::dispatch_row_plan(plan, [&](auto w, auto v) {
        constexpr int kW = decltype(w)::value, kV = decltype(v)::value;
        auto *kernel = detail::row_plan_exact<kW, kV>(cols) ? detail::softmax_rows_reg_kernel<kW, kV, true>
                                                              : detail::softmax_rows_reg_kernel<kW, kV, false>;
        launch_async(stream, kernel, detail::row_grid<kW>(rows),
                     detail::RowShape<kW>::kBlock, in, out, rows, cols);
    });
}

} // namespace opworks::ops

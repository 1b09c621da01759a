#pragma once

// ops::layer_norm — row-wise LayerNorm (reference: include/ops/layer_norm.cuh:10-47).
// Per row: mean = sum(x)/cols; var = sum((x-mean)^2)/cols; rstd = rsqrtf(var + eps);
// out = (x - mean) * rstd * gamma + beta. Two-pass statistics over the
// register-resident row (one HBM read, one write).

#include "rowwise_kernels.hpp"

namespace opworks::detail {

// Rows of up to 8 packs per lane are held to 64 registers, so 8 waves fit per SIMD: at 8192
// rows of 2048 (one wave each) the whole grid is then resident at once; at 67 registers the
// last 1024 rows waited for a second round (26.5 against ~22 us). One-wave rows stage gamma
// and beta in LDS once per workgroup, so the output loop does not hold every gamma/beta pack
// in registers at once (which had spilled 5 registers to scratch at that limit, +16% HBM
// traffic), and the workgroup's rows share one read of them.
template <int kW, int kV, bool kExact>
__global__ __launch_bounds__(RowShape<kW>::kBlock) __attribute__((amdgpu_waves_per_eu(kV <= 8 ? 8 : 1)))
void layer_norm_reg_kernel(
    const float *__restrict__ in, float *__restrict__ out, const float *__restrict__ gamma,
    const float *__restrict__ beta, int rows, int cols, float eps) {
    const RowPos p = row_position<kW>(rows);
    const int n4 = cols / 4;
    const f32x4 *src = reinterpret_cast<const f32x4 *>(in + p.row * cols);
    f32x4 x[kV];
    float local = 0.f;
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int q = pack_index<kW>(p, k);
        if (p.active && (kExact || q < n4)) {
            x[k] = __builtin_nontemporal_load(src + q);
            local += (x[k][0] + x[k][1]) + (x[k][2] + x[k][3]);
        }
    }
    const f32x4 *g4 = reinterpret_cast<const f32x4 *>(gamma);
    const f32x4 *b4 = reinterpret_cast<const f32x4 *>(beta);
    constexpr bool kStaged = kW == 1;
    __shared__ f32x4 gs[kStaged ? kV * kWaveSize : 1], bs[kStaged ? kV * kWaveSize : 1];
    if constexpr (kStaged) {
        for (int i = threadIdx.x; i < n4; i += RowShape<kW>::kBlock) {
            gs[i] = g4[i];
            bs[i] = b4[i];
        }
    }
    const float mean = row_combine<kW>(wave::sum(local), p, wave::Add{}) / cols;
    local = 0.f;
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int q = pack_index<kW>(p, k);
        if (p.active && (kExact || q < n4)) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float d = x[k][j] - mean;
                local = fmaf(d, d, local);
            }
        }
    }
    const float rstd = rsqrtf(row_combine<kW>(wave::sum(local), p, wave::Add{}) / cols + eps);
    if constexpr (kStaged)
        __syncthreads();
    f32x4 *dst = reinterpret_cast<f32x4 *>(out + p.row * cols);
#pragma unroll
    for (int k = 0; k < kV; ++k) {
        const int q = pack_index<kW>(p, k);
        if (p.active && (kExact || q < n4)) {
            const f32x4 g = kStaged ? gs[q] : g4[q], b = kStaged ? bs[q] : b4[q];
            f32x4 r;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                r[j] = fmaf((x[k][j] - mean) * rstd, g[j], b[j]);
            __builtin_nontemporal_store(r, dst + q);
        }
        if constexpr (!kStaged)
            __builtin_amdgcn_sched_barrier(0); // keep each pack's gamma/beta loads beside their use
    }
}

static __global__ void __launch_bounds__(kThreads)
    layer_norm_stream_kernel(const float *__restrict__ in, float *__restrict__ out, const float *__restrict__ gamma,
                             const float *__restrict__ beta, int cols, float eps) {
    const float *row_in = in + static_cast<int64_t>(blockIdx.x) * cols;
    float *row_out = out + static_cast<int64_t>(blockIdx.x) * cols;
    float local = 0.f;
    OPWORKS_BLOCK_LOOP(j, cols) { local += row_in[j]; }
    const float mean = block_reduce_all<ReduceSum>(local) / cols;
    local = 0.f;
    OPWORKS_BLOCK_LOOP(j, cols) {
        const float d = row_in[j] - mean;
        local = fmaf(d, d, local);
    }
    const float rstd = rsqrtf(block_reduce_all<ReduceSum>(local) / cols + eps);
    OPWORKS_BLOCK_LOOP(j, cols) { row_out[j] = fmaf((row_in[j] - mean) * rstd, gamma[j], beta[j]); }
}

} // namespace opworks::detail

namespace opworks::ops {

inline void layer_norm(const float *in, float *out, const float *gamma, const float *beta, int rows, int cols,
                       float eps = kLayerNormEps, hipStream_t stream = nullptr) {
    detail::validate_matrix(rows, cols);
    detail::require(std::isfinite(eps) && eps > 0, "layer norm epsilon must be finite and positive");
    if (rows == 0)
        return;
    detail::require(cols > 0, "layer norm requires positive columns for nonempty rows");
    detail::require(in && out && gamma && beta, "layer norm requires non-null pointers");
    const bool packed = detail::aligned16(in) && detail::aligned16(out) && detail::aligned16(gamma) &&
                        detail::aligned16(beta);
    const detail::RowPlan plan = detail::plan_row(cols, packed);
    if (plan.waves == 0) {
        launch_async(stream, detail::layer_norm_stream_kernel, rows, kThreads, in, out, gamma, beta, cols, eps);
        return;
    }
    detail::dispatch_row_plan(plan, [&](auto w, auto v) {
        constexpr int kW = decltype(w)::value, kV = decltype(v)::value;
        auto *kernel = detail::row_plan_exact<kW, kV>(cols) ? detail::layer_norm_reg_kernel<kW, kV, true>
                                                              : detail::layer_norm_reg_kernel<kW, kV, false>;
        launch_async(stream, kernel, detail::row_grid<kW>(rows),
                     detail::RowShape<kW>::kBlock, in, out, gamma, beta, rows, cols, eps);
    });
}

} // namespace opworks::ops

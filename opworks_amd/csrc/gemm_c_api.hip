// extern "C" GEMM / linear surface of libopworks_amd.so (include/opworks_ops.h).

#include <hip/hip_runtime.h>

#include "../include/builders/matmul.hpp"
#include "../include/ops/linear.hpp"
#include "../include/ops/linear_bf16.hpp"
#include "../include/ops/matmul.hpp"
#include "c_api_common.hpp"

using opworks::capi::guard;

extern "C" {

int opw_mat_mul_f32(const float *A, const float *B, float *C, int M, int N, int K, void *stream) {
    return guard([&] {
        opworks::ops::mat_mul(A, B, C, M, N, K, opworks::ops::PassThrough{}, static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_mat_mul_fused_f32(const float *A, const float *B, const float *bias, float *C, int M, int N, int K,
                          int b_transposed, int activation, void *stream) {
    return guard([&] {
        opworks::detail::require(activation >= 0 && activation <= 2, "activation must be 0 none, 1 relu, 2 gelu");
        opworks::ops::mat_mul_fused(A, B, bias, C, M, N, K, b_transposed != 0,
                                    static_cast<opworks::ops::Activation>(activation),
                                    static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_mat_mul_fused_ex_f32(const float *A, const float *B, const float *bias, float *C, int M, int N, int K,
                             int a_transposed, int b_transposed, int activation, void *stream) {
    return guard([&] {
        opworks::detail::require(activation >= 0 && activation <= 2, "activation must be 0 none, 1 relu, 2 gelu");
        opworks::ops::mat_mul_fused(A, B, bias, C, M, N, K, a_transposed != 0, b_transposed != 0,
                                    static_cast<opworks::ops::Activation>(activation),
                                    static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_linear_f32(const float *X, const float *W, float *Y, int rows, int in_features, int out_features,
                   void *stream) {
    return guard([&] {
        opworks::ops::linear(X, W, Y, rows, in_features, out_features, static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_linear_wbf16(const float *X, const uint16_t *W, float *Y, int rows, int in_features, int out_features,
                     void *stream) {
    return guard([&] {
        opworks::ops::linear(X, reinterpret_cast<const opworks::bf16 *>(W), Y, rows, in_features, out_features,
                             static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_linear_bf16(const float *X, const uint16_t *W, const float *bias, float *Y, int rows, int in_features,
                    int out_features, int activation, void *stream) {
    return guard([&] {
        opworks::detail::require(activation >= 0 && activation <= 2, "activation must be 0 none, 1 relu, 2 gelu");
        opworks::ops::linear_bf16_fused(X, reinterpret_cast<const opworks::bf16 *>(W), bias, Y, rows, in_features,
                                        out_features, static_cast<opworks::ops::Activation>(activation),
                                        static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_linear_bf16_bf16(const uint16_t *X, const uint16_t *W, const float *bias, float *Y, int rows,
                         int in_features, int out_features, int activation, void *stream) {
    return guard([&] {
        opworks::detail::require(activation >= 0 && activation <= 2, "activation must be 0 none, 1 relu, 2 gelu");
        opworks::ops::linear_bf16_fused(reinterpret_cast<const opworks::bf16 *>(X),
                                        reinterpret_cast<const opworks::bf16 *>(W), bias, Y, rows, in_features,
                                        out_features, static_cast<opworks::ops::Activation>(activation),
                                        static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_convert_f32_to_bf16(const float *src, uint16_t *dst, int64_t n, void *stream) {
    return guard([&] {
        opworks::ops::convert_f32_to_bf16(src, reinterpret_cast<opworks::bf16 *>(dst), n,
                                          static_cast<hipStream_t>(stream));
        return 0;
    });
}

} // extern "C"

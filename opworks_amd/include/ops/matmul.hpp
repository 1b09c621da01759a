#pragma once

// ops::mat_mul<Epilogue> — C(M x K) = epilogue(A(M x N) @ B(N x K)), all
// row-major, reduction over N (reference names and semantics:
// include/ops/matmul.cuh:70-91). M == 0 or K == 0 is a no-op; N == 0 writes
// epilogue(0). The output must not overlap an input.
//
// Runs on the fp32 MFMA kernel of gemm_f32.hpp. The reference computes a
// k-ascending fmaf chain per output; the matrix core sums the same products in
// a different order, so results agree to fp32 rounding of the dot products.

#include "../core/hip_utils.hpp"
#include "gemm_f32.hpp"

namespace opworks::ops {

// Default epilogue: identity.
struct PassThrough {
    __device__ float operator()(float x) const { return x; }
};

template <typename Epilogue = PassThrough>
inline void mat_mul(const float *A, const float *B, float *C, int M, int N, int K, Epilogue epilogue = {},
                    hipStream_t stream = nullptr) {
    detail::validate_matrix(M, N);
    detail::validate_matrix(N, K);
    detail::validate_matrix(M, K);
    if (M == 0 || K == 0)
        return;
    detail::require(C && (N == 0 || (A && B)), "matmul requires non-null pointers for nonempty tensors");
    detail::gemm_f32_launch<detail::BLayout::kn>(A, B, nullptr, C, M, K, N, epilogue, stream);
}

// Bias + activation epilogues of the fused path (MatmulBuilder, linear).
enum class Activation { none = 0, relu = 1, gelu = 2 };

struct ReluEpilogue {
    __device__ float operator()(float x) const { return fmaxf(x, 0.f); }
};
// GELU, erf form: 0.5 x (1 + erf(x / sqrt(2))). The reference names GELU
// (include/builders/matmul.cuh:7) without defining a kernel for it.
struct GeluEpilogue {
    __device__ float operator()(float x) const { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }
};

namespace detail_act {
template <detail::BLayout kB, detail::ALayout kA>
inline void gemm_act(const float *A, const float *B, const float *bias, float *C, int M, int N, int K,
                     Activation act, hipStream_t stream) {
    using detail::GemmStore;
    switch (act) {
    case Activation::none:
        detail::gemm_f32_launch<kB, PassThrough, GemmStore::store, float, kA>(A, B, bias, C, M, N, K, PassThrough{},
                                                                             stream);
        break;
    case Activation::relu:
        detail::gemm_f32_launch<kB, ReluEpilogue, GemmStore::store, float, kA>(A, B, bias, C, M, N, K, ReluEpilogue{},
                                                                              stream);
        break;
    case Activation::gelu:
        detail::gemm_f32_launch<kB, GeluEpilogue, GemmStore::store, float, kA>(A, B, bias, C, M, N, K, GeluEpilogue{},
                                                                              stream);
        break;
    default: throw std::invalid_argument("unknown activation");
    }
}
} // namespace detail_act

// C(M x K) = act(op(A) @ op(B) + bias[K]) with the reference's names: op(A) is
// M x N, stored (N x M) when a_transposed; op(B) is N x K, stored (K x N) when
// b_transposed. A transposed A is read by the GEMM in place (no copy).
inline void mat_mul_fused(const float *A, const float *B, const float *bias, float *C, int M, int N, int K,
                          bool a_transposed, bool b_transposed, Activation act, hipStream_t stream = nullptr) {
    detail::validate_matrix(M, N);
    detail::validate_matrix(N, K);
    detail::validate_matrix(M, K);
    if (M == 0 || K == 0)
        return;
    detail::require(C && (N == 0 || (A && B)), "matmul requires non-null pointers for nonempty tensors");
    using detail::ALayout;
    using detail::BLayout;
    if (a_transposed && b_transposed)
        detail_act::gemm_act<BLayout::nk, ALayout::km>(A, B, bias, C, M, K, N, act, stream);
    else if (a_transposed)
        detail_act::gemm_act<BLayout::kn, ALayout::km>(A, B, bias, C, M, K, N, act, stream);
    else if (b_transposed)
        detail_act::gemm_act<BLayout::nk, ALayout::mk>(A, B, bias, C, M, K, N, act, stream);
    else
        detail_act::gemm_act<BLayout::kn, ALayout::mk>(A, B, bias, C, M, K, N, act, stream);
}

// C(M x K) = act(A(M x N) @ B + bias[K]); B is (N x K), or (K x N) when b_transposed.
inline void mat_mul_fused(const float *A, const float *B, const float *bias, float *C, int M, int N, int K,
                          bool b_transposed, Activation act, hipStream_t stream = nullptr) {
    mat_mul_fused(A, B, bias, C, M, N, K, false, b_transposed, act, stream);
}

} // namespace opworks::ops

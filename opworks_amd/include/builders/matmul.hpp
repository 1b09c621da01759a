#pragma once

// MatmulBuilder — validated GEMM configuration (reference:
// include/builders/matmul.cuh:7-57). Same fluent surface: transpose_a/b,
// bias, activation and the apply(fn) callback. In addition run(stream)
// launches the fused MFMA kernel: C = act(A @ op(B) + bias), with the bias and
// activation applied in the kernel's epilogue (the reference has no kernel
// behind this builder). Shapes use the reference's names: A is m x n, B is
// n x k (k x n when transposed), output m x k.

#include "../ops/matmul.hpp"
#include "builder_common.hpp"

namespace opworks {

enum class MatmulActivation { none, relu, gelu };

class MatmulBuilder {
  public:
    MatmulBuilder(DeviceSpan<const float> a, DeviceSpan<const float> b, DeviceSpan<float> output, int m, int n, int k,
                  hipStream_t stream = nullptr)
        : a_(a), b_(b), output_(output), m_(m), n_(n), k_(k), stream_(stream) {
        detail::validate_matrix(m, n);
        detail::validate_matrix(n, k);
        detail::validate_matrix(m, k);
        detail::require(a.size() >= m * n && b.size() >= n * k && output.size() >= m * k,
                        "matmul buffer is too small");
    }
    MatmulBuilder &transpose_a(bool value = true) {
        transpose_a_ = value;
        return *this;
    }
    MatmulBuilder &transpose_b(bool value = true) {
        transpose_b_ = value;
        return *this;
    }
    MatmulBuilder &bias(DeviceSpan<const float> value) {
        bias_ = value;
        return *this;
    }
    MatmulBuilder &activation(MatmulActivation value) {
        activation_ = value;
        return *this;
    }
    bool transposed_a() const { return transpose_a_; }
    bool transposed_b() const { return transpose_b_; }
    DeviceSpan<const float> a() const { return a_; }
    DeviceSpan<const float> b() const { return b_; }
    DeviceSpan<float> output() const { return output_; }
    DeviceSpan<const float> bias() const { return bias_; }
    MatmulActivation activation() const { return activation_; }
    int m() const { return m_; }
    int n() const { return n_; }
    int k() const { return k_; }
    hipStream_t stream() const { return stream_; }

    template <typename Fn> decltype(auto) apply(Fn &&fn) const { return apply_builder(*this, static_cast<Fn &&>(fn)); }

    // Launches output = act(a @ op(b) + bias) on the builder's stream.
    void run() const {
        detail::require(!transpose_a_, "MatmulBuilder::run: transpose_a is not supported by the fused kernel");
        detail::require(bias_.size() == 0 || bias_.size() >= k_, "matmul bias is shorter than the output width");
        ops::mat_mul_fused(a_.data(), b_.data(), bias_.size() ? bias_.data() : nullptr, output_.data(), m_, n_, k_,
                           transpose_b_, static_cast<ops::Activation>(static_cast<int>(activation_)), stream_);
    }

  private:
    DeviceSpan<const float> a_, b_;
    DeviceSpan<float> output_;
    DeviceSpan<const float> bias_;
    int m_, n_, k_;
    bool transpose_a_ = false, transpose_b_ = false;
    MatmulActivation activation_ = MatmulActivation::none;
    hipStream_t stream_;
};

} // namespace opworks

#pragma once

// MatmulBuilder — a checked GEMM description with the reference's fluent
// surface (interface: include/builders/matmul.cuh:7-57: transpose_a/b, bias,
// activation, accessors, apply(fn)). run() is an addition: it launches the
// fused MFMA kernel, output = act(a @ op(b) + bias), with bias and activation
// applied in the kernel's epilogue; a transposed a or b is read in place.
// Shapes keep the reference's names: a is m x n (n x m when transposed), b
// is n x k (k x n when transposed), the output m x k.

#include <initializer_list>
#include <utility>

#include "../ops/matmul.hpp"
#include "builder_common.hpp"

namespace opworks {

enum class MatmulActivation { none, relu, gelu };

class MatmulBuilder : public detail::CallbackBuilder<MatmulBuilder> {
  public:
    MatmulBuilder(DeviceSpan<const float> a, DeviceSpan<const float> b, DeviceSpan<float> output, int m, int n, int k,
                  hipStream_t stream = nullptr)
        : lhs_(a), rhs_(b), out_(output), dims_{m, n, k}, stream_(stream) {
        for (auto [r, c] : {std::pair{m, n}, std::pair{n, k}, std::pair{m, k}})
            detail::validate_matrix(r, c);
        const bool fits = lhs_.size() >= int64_t(m) * n && rhs_.size() >= int64_t(n) * k &&
                          out_.size() >= int64_t(m) * k;
        detail::require(fits, "matmul buffer is too small");
    }

    MatmulBuilder &transpose_a(bool value = true) { return flags_.ta = value, *this; }
    MatmulBuilder &transpose_b(bool value = true) { return flags_.tb = value, *this; }
    MatmulBuilder &bias(DeviceSpan<const float> value) { return bias_ = value, *this; }
    MatmulBuilder &activation(MatmulActivation value) { return flags_.act = value, *this; }

    bool transposed_a() const { return flags_.ta; }
    bool transposed_b() const { return flags_.tb; }
    DeviceSpan<const float> a() const { return lhs_; }
    DeviceSpan<const float> b() const { return rhs_; }
    DeviceSpan<float> output() const { return out_; }
    DeviceSpan<const float> bias() const { return bias_; }
    MatmulActivation activation() const { return flags_.act; }
    int m() const { return dims_[0]; }
    int n() const { return dims_[1]; }
    int k() const { return dims_[2]; }
    hipStream_t stream() const { return stream_; }

    void run() const {
        detail::require(bias_.size() == 0 || bias_.size() >= k(), "matmul bias is shorter than the output width");
        const auto act = flags_.act == MatmulActivation::relu   ? ops::Activation::relu
                         : flags_.act == MatmulActivation::gelu ? ops::Activation::gelu
                                                                : ops::Activation::none;
        ops::mat_mul_fused(lhs_.data(), rhs_.data(), bias_.size() ? bias_.data() : nullptr, out_.data(), m(), n(),
                           k(), flags_.ta, flags_.tb, act, stream_);
    }

  private:
    struct Flags {
        bool ta = false, tb = false;
        MatmulActivation act = MatmulActivation::none;
    };
    DeviceSpan<const float> lhs_, rhs_;
    DeviceSpan<float> out_;
    DeviceSpan<const float> bias_;
    int dims_[3];
    Flags flags_;
    hipStream_t stream_;
};

} // namespace opworks

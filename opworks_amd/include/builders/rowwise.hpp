#pragma once

// RowwiseBuilder — a checked description of one row-wise operation
// (reference interface: include/builders/rowwise.cuh:9-63: the three
// factories, accessors, validation rules and apply(fn)). run() is an addition:
// it launches the matching row kernel on the builder's stream.

#include <cmath>

#include "../ops/layer_norm.hpp"
#include "../ops/rms_norm.hpp"
#include "../ops/softmax.hpp"
#include "builder_common.hpp"

namespace opworks {

enum class RowwiseOp { softmax, layer_norm, rms_norm };

class RowwiseBuilder : public detail::CallbackBuilder<RowwiseBuilder> {
    struct Spec {
        RowwiseOp op;
        DeviceSpan<const float> in;
        DeviceSpan<float> out;
        const float *scale;  // gamma (layer norm) or weight (rms norm)
        const float *shift;  // beta (layer norm only)
        int rows, cols;
        float eps;
        hipStream_t stream;
    };

  public:
    static RowwiseBuilder softmax(DeviceSpan<const float> input, DeviceSpan<float> output, int rows, int cols,
                                  hipStream_t stream = nullptr) {
        return RowwiseBuilder({RowwiseOp::softmax, input, output, nullptr, nullptr, rows, cols, kLayerNormEps, stream});
    }
    static RowwiseBuilder layer_norm(DeviceSpan<const float> input, DeviceSpan<float> output,
                                     DeviceSpan<const float> gamma, DeviceSpan<const float> beta, int rows, int cols,
                                     float eps = kLayerNormEps, hipStream_t stream = nullptr) {
        return RowwiseBuilder({RowwiseOp::layer_norm, input, output, gamma.data(), beta.data(), rows, cols, eps, stream});
    }
    static RowwiseBuilder rms_norm(DeviceSpan<const float> input, DeviceSpan<float> output,
                                   DeviceSpan<const float> weight, int rows, int cols, float eps = kLayerNormEps,
                                   hipStream_t stream = nullptr) {
        return RowwiseBuilder({RowwiseOp::rms_norm, input, output, weight.data(), nullptr, rows, cols, eps, stream});
    }

    RowwiseOp op() const { return s_.op; }
    DeviceSpan<const float> input() const { return s_.in; }
    DeviceSpan<float> output() const { return s_.out; }
    const float *parameter() const { return s_.scale; }
    const float *beta() const { return s_.shift; }
    int rows() const { return s_.rows; }
    int cols() const { return s_.cols; }
    float epsilon() const { return s_.eps; }
    hipStream_t stream() const { return s_.stream; }

    void run() const {
        if (s_.op == RowwiseOp::softmax)
            ops::softmax(s_.in.data(), s_.out.data(), s_.rows, s_.cols, s_.stream);
        else if (s_.op == RowwiseOp::layer_norm)
            ops::layer_norm(s_.in.data(), s_.out.data(), s_.scale, s_.shift, s_.rows, s_.cols, s_.eps, s_.stream);
        else
            ops::rms_norm(s_.in.data(), s_.scale, s_.out.data(), s_.rows, s_.cols, s_.eps, s_.stream);
    }

  private:
    explicit RowwiseBuilder(const Spec &s) : s_(s) { check(s_); }

    static void check(const Spec &s) {
        detail::validate_matrix(s.rows, s.cols);
        const int64_t elems = int64_t(s.rows) * s.cols;
        detail::require(s.in.size() >= elems && s.out.size() >= elems, "rowwise buffer is too small");
        detail::require(s.rows == 0 || s.cols > 0, "rowwise columns must be positive");
        detail::require(std::isfinite(s.eps) && s.eps > 0, "rowwise epsilon must be finite and positive");
        const bool empty_rows = s.cols == 0;
        if (s.op != RowwiseOp::softmax)
            detail::require(empty_rows || s.scale, "rowwise parameter is required");
        if (s.op == RowwiseOp::layer_norm)
            detail::require(empty_rows || s.shift, "layer norm beta is required");
    }

    Spec s_;
};

} // namespace opworks

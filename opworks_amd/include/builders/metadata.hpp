#pragma once

// Scan, Transform and GatherScatter builders: checked descriptions with the
// apply(fn) callback, the extension points the reference exposes (interfaces:
// include/builders/scan.cuh, include/builders/transform.cuh,
// include/builders/gather_scatter.cuh). run() is an addition: the reference
// leaves these operations to the callback, and run() launches this library's
// kernel for the configured operation on the builder's stream.

#include "../ops/gather_scatter.hpp"
#include "../ops/scan.hpp"
#include "../ops/transform.hpp"
#include "builder_common.hpp"

namespace opworks {

enum class ScanOp { sum, maximum };
enum class TransformOp { transpose, reshape, copy };
enum class GatherScatterOp { gather, scatter };

class ScanBuilder : public detail::CallbackBuilder<ScanBuilder> {
  public:
    ScanBuilder(DeviceSpan<const float> input, DeviceSpan<float> output, int n, ScanOp op = ScanOp::sum,
                bool inclusive = true, hipStream_t stream = nullptr)
        : in_(input), out_(output), n_(n), kind_(op), inclusive_(inclusive), stream_(stream) {
        detail::validate_size(n);
        detail::require(in_.size() >= n && out_.size() >= n, "scan buffers are too small");
    }

    // Fluent setters.
    ScanBuilder &op(ScanOp value) { return kind_ = value, *this; }
    ScanBuilder &inclusive(bool value = true) { return inclusive_ = value, *this; }

    DeviceSpan<const float> input() const { return in_; }
    DeviceSpan<float> output() const { return out_; }
    int size() const { return n_; }
    ScanOp operation() const { return kind_; }
    bool is_inclusive() const { return inclusive_; }
    hipStream_t stream() const { return stream_; }

    // Scratch comes from the stream-ordered allocator; see ops::scan.
    void run() const { ops::scan(in_.data(), out_.data(), n_, kind_ == ScanOp::maximum, inclusive_, stream_); }
    // Allocation-free form: `workspace` holds ops::scan_workspace_size(size()) floats.
    void run(DeviceSpan<float> workspace) const {
        ops::scan(in_.data(), out_.data(), n_, kind_ == ScanOp::maximum, inclusive_, workspace, stream_);
    }

  private:
    DeviceSpan<const float> in_;
    DeviceSpan<float> out_;
    int n_;
    ScanOp kind_;
    bool inclusive_;
    hipStream_t stream_;
};

class TransformBuilder : public detail::CallbackBuilder<TransformBuilder> {
  public:
    TransformBuilder(DeviceSpan<const float> input, DeviceSpan<float> output, int rows, int cols,
                     TransformOp op = TransformOp::copy, hipStream_t stream = nullptr)
        : in_(input), out_(output), rows_(rows), cols_(cols), kind_(op), stream_(stream) {
        detail::validate_matrix(rows, cols);
        const int64_t elems = int64_t(rows) * cols;
        detail::require(in_.size() >= elems && out_.size() >= elems, "transform buffers are too small");
    }

    TransformBuilder &op(TransformOp value) { return kind_ = value, *this; }

    DeviceSpan<const float> input() const { return in_; }
    DeviceSpan<float> output() const { return out_; }
    int rows() const { return rows_; }
    int cols() const { return cols_; }
    TransformOp operation() const { return kind_; }
    hipStream_t stream() const { return stream_; }

    // transpose writes a cols x rows matrix; reshape and copy copy rows * cols elements.
    void run() const {
        if (kind_ == TransformOp::transpose)
            ops::transpose(in_.data(), out_.data(), rows_, cols_, stream_);
        else
            ops::copy(in_.data(), out_.data(), rows_ * cols_, stream_);
    }

  private:
    DeviceSpan<const float> in_;
    DeviceSpan<float> out_;
    int rows_, cols_;
    TransformOp kind_;
    hipStream_t stream_;
};

class GatherScatterBuilder : public detail::CallbackBuilder<GatherScatterBuilder> {
  public:
    GatherScatterBuilder(DeviceSpan<const float> input, DeviceSpan<float> output, DeviceSpan<const int> indices,
                         int count, GatherScatterOp op, hipStream_t stream = nullptr)
        : in_(input), out_(output), idx_(indices), count_(count), kind_(op), stream_(stream) {
        detail::validate_size(count);
        detail::require(idx_.size() >= count, "index buffer is too small");
        detail::require(out_.size() >= count, "gather/scatter output is too small");
    }

    DeviceSpan<const float> input() const { return in_; }
    DeviceSpan<float> output() const { return out_; }
    DeviceSpan<const int> indices() const { return idx_; }
    int count() const { return count_; }
    GatherScatterOp operation() const { return kind_; }
    hipStream_t stream() const { return stream_; }

    // gather bounds indices by input().size(), scatter by output().size().
    void run() const {
        if (kind_ == GatherScatterOp::gather) {
            ops::gather(in_.data(), in_.size(), idx_.data(), out_.data(), count_, stream_);
        } else {
            detail::require(in_.size() >= count_, "scatter input is too small");
            ops::scatter(in_.data(), idx_.data(), out_.data(), out_.size(), count_, stream_);
        }
    }

  private:
    DeviceSpan<const float> in_;
    DeviceSpan<float> out_;
    DeviceSpan<const int> idx_;
    int count_;
    GatherScatterOp kind_;
    hipStream_t stream_;
};

} // namespace opworks

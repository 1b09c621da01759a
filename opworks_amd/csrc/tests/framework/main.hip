// Framework self-test of the C++ operator API, driven by data.
//
// The known answers of the reference's unit test (tests/unit/framework.cu) are
// stored as tests/golden/framework_kats.json; this program reads them with the
// library's own JSON parser and runs a table of sections, each turning one or
// more fixtures into device work and a comparison. Argument contracts form a
// table of (description, expected outcome, call). Failures are collected and
// reported together rather than stopping at the first.
//
//   framework <framework_kats.json>
//
// Exit status: 0 pass, 1 a check failed, 2 bad usage or fixture file,
// 77 no HIP device.
#include <opworks>
#include <runtime/json.hpp>

#include <cmath>
#include <cstdio>
#include <fstream>
#include <functional>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

using namespace opworks;

void second_translation_unit();

namespace {

// ---- functors in the shape the API documents --------------------------------
struct Add {
    static constexpr int kArity = 2;
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct Scale {
    static constexpr int kArity = 1;
    float factor = 2;
    __device__ float operator()(float x) const { return factor * x; }
};
struct Sum {
    static __device__ float identity() { return 0; }
    static __device__ float combine(float a, float b) { return a + b; }
};
struct Product {
    static __device__ float identity() { return 1; }
    static __device__ float combine(float a, float b) { return a * b; }
};

// ---- compile-time facts of the ownership model -------------------------------
namespace facts {
static_assert(!std::is_copy_constructible_v<DeviceBuffer>, "owners are move-only");
static_assert(std::is_nothrow_move_constructible_v<DeviceBuffer>, "moving an owner cannot throw");
static_assert(std::is_convertible_v<DeviceSpan<float>, DeviceSpan<const float>>, "spans add const");
static_assert(!std::is_convertible_v<DeviceSpan<const float>, DeviceSpan<float>>, "spans never drop const");
static_assert(std::is_same_v<decltype(std::declval<const DeviceBuffer &>().view().data()), const float *>,
              "a const owner lends read-only views");
static_assert(!std::is_constructible_v<ElementwiseBuilder, DeviceBuffer &&>, "builders refuse temporaries");
static_assert(!std::is_constructible_v<ElementwiseBuilder, DeviceBuffer &, DeviceBuffer &&>, "");
static_assert(!std::is_constructible_v<ElementwiseBuilder, DeviceBuffer &&, DeviceBuffer &>, "");
static_assert(!std::is_constructible_v<ReductionBuilder, DeviceBuffer &&>, "");
} // namespace facts

// ---- fixtures and reporting ---------------------------------------------------
using json::Value;

std::vector<float> floats(const Value &v) {
    std::vector<float> out;
    for (const Value &x : v.as_array())
        out.push_back(static_cast<float>(x.as_number()));
    return out;
}
std::vector<int> ints(const Value &v) {
    std::vector<int> out;
    for (const Value &x : v.as_array())
        out.push_back(static_cast<int>(x.as_int()));
    return out;
}

class Report {
  public:
    explicit Report(float tol) : tol_(tol) {}

    void begin(const char *section) { section_ = section; }

    void expect(bool ok, const std::string &what) {
        if (!ok)
            failures_.push_back(section_ + ": " + what);
    }

    // The reference's criterion |a - e| <= tol (1 + |e|) (framework.cu:45-48), element by element.
    void near(const std::vector<float> &got, const std::vector<float> &want, const std::string &what) {
        if (got.size() != want.size()) {
            expect(false, what + ": " + std::to_string(got.size()) + " values, want " + std::to_string(want.size()));
            return;
        }
        for (size_t i = 0; i < got.size(); ++i) {
            const bool ok = std::isfinite(got[i]) && std::fabs(got[i] - want[i]) <= tol_ * (1 + std::fabs(want[i]));
            if (!ok) {
                std::ostringstream msg;
                msg << what << " [" << i << "] got " << got[i] << " want " << want[i];
                expect(false, msg.str());
                return;
            }
        }
    }
    void near(float got, float want, const std::string &what) { near(std::vector<float>{got}, {want}, what); }

    const std::vector<std::string> &failures() const { return failures_; }

  private:
    float tol_;
    std::string section_;
    std::vector<std::string> failures_;
};

struct Fixtures {
    Value root;
    const Value &operator[](const char *key) const { return root.at(key); }
};

struct HipStream {
    hipStream_t s = nullptr;
    HipStream() { OPWORKS_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)); }
    ~HipStream() { (void)hipStreamDestroy(s); }
    HipStream(const HipStream &) = delete;
    HipStream &operator=(const HipStream &) = delete;
};

__global__ void write_value(float *out, float value) { out[0] = value; }

// ---- contracts: a table of calls and the outcome each must have -------------
enum class Outcome { runs, rejected };
struct Contract {
    const char *what;
    Outcome want;
    std::function<void()> call;
};

void run_contracts(Report &r, const std::vector<Contract> &table) {
    for (const Contract &c : table) {
        Outcome got = Outcome::runs;
        try {
            c.call();
        } catch (const std::invalid_argument &) {
            got = Outcome::rejected;
        }
        r.expect(got == c.want, std::string(c.what) + (c.want == Outcome::rejected ? ": not rejected"
                                                                                      : ": rejected"));
    }
}

// ---- sections ---------------------------------------------------------------
void section_translation_units(Report &r, const Fixtures &) {
    try {
        second_translation_unit();
    } catch (const std::exception &e) {
        r.expect(false, e.what());
    }
}

void section_ownership(Report &r, const Fixtures &f) {
    DeviceBuffer none(0);
    r.expect(none.data() == nullptr && none.to_host().empty(), "an empty owner holds no memory");
    r.expect(DeviceBuffer::from_host({}).size() == 0, "an empty host vector uploads to an empty owner");
    auto a = DeviceBuffer::from_host(floats(f["add"].at("a")));
    auto b = DeviceBuffer::from_host(floats(f["add"].at("b")));
    const float *address = a.data();
    const DeviceSpan<float> lent = a.view();
    DeviceBuffer taken(std::move(a));
    r.expect(a.data() == nullptr && a.size() == 0 && taken.data() == address, "move construction empties the source");
    b = std::move(taken);
    r.expect(taken.data() == nullptr && b.data() == lent.data(), "move assignment keeps the lent address");
    r.near(b.to_host(), floats(f["add"].at("a")), "moved contents");
    auto typed = TypedDeviceBuffer<int32_t>::from_host(std::vector<int32_t>{7, -3, 11});
    r.expect(typed.to_host() == std::vector<int32_t>{7, -3, 11} && typed.size() == 3, "typed int32 round trip");
    TypedDeviceBuffer<int32_t> typed_taken = std::move(typed);
    r.expect(typed.size() == 0 && typed.data() == nullptr && typed_taken.size() == 3, "typed move");
}

void section_contracts(Report &r, const Fixtures &f) {
    DeviceBuffer none(0);
    auto a = DeviceBuffer::from_host(floats(f["add"].at("a")));
    auto b = DeviceBuffer::from_host(floats(f["add"].at("b")));
    auto one = DeviceBuffer::from_host({1});
    const std::vector<Contract> table = {
        {"negative owner size", Outcome::rejected, [] { DeviceBuffer bad(-1); }},
        {"null span with elements", Outcome::rejected, [] { DeviceSpan<float> bad(nullptr, 1); }},
        {"scalar copy of an empty owner", Outcome::rejected, [&] { (void)none.to_host_scalar(); }},
        {"scalar copy of three elements", Outcome::rejected, [&] { (void)a.to_host_scalar(); }},
        {"builder inputs of unequal length", Outcome::rejected, [&] { ElementwiseBuilder bad(a, one); }},
        {"binary functor on one input", Outcome::rejected, [&] { (void)ElementwiseBuilder(a).apply<Add>(); }},
        {"unary functor on two inputs", Outcome::rejected, [&] { (void)ElementwiseBuilder(a, b).apply<Scale>(); }},
        {"empty map", Outcome::runs, [] { ops::map(nullptr, nullptr, 0, Scale{}); }},
        {"empty softmax", Outcome::runs, [] { ops::softmax(nullptr, nullptr, 0, 3); }},
        {"empty layer norm", Outcome::runs, [] { ops::layer_norm(nullptr, nullptr, nullptr, nullptr, 0, 3); }},
        {"empty matmul", Outcome::runs, [] { ops::mat_mul(nullptr, nullptr, nullptr, 0, 4, 5); }},
        {"negative map length", Outcome::rejected, [] { ops::map(nullptr, nullptr, -1, Scale{}); }},
        {"null map pointers", Outcome::rejected, [] { ops::map(nullptr, nullptr, 1, Scale{}); }},
        {"null reduce output", Outcome::rejected, [] { ops::reduce<Sum>(nullptr, nullptr, 0); }},
        {"softmax without columns", Outcome::rejected, [] { ops::softmax(nullptr, nullptr, 1, 0); }},
        {"softmax with negative rows", Outcome::rejected, [] { ops::softmax(nullptr, nullptr, -1, 2); }},
        {"layer norm without columns", Outcome::rejected,
         [] { ops::layer_norm(nullptr, nullptr, nullptr, nullptr, 1, 0); }},
        {"layer norm with eps 0", Outcome::rejected,
         [] { ops::layer_norm(nullptr, nullptr, nullptr, nullptr, 0, 3, 0); }},
        {"layer norm with infinite eps", Outcome::rejected,
         [] { ops::layer_norm(nullptr, nullptr, nullptr, nullptr, 0, 3, INFINITY); }},
        {"matmul with null operands", Outcome::rejected, [] { ops::mat_mul(nullptr, nullptr, nullptr, 2, 2, 2); }},
        {"matrix beyond INT_MAX elements", Outcome::rejected, [] { detail::validate_matrix(65536, 65536); }},
        {"launch with an empty grid", Outcome::rejected, [&] { launch_async(nullptr, write_value, 0, 1, a.data(), 0.f); }},
    };
    run_contracts(r, table);
    r.expect(detail::blocks_for(std::numeric_limits<int>::max(), 256) == 8388608, "ceil divide at INT_MAX");
    r.expect(num_blocks_for(0) == 0, "no workgroups for no work");
}

void section_map_known_answers(Report &r, const Fixtures &f) {
    const Value &add = f["add"], &scale = f["scale3"];
    auto a = DeviceBuffer::from_host(floats(add.at("a")));
    auto b = DeviceBuffer::from_host(floats(add.at("b")));
    r.near(ElementwiseBuilder(a, b).apply<Add>().to_host(), floats(add.at("out")), add.at("line").as_string());
    auto x = DeviceBuffer::from_host(floats(scale.at("x")));
    r.near(ElementwiseBuilder(x.view()).apply(Scale{3}).to_host(), floats(scale.at("out")),
           scale.at("line").as_string());
    DeviceBuffer none(0);
    r.expect(ElementwiseBuilder(none).apply<Scale>().size() == 0, "empty builder output");
}

void section_map_boundaries(Report &r, const Fixtures &f) {
    const Value &kat = f["elementwise_boundaries"];
    const float twice = static_cast<float>(kat.at("add_same").as_number());
    const float thrice = static_cast<float>(kat.at("scale_in_place").as_number());
    for (int n : ints(kat.at("n"))) {
        for (int offset : ints(kat.at("offsets"))) { // offset 1 misaligns every pointer: the scalar path
            std::vector<float> host(static_cast<size_t>(n + offset));
            for (size_t i = 0; i < host.size(); ++i)
                host[i] = static_cast<float>(static_cast<int>(i) - 10);
            auto a = DeviceBuffer::from_host(host);
            auto b = DeviceBuffer::from_host(host);
            DeviceBuffer out(n + offset);
            ops::map(a.data() + offset, b.data() + offset, out.data() + offset, n, Add{});
            std::vector<float> want(host.begin() + offset, host.end()), got = out.to_host();
            for (float &w : want)
                w *= twice;
            r.near(std::vector<float>(got.begin() + offset, got.end()), want, "add n=" + std::to_string(n));
            ops::map(a.data() + offset, a.data() + offset, n, Scale{thrice}); // exact in place
            got = a.to_host();
            for (size_t i = 0; i < want.size(); ++i)
                want[i] = thrice * host[i + static_cast<size_t>(offset)];
            r.near(std::vector<float>(got.begin() + offset, got.end()), want, "in-place scale n=" + std::to_string(n));
        }
    }
}

void section_reductions(Report &r, const Fixtures &f) {
    HipStream hs;
    const std::vector<int> sizes = ints(f["sum_of_ones"].at("n"));
    int largest = 0;
    for (int n : sizes)
        largest = n > largest ? n : largest;
    auto ones = DeviceBuffer::from_host(std::vector<float>(static_cast<size_t>(largest), 1.f), hs.s);
    DeviceBuffer result(1);
    DeviceBuffer ws(ops::reduction_workspace_size(largest));
    for (int n : sizes) {
        ops::reduce<Sum>(ones.data(), result.data(), n, ws.view(), hs.s);
        r.near(result.to_host_scalar(hs.s), static_cast<float>(n), "workspace sum of ones n=" + std::to_string(n));
        ops::reduce<Sum>(ones.data(), result.data(), n, hs.s);
        r.near(result.to_host_scalar(hs.s), static_cast<float>(n), "allocating sum of ones n=" + std::to_string(n));
    }
    DeviceBuffer none(0);
    r.near(ReductionBuilder(none).apply<Product>().to_host_scalar(),
           static_cast<float>(f["empty_product"].at("out").as_number()), "empty product");
    auto three = DeviceBuffer::from_host(floats(f["add"].at("a")));
    r.near(ReductionBuilder(three).apply<Sum>().to_host_scalar(), 6, "builder sum of 1, 2, 3");
    r.near(ReductionBuilder(ones).apply<Sum>(ws.view(), hs.s).to_host_scalar(hs.s), static_cast<float>(largest),
           "builder sum with a workspace, on a stream");
    r.near(ElementwiseBuilder(ones).apply(Scale{3}, hs.s).to_host(hs.s).back(), 3, "builder map on a stream");

    // Partials appear past one 8192-element workgroup chunk; a missing workspace is then a contract error.
    r.expect(ops::reduction_workspace_size(8192) == 0 && ops::reduction_workspace_size(20000) == 3,
             "workspace sizes");
    auto many = DeviceBuffer::from_host(std::vector<float>(20000, 1.f), hs.s);
    run_contracts(r, {{"multi-chunk reduce without a workspace", Outcome::rejected,
                       [&] { ops::reduce<Sum>(many.data(), result.data(), 20000, DeviceSpan<float>{}, hs.s); }},
                      {"negative reduce length", Outcome::rejected,
                       [&] { ops::reduce<Sum>(ones.data(), result.data(), -1, hs.s); }}});
    DeviceBuffer ws3(3);
    ops::reduce<Sum>(many.data(), result.data(), many.size(), ws3.view(), hs.s);
    r.near(result.to_host_scalar(hs.s), 20000, "multi-chunk sum");
}

void section_graph_replay(Report &r, const Fixtures &f) {
    const Value &kat = f["graph_replays"];
    HipStream hs;
    const int n = static_cast<int>(kat.at("n").as_int());
    auto data = DeviceBuffer::from_host(std::vector<float>(static_cast<size_t>(n), 1.f), hs.s);
    DeviceBuffer result(1);
    DeviceBuffer ws(ops::reduction_workspace_size(n));
    // One captured store, an in-place doubling and a reduction: each replay doubles
    // the data again and nothing inside allocates or synchronizes.
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    OPWORKS_HIP_CHECK(hipStreamBeginCapture(hs.s, hipStreamCaptureModeGlobal));
    launch_async(hs.s, write_value, 1, 1, result.data(), -1.f);
    ops::map(data.data(), data.data(), n, Scale{2}, hs.s);
    ops::reduce<Sum>(data.data(), result.data(), n, ws.view(), hs.s);
    OPWORKS_HIP_CHECK(hipStreamEndCapture(hs.s, &graph));
    OPWORKS_HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    for (const char *key : {"after_first", "after_second"}) {
        OPWORKS_HIP_CHECK(hipGraphLaunch(exec, hs.s));
        r.near(result.to_host_scalar(hs.s), static_cast<float>(kat.at(key).as_number()), key);
    }
    OPWORKS_HIP_CHECK(hipGraphExecDestroy(exec));
    OPWORKS_HIP_CHECK(hipGraphDestroy(graph));
}

void section_launch_helpers(Report &r, const Fixtures &) {
    HipStream hs;
    DeviceBuffer cell(1);
    launch_sync(hs.s, write_value, 1, 1, cell.data(), 7.f);
    r.expect(hipStreamQuery(hs.s) == hipSuccess, "launch_sync leaves its stream idle");
    r.near(cell.to_host_scalar(hs.s), 7, "launch_sync on a stream");
    launch(write_value, 1, 1, cell.data(), 8.f);
    synchronize();
    r.near(cell.to_host_scalar(), 8, "launch then synchronize");
    launch_sync(write_value, 1, 1, cell.data(), 9.f);
    r.near(cell.to_host_scalar(), 9, "launch_sync on the null stream");
}

void section_row_ops(Report &r, const Fixtures &f) {
    HipStream hs;
    const Value &sm = f["softmax_2x5"], &ln = f["layer_norm_2x5"];
    const std::vector<float> hx = floats(sm.at("x"));
    const int rows = 2, cols = 5;
    auto x = DeviceBuffer::from_host(hx);
    DeviceBuffer y(rows * cols);
    ops::softmax(x.data(), y.data(), rows, cols, hs.s);
    r.near(y.to_host(hs.s), floats(sm.at("out")), "softmax " + sm.at("line").as_string());
    RowwiseBuilder::softmax(x.view(), y.view(), rows, cols, hs.s).run();
    r.near(y.to_host(hs.s), floats(sm.at("out")), "RowwiseBuilder softmax");

    auto gamma = DeviceBuffer::from_host(std::vector<float>(cols, static_cast<float>(ln.at("gamma").as_number())));
    auto beta = DeviceBuffer::from_host(std::vector<float>(cols, static_cast<float>(ln.at("beta").as_number())));
    const float eps = static_cast<float>(ln.at("eps").as_number());
    ops::layer_norm(x.data(), y.data(), gamma.data(), beta.data(), rows, cols, eps, hs.s);
    r.near(y.to_host(hs.s), floats(ln.at("out")), "layer norm " + ln.at("line").as_string());
    RowwiseBuilder::layer_norm(x.view(), y.view(), gamma.view(), beta.view(), rows, cols, eps, hs.s).run();
    r.near(y.to_host(hs.s), floats(ln.at("out")), "RowwiseBuilder layer norm");

    // rms_norm: x * g / sqrt(mean(x^2) + eps), with the layer-norm fixture's gamma
    std::vector<float> want(hx.size());
    for (int row = 0; row < rows; ++row) {
        float ms = 0;
        for (int c = 0; c < cols; ++c)
            ms += hx[row * cols + c] * hx[row * cols + c];
        ms /= cols;
        for (int c = 0; c < cols; ++c)
            want[row * cols + c] = hx[row * cols + c] * static_cast<float>(ln.at("gamma").as_number()) /
                                   std::sqrt(ms + eps);
    }
    RowwiseBuilder::rms_norm(x.view(), y.view(), gamma.view(), rows, cols, eps, hs.s).run();
    r.near(y.to_host(hs.s), want, "RowwiseBuilder rms norm");
    run_contracts(r, {{"rms norm with NaN eps", Outcome::rejected,
                       [&] { RowwiseBuilder::rms_norm(x.view(), y.view(), gamma.view(), rows, cols, NAN, hs.s); }},
                      {"softmax rows beyond the buffer", Outcome::rejected,
                       [&] { RowwiseBuilder::softmax(x.view(), y.view(), rows + 1, cols, hs.s); }}});
}

// Stores an M x N row-major matrix as its N x M transpose.
std::vector<float> transposed(const std::vector<float> &m, int rows, int cols) {
    std::vector<float> t(m.size());
    for (int i = 0; i < rows; ++i)
        for (int j = 0; j < cols; ++j)
            t[static_cast<size_t>(j) * rows + i] = m[static_cast<size_t>(i) * cols + j];
    return t;
}

void section_matmul(Report &r, const Fixtures &f) {
    HipStream hs;
    const Value &kat = f["mat_mul_3x5x7_scale2"];
    const int M = static_cast<int>(kat.at("M").as_int()), N = static_cast<int>(kat.at("N").as_int()),
              K = static_cast<int>(kat.at("K").as_int());
    const std::vector<float> ha = floats(kat.at("a")), hb = floats(kat.at("b"));
    auto a = DeviceBuffer::from_host(ha);
    auto b = DeviceBuffer::from_host(hb);
    DeviceBuffer c(M * K);
    ops::mat_mul(a.data(), b.data(), c.data(), M, N, K, Scale{2}, hs.s);
    r.near(c.to_host(hs.s), floats(kat.at("out")), "mat_mul epilogue " + kat.at("line").as_string());

    const Value &fused = f["builder_relu_bias"];
    auto bias = DeviceBuffer::from_host(floats(fused.at("bias")));
    MatmulBuilder(a.view(), b.view(), c.view(), M, N, K, hs.s).bias(bias.view()).activation(MatmulActivation::relu).run();
    r.near(c.to_host(hs.s), floats(fused.at("out")), "MatmulBuilder relu(a @ b + bias)");
    auto at = DeviceBuffer::from_host(transposed(ha, M, N));
    auto bt = DeviceBuffer::from_host(transposed(hb, N, K));
    MatmulBuilder(at.view(), bt.view(), c.view(), M, N, K, hs.s)
        .transpose_a()
        .transpose_b()
        .bias(bias.view())
        .activation(MatmulActivation::relu)
        .run();
    r.near(c.to_host(hs.s), floats(fused.at("out")), "MatmulBuilder with both operands transposed");

    const Value &zero = f["mat_mul_zero_inner"];
    ops::mat_mul(nullptr, nullptr, c.data(), static_cast<int>(zero.at("M").as_int()),
                 static_cast<int>(zero.at("N").as_int()), static_cast<int>(zero.at("K").as_int()), ops::PassThrough{},
                 hs.s);
    r.near(c.to_host(hs.s), std::vector<float>(c.size(), static_cast<float>(zero.at("out").as_number())),
           "zero inner dimension " + zero.at("line").as_string());
}

void section_metadata_builders(Report &r, const Fixtures &) {
    auto x = DeviceBuffer::from_host({1, 2, 3, 4});
    DeviceBuffer y(4);
    const int n = ScanBuilder(x.view(), y.view(), 4).op(ScanOp::maximum).inclusive(false).apply([](const auto &sb) {
        return sb.operation() == ScanOp::maximum && !sb.is_inclusive() ? sb.size() : -1;
    });
    r.expect(n == 4, "scan builder fields reach the callback");
    TransformBuilder tb(x.view(), y.view(), 2, 2, TransformOp::transpose);
    r.expect(tb.apply([](const auto &t) { return t.rows() * 10 + t.cols(); }) == 22, "transform builder fields");
    DeviceSpan<const int> no_idx;
    run_contracts(r, {{"scan beyond the buffer", Outcome::rejected, [&] { ScanBuilder(x.view(), y.view(), 5); }},
                      {"transform beyond the buffer", Outcome::rejected,
                       [&] { TransformBuilder(x.view(), y.view(), 3, 2); }},
                      {"gather with too few indices", Outcome::rejected,
                       [&] { GatherScatterBuilder(x.view(), y.view(), no_idx, 2, GatherScatterOp::gather); }}});

    struct RunCase {
        const char *what;
        std::function<void()> run;
        std::vector<float> want;
    };
    auto idx = TypedDeviceBuffer<int>::from_host(std::vector<int>{3, 0, 2, 1});
    const DeviceSpan<const int> ids(idx.data(), 4);
    const std::vector<RunCase> runs = {
        {"inclusive prefix sum", [&] { ScanBuilder(x.view(), y.view(), 4).run(); }, {1, 3, 6, 10}},
        {"exclusive prefix maximum",
         [&] { ScanBuilder(x.view(), y.view(), 4).op(ScanOp::maximum).inclusive(false).run(); },
         {-INFINITY, 1, 2, 3}},
        {"transpose", [&] { TransformBuilder(x.view(), y.view(), 2, 2, TransformOp::transpose).run(); }, {1, 3, 2, 4}},
        {"reshape copies", [&] { TransformBuilder(x.view(), y.view(), 1, 4, TransformOp::reshape).run(); },
         {1, 2, 3, 4}},
        {"gather", [&] { GatherScatterBuilder(x.view(), y.view(), ids, 4, GatherScatterOp::gather).run(); },
         {4, 1, 3, 2}},
        {"scatter", [&] { GatherScatterBuilder(x.view(), y.view(), ids, 4, GatherScatterOp::scatter).run(); },
         {2, 4, 3, 1}},
    };
    for (const RunCase &c : runs) {
        c.run();
        const std::vector<float> got = y.to_host();
        r.expect(got == c.want, c.what);
    }
    const int big_n = 10000;
    auto big = DeviceBuffer::from_host(std::vector<float>(big_n, 1.f));
    DeviceBuffer big_out(big_n);
    DeviceBuffer ws(ops::scan_workspace_size(big_n));
    ScanBuilder(big.view(), big_out.view(), big_n).run(ws.view());
    const std::vector<float> prefix = big_out.to_host();
    bool ok = true;
    for (int i = 0; i < big_n; ++i)
        ok = ok && prefix[static_cast<size_t>(i)] == static_cast<float>(i + 1);
    r.expect(ok, "multi-tile prefix sum with a caller workspace");
}

struct Section {
    const char *name;
    void (*run)(Report &, const Fixtures &);
};

constexpr Section kSections[] = {
    {"translation units", section_translation_units},
    {"ownership", section_ownership},
    {"contracts", section_contracts},
    {"map known answers", section_map_known_answers},
    {"map boundaries", section_map_boundaries},
    {"reductions", section_reductions},
    {"graph replay", section_graph_replay},
    {"launch helpers", section_launch_helpers},
    {"row ops", section_row_ops},
    {"matmul", section_matmul},
    {"metadata builders", section_metadata_builders},
};

} // namespace

int main(int argc, char **argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s <framework_kats.json>\n", argv[0]);
        return 2;
    }
    Fixtures fx;
    try {
        std::ifstream in(argv[1]);
        if (!in)
            throw std::runtime_error(std::string("cannot open ") + argv[1]);
        std::stringstream text;
        text << in.rdbuf();
        fx.root = json::parse(text.str());
    } catch (const std::exception &e) {
        std::fprintf(stderr, "fixture error: %s\n", e.what());
        return 2;
    }
    int devices = 0;
    const hipError_t st = hipGetDeviceCount(&devices);
    if (st == hipErrorNoDevice || st == hipErrorInsufficientDriver || (st == hipSuccess && devices == 0)) {
        std::puts("SKIP: no HIP device");
        return 77;
    }
    OPWORKS_HIP_CHECK(st);

    Report report(1e-5f);
    for (const Section &s : kSections) {
        report.begin(s.name);
        try {
            s.run(report, fx);
        } catch (const std::exception &e) {
            report.expect(false, std::string("unexpected exception: ") + e.what());
        }
    }
    if (!report.failures().empty()) {
        for (const std::string &msg : report.failures())
            std::fprintf(stderr, "FAIL %s\n", msg.c_str());
        return 1;
    }
    std::printf("PASS: %zu sections (", sizeof(kSections) / sizeof(kSections[0]));
    for (size_t i = 0; i < sizeof(kSections) / sizeof(kSections[0]); ++i)
        std::printf("%s%s", i ? ", " : "", kSections[i].name);
    std::puts(")");
    return 0;
}

// Framework self-test of the C++ operator API: ownership and contract rules,
// elementwise boundaries, streams, graph capture/replay, reductions, row ops,
// GEMM and the builders. Restates the checks of the reference's unit test
// (tests/unit/framework.cu:30-214) with its known answers, plus the run()
// additions of the builders. Exit status: 0 pass, 1 fail, 77 no device.
#include <opworks>

#include <cmath>
#include <cstdio>
#include <limits>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

using namespace opworks;

void second_translation_unit();

namespace {

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

// Ownership rules are compile-time facts.
static_assert(!std::is_copy_constructible_v<DeviceBuffer>);
static_assert(std::is_nothrow_move_constructible_v<DeviceBuffer>);
static_assert(std::is_convertible_v<DeviceSpan<float>, DeviceSpan<const float>>);
static_assert(!std::is_convertible_v<DeviceSpan<const float>, DeviceSpan<float>>);
static_assert(std::is_same_v<decltype(std::declval<const DeviceBuffer &>().view().data()), const float *>);
static_assert(!std::is_constructible_v<ElementwiseBuilder, DeviceBuffer &&>);
static_assert(!std::is_constructible_v<ElementwiseBuilder, DeviceBuffer &, DeviceBuffer &&>);
static_assert(!std::is_constructible_v<ElementwiseBuilder, DeviceBuffer &&, DeviceBuffer &>);
static_assert(!std::is_constructible_v<ReductionBuilder, DeviceBuffer &&>);

struct Failure : std::runtime_error {
    using std::runtime_error::runtime_error;
};

std::string g_section;

void expect(bool ok, const std::string &what) {
    if (!ok)
        throw Failure(g_section + ": " + what);
}

void near(float got, float want, const std::string &what, float tol = 1e-5f) {
    const bool ok = std::isfinite(got) && std::fabs(got - want) <= tol * (1 + std::fabs(want));
    if (!ok)
        throw Failure(g_section + ": " + what + " got " + std::to_string(got) + " want " + std::to_string(want));
}

template <typename Fn> void rejects(Fn &&fn, const std::string &what) {
    bool thrown = false;
    try {
        fn();
    } catch (const std::invalid_argument &) {
        thrown = true;
    }
    expect(thrown, "expected invalid_argument: " + what);
}

struct StreamGuard {
    hipStream_t s = nullptr;
    StreamGuard() { OPWORKS_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)); }
    ~StreamGuard() { (void)hipStreamDestroy(s); }
};

__global__ void store_one(float *out, float value) { out[0] = value; }

void ownership_and_contracts() {
    g_section = "ownership_and_contracts";
    DeviceBuffer none(0);
    expect(none.data() == nullptr && none.to_host().empty(), "empty buffer");
    expect(DeviceBuffer::from_host({}).size() == 0, "empty host copy");
    rejects([] { DeviceBuffer bad(-1); }, "negative buffer");
    rejects([] { DeviceSpan<float> bad(nullptr, 1); }, "null span with size");
    rejects([&] { (void)none.to_host_scalar(); }, "scalar of empty buffer");

    auto a = DeviceBuffer::from_host({1, 2, 3});
    auto b = DeviceBuffer::from_host({4, 5, 6});
    auto one = DeviceBuffer::from_host({1});
    rejects([&] { ElementwiseBuilder bad(a, one); }, "length mismatch");
    rejects([&] { (void)ElementwiseBuilder(a).apply<Add>(); }, "binary op on one input");
    rejects([&] { (void)ElementwiseBuilder(a, b).apply<Scale>(); }, "unary op on two inputs");
    rejects([&] { (void)a.to_host_scalar(); }, "scalar of 3 elements");

    const auto added = ElementwiseBuilder(a, b).apply<Add>().to_host();
    for (int i = 0; i < 3; ++i)
        near(added[i], 5.f + 2 * i, "builder add");
    const auto tripled = ElementwiseBuilder(a.view()).apply(Scale{3}).to_host();
    for (int i = 0; i < 3; ++i)
        near(tripled[i], 3.f * (i + 1), "builder scale");
    near(ReductionBuilder(a).apply<Sum>().to_host_scalar(), 6, "builder sum");
    near(ReductionBuilder(none).apply<Product>().to_host_scalar(), 1, "empty product is identity");
    expect(ElementwiseBuilder(none).apply<Scale>().size() == 0, "empty builder output");

    const float *address = a.data();
    const auto borrowed = a.view();
    DeviceBuffer taken(std::move(a));
    expect(a.data() == nullptr && a.size() == 0 && taken.data() == address, "move construction");
    b = std::move(taken);
    expect(taken.data() == nullptr && b.data() == borrowed.data(), "move assignment keeps the address");
    near(b.to_host()[2], 3, "moved contents");

    // Empty launches are no-ops, malformed ones are rejected before the device.
    ops::map(nullptr, nullptr, 0, Scale{});
    ops::softmax(nullptr, nullptr, 0, 3);
    ops::layer_norm(nullptr, nullptr, nullptr, nullptr, 0, 3);
    ops::mat_mul(nullptr, nullptr, nullptr, 0, 4, 5);
    rejects([] { ops::map(nullptr, nullptr, -1, Scale{}); }, "negative map");
    rejects([] { ops::map(nullptr, nullptr, 1, Scale{}); }, "null map");
    rejects([] { ops::reduce<Sum>(nullptr, nullptr, 0); }, "null reduce output");
    rejects([] { ops::softmax(nullptr, nullptr, 1, 0); }, "softmax zero columns");
    rejects([] { ops::softmax(nullptr, nullptr, -1, 2); }, "softmax negative rows");
    rejects([] { ops::layer_norm(nullptr, nullptr, nullptr, nullptr, 1, 0); }, "layer norm zero columns");
    rejects([] { ops::layer_norm(nullptr, nullptr, nullptr, nullptr, 0, 3, 0); }, "layer norm zero eps");
    rejects([] { ops::layer_norm(nullptr, nullptr, nullptr, nullptr, 0, 3, INFINITY); }, "layer norm inf eps");
    rejects([] { ops::mat_mul(nullptr, nullptr, nullptr, 2, 2, 2); }, "null matmul");
    rejects([] { detail::validate_matrix(65536, 65536); }, "matrix over INT_MAX elements");
    expect(detail::blocks_for(std::numeric_limits<int>::max(), 256) == 8388608, "overflow-safe ceil divide");
    expect(num_blocks_for(0) == 0, "empty grid");
}

void elementwise_edges() {
    g_section = "elementwise_edges";
    for (int n : {1, 2, 3, 4, 5, 31, 32, 33, 255, 256, 257, 1025}) {
        for (int shift : {0, 1}) { // shift 1 misaligns every pointer: scalar path
            std::vector<float> h(n + shift);
            for (int i = 0; i < n + shift; ++i)
                h[i] = float(i - 10);
            auto a = DeviceBuffer::from_host(h);
            auto b = DeviceBuffer::from_host(h);
            DeviceBuffer out(n + shift);
            ops::map(a.data() + shift, b.data() + shift, out.data() + shift, n, Add{});
            auto got = out.to_host();
            for (int i = shift; i < n + shift; ++i)
                near(got[i], 2 * h[i], "add n=" + std::to_string(n));
            ops::map(a.data() + shift, a.data() + shift, n, Scale{3}); // exact in-place
            got = a.to_host();
            for (int i = shift; i < n + shift; ++i)
                near(got[i], 3 * h[i], "in-place scale n=" + std::to_string(n));
        }
    }
}

void streams_graphs_reductions() {
    g_section = "streams_graphs_reductions";
    StreamGuard sg;
    hipStream_t s = sg.s;
    auto ones = DeviceBuffer::from_host(std::vector<float>(4099, 1.f), s);
    DeviceBuffer result(1);
    DeviceBuffer ws(ops::reduction_workspace_size(ones.size()));
    // Up to one workgroup chunk (8192 elements) needs no partials; beyond it
    // an empty workspace is a contract violation.
    expect(ops::reduction_workspace_size(ones.size()) == 0, "one chunk needs no workspace");
    auto many = DeviceBuffer::from_host(std::vector<float>(20000, 1.f), s);
    expect(ops::reduction_workspace_size(many.size()) == 3, "partials of 20000 elements");
    rejects([&] { ops::reduce<Sum>(many.data(), result.data(), many.size(), DeviceSpan<float>{}, s); },
            "missing workspace");
    DeviceBuffer ws3(3);
    ops::reduce<Sum>(many.data(), result.data(), many.size(), ws3.view(), s);
    near(result.to_host_scalar(s), 20000, "multi-chunk sum");
    rejects([&] { ops::reduce<Sum>(ones.data(), result.data(), -1, s); }, "negative reduce");
    for (int n : {0, 1, 31, 32, 33, 255, 256, 257, 4099}) {
        ops::reduce<Sum>(ones.data(), result.data(), n, ws.view(), s);
        near(result.to_host_scalar(s), float(n), "workspace sum n=" + std::to_string(n));
        ops::reduce<Sum>(ones.data(), result.data(), n, s);
        near(result.to_host_scalar(s), float(n), "convenience sum n=" + std::to_string(n));
    }
    near(ReductionBuilder(ones).apply<Sum>(ws.view(), s).to_host_scalar(s), 4099, "builder sum on stream");
    near(ElementwiseBuilder(ones).apply(Scale{3}, s).to_host(s).back(), 3, "builder scale on stream");

    // A captured store + in-place doubling + reduction: every replay doubles
    // the input again, so the sums are 2*4099 then 4*4099; nothing inside
    // allocates or synchronizes.
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    OPWORKS_HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
    launch_async(s, store_one, 1, 1, result.data(), -1.f);
    ops::map(ones.data(), ones.data(), ones.size(), Scale{2}, s);
    ops::reduce<Sum>(ones.data(), result.data(), ones.size(), ws.view(), s);
    OPWORKS_HIP_CHECK(hipStreamEndCapture(s, &graph));
    OPWORKS_HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    OPWORKS_HIP_CHECK(hipGraphLaunch(exec, s));
    near(result.to_host_scalar(s), 8198, "first replay");
    OPWORKS_HIP_CHECK(hipGraphLaunch(exec, s));
    near(result.to_host_scalar(s), 16396, "second replay");
    OPWORKS_HIP_CHECK(hipGraphExecDestroy(exec));
    OPWORKS_HIP_CHECK(hipGraphDestroy(graph));

    launch_sync(s, store_one, 1, 1, result.data(), 7.f);
    expect(hipStreamQuery(s) == hipSuccess, "launch_sync leaves the stream idle");
    near(result.to_host_scalar(s), 7, "launch_sync");
    launch(store_one, 1, 1, result.data(), 8.f);
    synchronize();
    near(result.to_host_scalar(), 8, "launch + synchronize");
    launch_sync(store_one, 1, 1, result.data(), 9.f);
    near(result.to_host_scalar(), 9, "launch_sync default stream");
    rejects([&] { launch_async(s, store_one, 0, 1, result.data(), 0.f); }, "zero grid");
}

void rows_and_matmul() {
    g_section = "rows_and_matmul";
    StreamGuard sg;
    hipStream_t s = sg.s;
    auto x = DeviceBuffer::from_host({-2, -1, 0, 1, 2, 3, 4, 5, 6, 7});
    auto gamma = DeviceBuffer::from_host(std::vector<float>(5, 2));
    auto beta = DeviceBuffer::from_host(std::vector<float>(5, 1));
    DeviceBuffer y(10);

    // softmax of (j - 4) for j = 0..4 in both rows (shift invariance).
    float z = 0;
    for (int j = 0; j < 5; ++j)
        z += std::exp(float(j - 4));
    ops::softmax(x.data(), y.data(), 2, 5, s);
    auto got = y.to_host(s);
    for (int i = 0; i < 10; ++i)
        near(got[i], std::exp(float(i % 5 - 4)) / z, "softmax");
    RowwiseBuilder::softmax(x.view(), y.view(), 2, 5, s).run();
    got = y.to_host(s);
    for (int i = 0; i < 10; ++i)
        near(got[i], std::exp(float(i % 5 - 4)) / z, "builder softmax");

    // Each row is {c-2..c+2}: mean c, variance 2.
    ops::layer_norm(x.data(), y.data(), gamma.data(), beta.data(), 2, 5, 1e-5f, s);
    got = y.to_host(s);
    for (int i = 0; i < 10; ++i)
        near(got[i], (i % 5 - 2) * 2.f / std::sqrt(2.f + 1e-5f) + 1, "layer norm");
    RowwiseBuilder::layer_norm(x.view(), y.view(), gamma.view(), beta.view(), 2, 5, 1e-5f, s).run();
    got = y.to_host(s);
    for (int i = 0; i < 10; ++i)
        near(got[i], (i % 5 - 2) * 2.f / std::sqrt(2.f + 1e-5f) + 1, "builder layer norm");

    // rms_norm: out = x * w / sqrt(mean(x^2) + eps), here with w = 2.
    RowwiseBuilder::rms_norm(x.view(), y.view(), gamma.view(), 2, 5, 1e-5f, s).run();
    got = y.to_host(s);
    const float ms0 = (4 + 1 + 0 + 1 + 4) / 5.f, ms1 = (9 + 16 + 25 + 36 + 49) / 5.f;
    for (int i = 0; i < 10; ++i) {
        const float xi = float(i - 2);
        near(got[i], xi * 2.f / std::sqrt((i < 5 ? ms0 : ms1) + 1e-5f), "builder rms norm");
    }
    rejects([&] { RowwiseBuilder::rms_norm(x.view(), y.view(), gamma.view(), 2, 5, NAN, s); }, "nan eps");
    rejects([&] { RowwiseBuilder::softmax(x.view(), y.view(), 3, 5, s); }, "rows beyond buffer");

    // 3x5 times 5x7 on small integers is exact in fp32.
    std::vector<float> ha(15), hb(35);
    for (int i = 0; i < 15; ++i)
        ha[i] = float(i % 7 - 3);
    for (int i = 0; i < 35; ++i)
        hb[i] = float(i % 5 - 2);
    auto a = DeviceBuffer::from_host(ha);
    auto b = DeviceBuffer::from_host(hb);
    auto bias = DeviceBuffer::from_host({-3, -2, -1, 0, 1, 2, 3});
    DeviceBuffer c(21);
    auto dot = [&](int r, int col) {
        float acc = 0;
        for (int k = 0; k < 5; ++k)
            acc += ha[r * 5 + k] * hb[k * 7 + col];
        return acc;
    };
    ops::mat_mul(a.data(), b.data(), c.data(), 3, 5, 7, Scale{2}, s);
    got = c.to_host(s);
    for (int r = 0; r < 3; ++r)
        for (int col = 0; col < 7; ++col)
            near(got[r * 7 + col], 2 * dot(r, col), "mat_mul epilogue");
    MatmulBuilder(a.view(), b.view(), c.view(), 3, 5, 7, s)
        .bias(bias.view())
        .activation(MatmulActivation::relu)
        .run();
    got = c.to_host(s);
    const auto hbias = bias.to_host();
    for (int r = 0; r < 3; ++r)
        for (int col = 0; col < 7; ++col)
            near(got[r * 7 + col], std::fmax(dot(r, col) + hbias[col], 0.f), "builder relu(a@b+bias)");
    ops::mat_mul(nullptr, nullptr, c.data(), 3, 0, 7, ops::PassThrough{}, s);
    for (float v : c.to_host(s))
        near(v, 0, "zero inner dimension");
}

void metadata_builders() {
    g_section = "metadata_builders";
    auto x = DeviceBuffer::from_host({1, 2, 3, 4});
    DeviceBuffer y(4);
    const int n = ScanBuilder(x.view(), y.view(), 4).op(ScanOp::maximum).inclusive(false).apply([](const auto &sb) {
        return sb.operation() == ScanOp::maximum && !sb.is_inclusive() ? sb.size() : -1;
    });
    expect(n == 4, "scan builder fields");
    rejects([&] { ScanBuilder(x.view(), y.view(), 5); }, "scan beyond buffer");
    TransformBuilder tb(x.view(), y.view(), 2, 2, TransformOp::transpose);
    expect(tb.apply([](const auto &t) { return t.rows() * 10 + t.cols(); }) == 22, "transform builder fields");
    rejects([&] { TransformBuilder(x.view(), y.view(), 3, 2); }, "transform beyond buffer");
    DeviceSpan<const int> no_idx;
    rejects([&] { GatherScatterBuilder(x.view(), y.view(), no_idx, 2, GatherScatterOp::gather); }, "short indices");

    // run(): the kernels this build adds behind the callback boundary
    auto expect_y = [&](std::initializer_list<float> want, const char *what) {
        const auto got = y.to_host();
        int i = 0;
        for (float w : want)
            expect(got[i++] == w, what);
    };
    ScanBuilder(x.view(), y.view(), 4).run();
    expect_y({1, 3, 6, 10}, "inclusive prefix sum");
    ScanBuilder(x.view(), y.view(), 4).op(ScanOp::maximum).inclusive(false).run();
    expect_y({-INFINITY, 1, 2, 3}, "exclusive prefix maximum");
    TransformBuilder(x.view(), y.view(), 2, 2, TransformOp::transpose).run();
    expect_y({1, 3, 2, 4}, "transpose");
    TransformBuilder(x.view(), y.view(), 1, 4, TransformOp::reshape).run();
    expect_y({1, 2, 3, 4}, "reshape copies");
    auto idx = TypedDeviceBuffer<int>::from_host(std::vector<int>{3, 0, 2, 1});
    GatherScatterBuilder(x.view(), y.view(), DeviceSpan<const int>(idx.data(), 4), 4, GatherScatterOp::gather).run();
    expect_y({4, 1, 3, 2}, "gather");
    GatherScatterBuilder(x.view(), y.view(), DeviceSpan<const int>(idx.data(), 4), 4, GatherScatterOp::scatter).run();
    expect_y({2, 4, 3, 1}, "scatter");
    auto big = DeviceBuffer::from_host(std::vector<float>(10000, 1.f));
    DeviceBuffer big_out(10000);
    DeviceBuffer ws(ops::scan_workspace_size(10000));
    ScanBuilder(big.view(), big_out.view(), 10000).run(ws.view());
    const auto prefix = big_out.to_host();
    for (int i = 0; i < 10000; i += 999)
        expect(prefix[i] == float(i + 1), "multi-tile prefix sum with a caller workspace");
}

} // namespace

int main() {
    int devices = 0;
    const hipError_t st = hipGetDeviceCount(&devices);
    if (st == hipErrorNoDevice || st == hipErrorInsufficientDriver || (st == hipSuccess && devices == 0)) {
        std::puts("SKIP: no HIP device");
        return 77;
    }
    OPWORKS_HIP_CHECK(st);
    try {
        second_translation_unit();
        ownership_and_contracts();
        elementwise_edges();
        streams_graphs_reductions();
        rows_and_matmul();
        metadata_builders();
    } catch (const std::exception &e) {
        std::fprintf(stderr, "FAIL: %s\n", e.what());
        return 1;
    }
    std::puts("PASS: contracts, ownership, boundaries, streams, graph replay, reduction, row ops, matmul, builders, "
              "multi-TU");
    return 0;
}

// Fixed cost of a kernel on this part and the rate of plain streams, the two
// terms of t = c + bytes / r that bound every HBM-streaming op here.
//
// Each case is captured 16 or 80 times in one HIP graph and the graph is
// replayed; the figure is the replay time divided by the kernels it holds, so
// host launch cost is excluded (eager back-to-back launches are timed too).
// Streams rotate over a 1 GiB buffer, four times the 256 MB Infinity Cache.
//   * empty / one store per workgroup / a dependent load + store per workgroup;
//   * read-only streams (16-byte non-temporal loads, grid-stride, 2048 x 256
//     lanes) of 16, 64, 134 and 256 MiB;
//   * copies (read + write) of 16, 64 and 256 MiB.
// The fitted line reported at the end is the least-squares fit of the stream
// times against their bytes.
//
//   launch_floor            prints one line per case and two fits

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(call)                                                                                                    \
    do {                                                                                                               \
        hipError_t e_ = (call);                                                                                        \
        if (e_ != hipSuccess) {                                                                                        \
            std::fprintf(stderr, "HIP error %s at line %d: %s\n", #call, __LINE__, hipGetErrorString(e_));            \
            std::exit(1);                                                                                              \
        }                                                                                                              \
    } while (0)

namespace {

using f32x4 = float __attribute__((ext_vector_type(4)));

__global__ void empty_kernel() {}

__global__ void store_kernel(float *p) {
    if (threadIdx.x == 0)
        p[blockIdx.x * 64] += 1.f;
}

__global__ void dependent_kernel(const float *in, float *out) {
    if (threadIdx.x == 0)
        out[blockIdx.x * 64] = in[blockIdx.x * 64] + 1.f;
}

__global__ __launch_bounds__(256) void read_kernel(const f32x4 *in, float *sink, long n4) {
    float acc = 0.f;
    for (long i = blockIdx.x * 256L + threadIdx.x; i < n4; i += static_cast<long>(gridDim.x) * 256) {
        const f32x4 v = __builtin_nontemporal_load(in + i);
        acc += (v[0] + v[1]) + (v[2] + v[3]);
    }
    if (acc == 1234.5f) // never true for the zero-filled input: keeps the loads alive
        sink[0] = acc;
}

__global__ __launch_bounds__(256) void copy_kernel(const f32x4 *in, f32x4 *out, long n4) {
    for (long i = blockIdx.x * 256L + threadIdx.x; i < n4; i += static_cast<long>(gridDim.x) * 256)
        __builtin_nontemporal_store(__builtin_nontemporal_load(in + i), out + i);
}

struct Fit {
    std::vector<double> bytes, us;
    void add(double b, double t) {
        bytes.push_back(b);
        us.push_back(t);
    }
    void report(const char *what) const {
        const double n = static_cast<double>(bytes.size());
        double sb = 0, st = 0, sbb = 0, sbt = 0;
        for (size_t i = 0; i < bytes.size(); ++i) {
            sb += bytes[i];
            st += us[i];
            sbb += bytes[i] * bytes[i];
            sbt += bytes[i] * us[i];
        }
        const double slope = (n * sbt - sb * st) / (n * sbb - sb * sb); // us per byte
        const double c = (st - slope * sb) / n;
        std::printf("fit %-6s t = %.2f us + bytes / %.0f GB/s\n", what, c, 1e-3 / slope);
    }
};

} // namespace

int main() {
    hipStream_t s;
    CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    constexpr long kBig = 1L << 30;
    float *small = nullptr, *big = nullptr, *dst = nullptr;
    CHECK(hipMalloc(&small, 64 << 20));
    CHECK(hipMemset(small, 0, 64 << 20));
    CHECK(hipMalloc(&big, kBig));
    CHECK(hipMemset(big, 0, kBig));
    CHECK(hipMalloc(&dst, kBig));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));

    auto eager = [&](const char *name, auto launch, int n) {
        for (int i = 0; i < 50; ++i)
            launch(i);
        CHECK(hipEventRecord(e0, s));
        for (int i = 0; i < n; ++i)
            launch(i);
        CHECK(hipEventRecord(e1, s));
        CHECK(hipEventSynchronize(e1));
        float ms = 0;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        std::printf("eager %-36s %9.3f us per kernel\n", name, 1e3 * ms / n);
    };
    auto graph = [&](const char *name, auto launch, int per_graph, int reps) {
        hipGraph_t g;
        hipGraphExec_t ge;
        CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        for (int i = 0; i < per_graph; ++i)
            launch(i);
        CHECK(hipStreamEndCapture(s, &g));
        CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        for (int i = 0; i < 5; ++i)
            CHECK(hipGraphLaunch(ge, s));
        CHECK(hipEventRecord(e0, s));
        for (int i = 0; i < reps; ++i)
            CHECK(hipGraphLaunch(ge, s));
        CHECK(hipEventRecord(e1, s));
        CHECK(hipEventSynchronize(e1));
        float ms = 0;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        CHECK(hipGraphExecDestroy(ge));
        CHECK(hipGraphDestroy(g));
        const double us = 1e3 * ms / (reps * per_graph);
        std::printf("graph %-36s %9.3f us per kernel\n", name, us);
        return us;
    };

    // queue a few long kernels first, so the host is never what the eager figures measure
    for (int i = 0; i < 20; ++i)
        read_kernel<<<1024, 256, 0, s>>>(reinterpret_cast<const f32x4 *>(big), small, kBig / 16);
    eager("empty, 1 workgroup", [&](int) { empty_kernel<<<1, 64, 0, s>>>(); }, 2000);
    eager("one store per workgroup, 2048 wg", [&](int) { store_kernel<<<2048, 256, 0, s>>>(small); }, 2000);
    graph("empty, 1 workgroup", [&](int) { empty_kernel<<<1, 64, 0, s>>>(); }, 80, 50);
    graph("one store per workgroup, 256 wg", [&](int) { store_kernel<<<256, 256, 0, s>>>(small); }, 80, 50);
    graph("one store per workgroup, 2048 wg", [&](int) { store_kernel<<<2048, 256, 0, s>>>(small); }, 80, 50);
    graph("dependent load + store, 512 wg", [&](int i) {
        float *a = small + (i & 1) * (1 << 20), *b = small + ((i + 1) & 1) * (1 << 20);
        dependent_kernel<<<512, 64, 0, s>>>(a, b);
    }, 80, 50);

    Fit reads, copies;
    char name[64];
    for (long mib : {16L, 64L, 134L, 256L}) {
        const long n4 = mib * (1L << 20) / 16, total4 = kBig / 16;
        std::snprintf(name, sizeof name, "read %ld MiB", mib);
        const double us = graph(name, [&](int i) {
            const long off = (static_cast<long>(i) * n4) % (total4 - n4);
            read_kernel<<<2048, 256, 0, s>>>(reinterpret_cast<const f32x4 *>(big) + off, small, n4);
        }, 16, 20);
        reads.add(static_cast<double>(mib << 20), us);
    }
    for (long mib : {16L, 64L, 256L}) { // bytes moved = 2 x mib
        const long n4 = mib * (1L << 20) / 16, total4 = kBig / 16;
        std::snprintf(name, sizeof name, "copy %ld MiB (read + write)", mib);
        const double us = graph(name, [&](int i) {
            const long off = (static_cast<long>(i) * n4) % (total4 - n4);
            copy_kernel<<<2048, 256, 0, s>>>(reinterpret_cast<const f32x4 *>(big) + off,
                                             reinterpret_cast<f32x4 *>(dst) + off, n4);
        }, 16, 20);
        copies.add(static_cast<double>(2 * (mib << 20)), us);
    }
    reads.report("read");
    copies.report("copy");
    return 0;
}

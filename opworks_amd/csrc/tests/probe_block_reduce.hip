// Test library: a user kernel that calls the public workgroup reductions
// block_reduce<Op> / block_reduce_all<Op> (reference contract: a 1-D
// workgroup whose size is a positive multiple of 32, every thread taking
// part; include/core/block_reduce.cuh:9-41, README.md:228-229). Each
// workgroup reduces its own slice of `in`; the functors are user-defined in
// the reference's shape (static identity() and combine()).
//
//   mode 0: block_reduce       out[block]              = the workgroup's result (thread 0)
//   mode 1: block_reduce_all   out[block * nt + t]     = the result every thread sees
//   mode 2: two block_reduce_all calls in a row on the same values; out as in
//           mode 1 holds the second call's result when both agree, NaN otherwise
#include <opworks>

#include <cmath>
#include <cstdio>

namespace {

struct UserSum {
    static __device__ float identity() { return 0.f; }
    static __device__ float combine(float a, float b) { return a + b; }
};
struct UserMax {
    static __device__ float identity() { return -INFINITY; }
    static __device__ float combine(float a, float b) { return fmaxf(a, b); }
};
struct UserProduct {
    static __device__ float identity() { return 1.f; }
    static __device__ float combine(float a, float b) { return a * b; }
};

template <typename Op, int kMode> __global__ void user_reduce_kernel(const float *in, float *out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const float v = in[i];
    if constexpr (kMode == 0) {
        const float r = opworks::block_reduce<Op>(v);
        if (threadIdx.x == 0)
            out[blockIdx.x] = r;
    } else if constexpr (kMode == 1) {
        out[i] = opworks::block_reduce_all<Op>(v);
    } else {
        const float first = opworks::block_reduce_all<Op>(v);
        const float second = opworks::block_reduce_all<Op>(v);
        out[i] = first == second ? second : NAN;
    }
}

template <typename Op> void launch_mode(const float *in, float *out, int nthreads, int nblocks, int mode) {
    if (mode == 0)
        opworks::launch_sync(user_reduce_kernel<Op, 0>, nblocks, nthreads, in, out);
    else if (mode == 1)
        opworks::launch_sync(user_reduce_kernel<Op, 1>, nblocks, nthreads, in, out);
    else
        opworks::launch_sync(user_reduce_kernel<Op, 2>, nblocks, nthreads, in, out);
}

} // namespace

extern "C" {

// op: 0 sum, 1 max, 2 product. Returns 0, or -1 for arguments outside the
// contract (nothing is launched then).
int probe_block_reduce(const float *in, float *out, int nthreads, int nblocks, int op, int mode) {
    if (!in || !out || nthreads < 32 || nthreads > 1024 || nthreads % 32 != 0 || nblocks < 1 || op < 0 || op > 2 ||
        mode < 0 || mode > 2) {
        std::fprintf(stderr, "probe_block_reduce: arguments outside the contract\n");
        return -1;
    }
    if (op == 0)
        launch_mode<UserSum>(in, out, nthreads, nblocks, mode);
    else if (op == 1)
        launch_mode<UserMax>(in, out, nthreads, nblocks, mode);
    else
        launch_mode<UserProduct>(in, out, nthreads, nblocks, mode);
    return 0;
}

} // extern "C"

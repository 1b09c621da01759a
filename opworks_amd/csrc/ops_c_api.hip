// extern "C" operator surface of libopworks_amd.so (declared in
// include/opworks_ops.h). Each entry point validates through the same
// opworks::ops function a C++ caller would use, then enqueues.

#include <hip/hip_runtime.h>

#include "../include/core/random.hpp"
#include "../include/ops/argmax.hpp"
#include "../include/ops/elementwise.hpp"
#include "../include/ops/gather_scatter.hpp"
#include "../include/ops/heads.hpp"
#include "../include/ops/layer_norm.hpp"
#include "../include/ops/model_pointwise.hpp"
#include "../include/ops/reduction.hpp"
#include "../include/ops/rms_norm.hpp"
#include "../include/ops/rope.hpp"
#include "../include/ops/scan.hpp"
#include "../include/ops/softmax.hpp"
#include "../include/ops/transform.hpp"
#include "c_api_common.hpp"

using opworks::capi::guard;

namespace {

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

struct ScaleAdd {
    float alpha;
    __device__ float operator()(float a, float b) const { return fmaf(alpha, a, b); }
};
struct Add {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct Scale {
    float factor;
    __device__ float operator()(float x) const { return factor * x; }
};
struct Relu {
    __device__ float operator()(float x) const { return fmaxf(x, 0.f); }
};
struct Sum {
    static __device__ float identity() { return 0.f; }
    static __device__ float combine(float a, float b) { return a + b; }
};
struct Max {
    static __device__ float identity() { return -INFINITY; }
    static __device__ float combine(float a, float b) { return fmaxf(a, b); }
};
struct Product {
    static __device__ float identity() { return 1.f; }
    static __device__ float combine(float a, float b) { return a * b; }
};

__global__ void __launch_bounds__(256) fill_uniform_kernel(float *dst, int64_t n, uint64_t key, float lo, float hi) {
    OPWORKS_GRID_LOOP(i, n) { dst[i] = opworks::rng::uniform(key, static_cast<uint64_t>(i), lo, hi); }
}
__global__ void __launch_bounds__(256) fill_normal_kernel(float *dst, int64_t n, uint64_t key, float mean, float sd) {
    OPWORKS_GRID_LOOP(i, n) { dst[i] = opworks::rng::normal(key, static_cast<uint64_t>(i), mean, sd); }
}

int fill_grid(int64_t n) {
    const int64_t cap = static_cast<int64_t>(opworks::detail::cu_count()) * 16;
    const int64_t need = opworks::detail::blocks_for64(n, 256);
    return static_cast<int>(need < cap ? need : cap);
}

template <typename Op> void reduce_dispatch(const float *in, float *out, int n, float *ws, int ws_size, hipStream_t s) {
    if (ws)
        opworks::ops::reduce<Op>(in, out, n, opworks::DeviceSpan<float>(ws, ws_size), s);
    else
        opworks::ops::reduce<Op>(in, out, n, s);
}

} // namespace

extern "C" {

const char *opw_last_error(void) { return opworks::capi::last_error().c_str(); }

int opw_device_count(int *count) {
    return guard([&] {
        opworks::detail::require(count != nullptr, "null count pointer");
        OPWORKS_HIP_CHECK(hipGetDeviceCount(count));
        return 0;
    });
}

int opw_set_device(int device) {
    return guard([&] {
        OPWORKS_HIP_CHECK(hipSetDevice(device));
        return 0;
    });
}

int opw_device_name(char *out, int out_len) {
    return guard([&] {
        opworks::detail::require(out != nullptr && out_len > 0, "null name buffer");
        int dev = 0;
        OPWORKS_HIP_CHECK(hipGetDevice(&dev));
        hipDeviceProp_t prop;
        OPWORKS_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
        // some driver stacks leave the marketing name empty: then the architecture and CU count name it
        if (prop.name[0] != '\0')
            std::snprintf(out, static_cast<size_t>(out_len), "%s (%s)", prop.name, prop.gcnArchName);
        else
            std::snprintf(out, static_cast<size_t>(out_len), "%s, %d CUs", prop.gcnArchName, prop.multiProcessorCount);
        return 0;
    });
}

int opw_device_cu_count(int *cus) {
    return guard([&] {
        opworks::detail::require(cus != nullptr, "null pointer");
        *cus = opworks::detail::cu_count();
        return 0;
    });
}

int opw_malloc(void **ptr, size_t bytes) {
    return guard([&] {
        opworks::detail::require(ptr != nullptr, "null output pointer");
        *ptr = nullptr;
        if (bytes)
            OPWORKS_HIP_CHECK(hipMalloc(ptr, bytes));
        return 0;
    });
}

int opw_free(void *ptr) {
    return guard([&] {
        if (ptr) {
            // Blocking, like the reference DeviceBuffer's cudaFree: queued work may still read ptr.
            OPWORKS_HIP_CHECK(hipDeviceSynchronize());
            OPWORKS_HIP_CHECK(hipFree(ptr));
        }
        return 0;
    });
}

int opw_memcpy_htod(void *dst, const void *src, size_t bytes, void *stream) {
    return guard([&] {
        opworks::detail::require(bytes == 0 || (dst && src), "null copy pointer");
        if (bytes) {
            OPWORKS_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
            opworks::synchronize(as_stream(stream));
        }
        return 0;
    });
}

int opw_memcpy_dtoh(void *dst, const void *src, size_t bytes, void *stream) {
    return guard([&] {
        opworks::detail::require(bytes == 0 || (dst && src), "null copy pointer");
        if (bytes) {
            OPWORKS_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
            opworks::synchronize(as_stream(stream));
        }
        return 0;
    });
}

int opw_memcpy_dtod(void *dst, const void *src, size_t bytes, void *stream) {
    return guard([&] {
        opworks::detail::require(bytes == 0 || (dst && src), "null copy pointer");
        if (bytes)
            OPWORKS_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
        return 0;
    });
}

int opw_memset(void *dst, int value, size_t bytes, void *stream) {
    return guard([&] {
        opworks::detail::require(bytes == 0 || dst, "null memset pointer");
        if (bytes)
            OPWORKS_HIP_CHECK(hipMemsetAsync(dst, value, bytes, as_stream(stream)));
        return 0;
    });
}

int opw_stream_create(void **stream) {
    return guard([&] {
        opworks::detail::require(stream != nullptr, "null stream pointer");
        hipStream_t s;
        OPWORKS_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        *stream = s;
        return 0;
    });
}

int opw_stream_destroy(void *stream) {
    return guard([&] {
        if (stream)
            OPWORKS_HIP_CHECK(hipStreamDestroy(as_stream(stream)));
        return 0;
    });
}

int opw_stream_synchronize(void *stream) {
    return guard([&] {
        opworks::synchronize(as_stream(stream));
        return 0;
    });
}

int opw_device_synchronize(void) {
    return guard([&] {
        OPWORKS_HIP_CHECK(hipDeviceSynchronize());
        return 0;
    });
}

// Graph capture of the work enqueued on one library stream, in global mode as the reference's
// framework test captures (tests/unit/framework.cu:154-169): a capture-unsafe call such as a
// blocking allocation or a synchronization while it is open invalidates it. A capture that the
// runtime refuses comes back as -1 with the runtime's message instead of aborting.
static void capture_check(hipError_t st, const char *what) {
    if (st != hipSuccess)
        throw std::runtime_error(std::string(what) + " failed: " + hipGetErrorString(st));
}

int opw_graph_capture_begin(void *stream) {
    return guard([&] {
        opworks::detail::require(stream != nullptr, "graph capture needs a created stream, not the null stream");
        capture_check(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeGlobal),
                      "hipStreamBeginCapture");
        return 0;
    });
}

int opw_graph_capture_end(void *stream, void **graph_exec) {
    return guard([&] {
        opworks::detail::require(stream != nullptr && graph_exec != nullptr, "null stream or graph pointer");
        hipGraph_t graph = nullptr;
        capture_check(hipStreamEndCapture(as_stream(stream), &graph), "hipStreamEndCapture");
        hipGraphExec_t exec = nullptr;
        const hipError_t st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        OPWORKS_HIP_CHECK(hipGraphDestroy(graph));
        capture_check(st, "hipGraphInstantiate");
        *graph_exec = exec;
        return 0;
    });
}

int opw_graph_launch(void *graph_exec, void *stream) {
    return guard([&] {
        opworks::detail::require(graph_exec != nullptr, "null graph");
        OPWORKS_HIP_CHECK(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)));
        return 0;
    });
}

int opw_graph_destroy(void *graph_exec) {
    return guard([&] {
        if (graph_exec)
            OPWORKS_HIP_CHECK(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)));
        return 0;
    });
}

int opw_event_create(void **event) {
    return guard([&] {
        opworks::detail::require(event != nullptr, "null event pointer");
        hipEvent_t e;
        OPWORKS_HIP_CHECK(hipEventCreate(&e));
        *event = e;
        return 0;
    });
}

int opw_event_destroy(void *event) {
    return guard([&] {
        if (event)
            OPWORKS_HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(event)));
        return 0;
    });
}

int opw_event_record(void *event, void *stream) {
    return guard([&] {
        opworks::detail::require(event != nullptr, "null event");
        OPWORKS_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)));
        return 0;
    });
}

int opw_event_synchronize(void *event) {
    return guard([&] {
        opworks::detail::require(event != nullptr, "null event");
        OPWORKS_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(event)));
        return 0;
    });
}

int opw_event_elapsed_ms(void *start, void *stop, float *ms) {
    return guard([&] {
        opworks::detail::require(start && stop && ms, "null event or output");
        OPWORKS_HIP_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
        return 0;
    });
}

int opw_fill_uniform_f32(float *dst, int64_t n, uint64_t seed, uint64_t stream_id, float lo, float hi, void *stream) {
    return guard([&] {
        opworks::detail::require(n >= 0 && (n == 0 || dst), "fill requires a buffer and a nonnegative size");
        if (n)
            opworks::launch_async(as_stream(stream), fill_uniform_kernel, fill_grid(n), 256, dst, n,
                                  opworks::rng::stream_key(seed, stream_id), lo, hi);
        return 0;
    });
}

int opw_fill_normal_f32(float *dst, int64_t n, uint64_t seed, uint64_t stream_id, float mean, float stddev,
                        void *stream) {
    return guard([&] {
        opworks::detail::require(n >= 0 && (n == 0 || dst), "fill requires a buffer and a nonnegative size");
        if (n)
            opworks::launch_async(as_stream(stream), fill_normal_kernel, fill_grid(n), 256, dst, n,
                                  opworks::rng::stream_key(seed, stream_id), mean, stddev);
        return 0;
    });
}

int opw_map_scale_add_f32(const float *a, const float *b, float *out, int n, float alpha, void *stream) {
    return guard([&] {
        opworks::ops::map(a, b, out, n, ScaleAdd{alpha}, as_stream(stream));
        return 0;
    });
}

int opw_map_add_f32(const float *a, const float *b, float *out, int n, void *stream) {
    return guard([&] {
        opworks::ops::map(a, b, out, n, Add{}, as_stream(stream));
        return 0;
    });
}

int opw_map_scale_f32(const float *in, float *out, int n, float factor, void *stream) {
    return guard([&] {
        opworks::ops::map(in, out, n, Scale{factor}, as_stream(stream));
        return 0;
    });
}

int opw_map_relu_f32(const float *in, float *out, int n, void *stream) {
    return guard([&] {
        opworks::ops::map(in, out, n, Relu{}, as_stream(stream));
        return 0;
    });
}

int opw_reduction_workspace_size(int n) {
    return guard([&] { return opworks::ops::reduction_workspace_size(n); });
}

int opw_reduce_f32(const float *in, float *out, int n, int op, float *workspace, int workspace_size, void *stream) {
    return guard([&] {
        hipStream_t s = as_stream(stream);
        switch (op) {
        case 0: reduce_dispatch<Sum>(in, out, n, workspace, workspace_size, s); break;
        case 1: reduce_dispatch<Max>(in, out, n, workspace, workspace_size, s); break;
        case 2: reduce_dispatch<Product>(in, out, n, workspace, workspace_size, s); break;
        default: throw std::invalid_argument("unknown reduction op (0 sum, 1 max, 2 product)");
        }
        return 0;
    });
}

int opw_softmax_f32(const float *in, float *out, int rows, int cols, void *stream) {
    return guard([&] {
        opworks::ops::softmax(in, out, rows, cols, as_stream(stream));
        return 0;
    });
}

int opw_layer_norm_f32(const float *in, float *out, const float *gamma, const float *beta, int rows, int cols,
                       float eps, void *stream) {
    return guard([&] {
        opworks::ops::layer_norm(in, out, gamma, beta, rows, cols, eps, as_stream(stream));
        return 0;
    });
}

int opw_rms_norm_f32(const float *x, const float *weight, float *out, int rows, int cols, float eps, void *stream) {
    return guard([&] {
        opworks::ops::rms_norm(x, weight, out, rows, cols, eps, as_stream(stream));
        return 0;
    });
}

int opw_add_f32(const float *a, const float *b, float *out, long long n, void *stream) {
    return guard([&] {
        opworks::ops::add(a, b, out, n, as_stream(stream));
        return 0;
    });
}

int opw_swiglu_f32(const float *gate, const float *up, float *out, long long n, void *stream) {
    return guard([&] {
        opworks::ops::swiglu(gate, up, out, n, as_stream(stream));
        return 0;
    });
}

int opw_causal_scale_f32(float *scores, int rows, int cols, float scale, void *stream) {
    return guard([&] {
        opworks::ops::causal_scale(scores, rows, cols, scale, as_stream(stream));
        return 0;
    });
}

int opw_embedding_f32(const float *table, long long vocab, const int *ids, float *out, int n, int hidden,
                      void *stream) {
    return guard([&] {
        opworks::detail::require(vocab > 0, "embedding vocab must be positive");
        opworks::ops::embedding(table, ids, out, n, hidden, as_stream(stream), vocab);
        return 0;
    });
}

int opw_embedding_bf16(const uint16_t *table, long long vocab, const int *ids, float *out, int n, int hidden,
                       void *stream) {
    return guard([&] {
        opworks::detail::require(vocab > 0, "embedding vocab must be positive");
        opworks::ops::embedding(reinterpret_cast<const opworks::bf16 *>(table), ids, out, n, hidden,
                                as_stream(stream), vocab);
        return 0;
    });
}

int opw_split_heads_f32(const float *in, float *out, int rows, int heads, int head_dim, int out_row_stride,
                        int out_row_offset, void *stream) {
    return guard([&] {
        opworks::ops::split_heads(in, out, rows, heads, head_dim, out_row_stride, out_row_offset, as_stream(stream));
        return 0;
    });
}

int opw_merge_heads_f32(const float *in, float *out, int rows, int heads, int head_dim, int in_row_stride,
                        int in_row_offset, void *stream) {
    return guard([&] {
        opworks::ops::merge_heads(in, out, rows, heads, head_dim, in_row_stride, in_row_offset, as_stream(stream));
        return 0;
    });
}

int opw_rope_f32(float *x, const float *inv_freq, int rows, int heads, int head_dim, int pos_start, void *stream) {
    return guard([&] {
        opworks::ops::rope(x, inv_freq, rows, heads, head_dim, pos_start, as_stream(stream));
        return 0;
    });
}

int opw_argmax_f32(const float *x, int n, int *out, void *stream) {
    return guard([&] {
        opworks::ops::argmax(x, n, out, as_stream(stream));
        return 0;
    });
}

int opw_scan_workspace_size(int n) {
    return guard([&] { return opworks::ops::scan_workspace_size(n); });
}

int opw_scan_f32(const float *in, float *out, int n, int op, int inclusive, float *workspace, int workspace_size,
                 void *stream) {
    return guard([&] {
        if (op != 0 && op != 1)
            throw std::invalid_argument("unknown scan op (0 sum, 1 maximum)");
        hipStream_t s = as_stream(stream);
        if (workspace)
            opworks::ops::scan(in, out, n, op == 1, inclusive != 0, opworks::DeviceSpan<float>(workspace, workspace_size),
                               s);
        else
            opworks::ops::scan(in, out, n, op == 1, inclusive != 0, s);
        return 0;
    });
}

int opw_transpose_f32(const float *in, float *out, int rows, int cols, void *stream) {
    return guard([&] {
        opworks::ops::transpose(in, out, rows, cols, as_stream(stream));
        return 0;
    });
}

int opw_copy_f32(const float *in, float *out, int n, void *stream) {
    return guard([&] {
        opworks::ops::copy(in, out, n, as_stream(stream));
        return 0;
    });
}

int opw_gather_f32(const float *in, long long in_size, const int *idx, float *out, int count, void *stream) {
    return guard([&] {
        opworks::ops::gather(in, in_size, idx, out, count, as_stream(stream));
        return 0;
    });
}

int opw_scatter_f32(const float *in, const int *idx, float *out, long long out_size, int count, void *stream) {
    return guard([&] {
        opworks::ops::scatter(in, idx, out, out_size, count, as_stream(stream));
        return 0;
    });
}

} // extern "C"

/* C ABI of libopworks_amd.so: the fixed-function operators of the OpWorks hot
 * path, plus the device-memory, stream and event plumbing a host without HIP
 * headers (ctypes, cgo, JNI) needs to drive them.
 *
 * Conventions (all functions):
 *  - plain pointers and sizes; `stream` is a hipStream_t passed as void*
 *    (NULL = the legacy default stream, as in the reference's C++ API);
 *  - operator entry points enqueue asynchronously and return 0, or -1 after a
 *    contract violation (the reference throws std::invalid_argument there:
 *    include/core/cuda_utils.cuh:29-49); the message is then available from
 *    opw_last_error() on the calling thread. No C++ exception crosses the ABI.
 *  - HIP runtime failures abort the process, as OPWORKS_CUDA_CHECK does in the
 *    reference (include/core/cuda_utils.cuh:13-21).
 *  - sizes follow the reference: nonnegative int, at most INT_MAX elements.
 */
#ifndef OPWORKS_OPS_H
#define OPWORKS_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call on this thread ("" if none). */
const char *opw_last_error(void);

/* ---- device plumbing (reference: include/core/device_buffer.cuh:12-67) ---- */
int opw_device_count(int *count);
int opw_set_device(int device);
int opw_device_name(char *out, int out_len);
int opw_device_cu_count(int *cus);
int opw_malloc(void **ptr, size_t bytes);
/* Waits for the device, then frees (blocking like the reference DeviceBuffer destructor). */
int opw_free(void *ptr);
/* Blocking copies on `stream` (DeviceBuffer::from_host / to_host semantics). */
int opw_memcpy_htod(void *dst, const void *src, size_t bytes, void *stream);
int opw_memcpy_dtoh(void *dst, const void *src, size_t bytes, void *stream);
int opw_memcpy_dtod(void *dst, const void *src, size_t bytes, void *stream);
int opw_memset(void *dst, int value, size_t bytes, void *stream);
int opw_stream_create(void **stream);
int opw_stream_destroy(void *stream);
/* reference: synchronize(stream), include/core/cuda_utils.cuh:100-102 */
int opw_stream_synchronize(void *stream);
int opw_device_synchronize(void);
int opw_event_create(void **event);
int opw_event_destroy(void *event);
int opw_event_record(void *event, void *stream);
int opw_event_synchronize(void *event);
int opw_event_elapsed_ms(void *start, void *stop, float *ms);
/* HIP graph capture (global mode) of what is enqueued on `stream` (a created stream, not NULL)
 * between begin and end; end instantiates it into *graph_exec. The reference's equivalent is the
 * caller's own cudaStreamBeginCapture around its ops (tests/unit/framework.cu:154-169); these exist
 * so a host without HIP headers can capture and replay library calls. A capture the runtime
 * refuses (an allocation or synchronization while it is open) returns -1 with its message. */
int opw_graph_capture_begin(void *stream);
int opw_graph_capture_end(void *stream, void **graph_exec);
int opw_graph_launch(void *graph_exec, void *stream);
int opw_graph_destroy(void *graph_exec);

/* ---- seeded synthetic inputs (counter-based; bit-identical to the CPU
 * restatement in oracle/, so the checker regenerates the same arrays) ---- */
int opw_fill_uniform_f32(float *dst, int64_t n, uint64_t seed, uint64_t stream_id, float lo, float hi, void *stream);
int opw_fill_normal_f32(float *dst, int64_t n, uint64_t seed, uint64_t stream_id, float mean, float stddev,
                        void *stream);

/* ---- map (reference: ops::map, include/ops/elementwise.cuh:68-77) ----
 * Exact in-place use is allowed, partial overlap is not. n == 0 is a no-op. */
/* out[i] = fmaf(alpha, a[i], b[i])  — README ScaleAdd functor (README.md:78-83) under nvcc's FMA contraction */
int opw_map_scale_add_f32(const float *a, const float *b, float *out, int n, float alpha, void *stream);
/* out[i] = a[i] + b[i]  — framework.cu Add / tests/integration/vector_add.cu:7-11 */
int opw_map_add_f32(const float *a, const float *b, float *out, int n, void *stream);
/* out[i] = factor * in[i]  — framework.cu Scale */
int opw_map_scale_f32(const float *in, float *out, int n, float factor, void *stream);
/* out[i] = fmaxf(in[i], 0)  — tests/integration/relu.cu:7-10 */
int opw_map_relu_f32(const float *in, float *out, int n, void *stream);

/* ---- reduce (reference: ops::reduce<Op>, include/ops/reduction.cuh:34-67) ---- */
int opw_reduction_workspace_size(int n);
/* op: 0 = sum, 1 = max, 2 = product. workspace == NULL selects the
 * stream-ordered-allocation convenience overload. */
int opw_reduce_f32(const float *in, float *out, int n, int op, float *workspace, int workspace_size, void *stream);
/* The same reduction, allocating nothing: no counterpart in the reference. For callers that cannot
 * allocate device memory (HIP graph capture, serving loops, harnesses that forbid hipMalloc). The
 * partials live in a static 256 KiB device array of this library (one copy per GPU, kept until the
 * process ends), so n <= 2^29 (536870912); larger n is rejected before any launch. All calls on one
 * GPU share that array: calls that overlap on a GPU race. Results equal opw_reduce_f32's bit for bit. */
int opw_reduce_f32_noalloc(const float *in, float *out, int n, int op, void *stream);

/* ---- rows (reference: include/ops/softmax.cuh:36-43, layer_norm.cuh:38-47, rms_norm.cuh:31-40) ---- */
int opw_softmax_f32(const float *in, float *out, int rows, int cols, void *stream);
int opw_layer_norm_f32(const float *in, float *out, const float *gamma, const float *beta, int rows, int cols,
                       float eps, void *stream);
int opw_rms_norm_f32(const float *x, const float *weight, float *out, int rows, int cols, float eps, void *stream);

/* ---- GEMM (reference: ops::mat_mul, include/ops/matmul.cuh:77-91; names as in
 * the reference: A is M x N, B is N x K, C is M x K, reduction over N) ---- */
/* C = A @ B  (PassThrough epilogue). M == 0 or K == 0: no-op; N == 0 writes zeros. */
int opw_mat_mul_f32(const float *A, const float *B, float *C, int M, int N, int K, void *stream);
/* C = act(A @ op(B) + bias[K]); op(B) = B (N x K) or, when b_transposed, B^T with B stored K x N;
 * bias may be NULL; activation 0 none, 1 relu, 2 gelu (erf form). This is what
 * MatmulBuilder(...).transpose_b().bias().activation() configures (include/builders/matmul.cuh:7-57),
 * executed as one fused kernel. */
int opw_mat_mul_fused_f32(const float *A, const float *B, const float *bias, float *C, int M, int N, int K,
                          int b_transposed, int activation, void *stream);
/* The same with a transposed A as well: op(A) is M x N, stored N x M (column-major) when a_transposed
 * (MatmulBuilder::transpose_a, include/builders/matmul.cuh:19-20,35); read in place by the GEMM. */
int opw_mat_mul_fused_ex_f32(const float *A, const float *B, const float *bias, float *C, int M, int N, int K,
                             int a_transposed, int b_transposed, int activation, void *stream);
/* Y[rows][out] = X[rows][in] @ W[out][in]^T (reference: ops::linear, include/ops/linear.cuh:130-153) */
int opw_linear_f32(const float *X, const float *W, float *Y, int rows, int in_features, int out_features,
                   void *stream);

/* Y[rows][out] = X[rows][in] @ W[out][in]^T with bf16 weights W (raw bits), fp32 X and Y: every weight is
 * widened exactly and products accumulate in fp32 (reference: ops::linear<__nv_bfloat16>,
 * include/ops/linear.cuh:99-153: gemv_bf16_kernel at rows == 1, the fp32 tiled kernel above). */
int opw_linear_wbf16(const float *X, const uint16_t *W, float *Y, int rows, int in_features, int out_features,
                     void *stream);

/* ---- bf16 matrix-core path (reference: ops::linear_mma_bf16, include/ops/linear_mma.cuh:99-115) ----
 * Y[rows][out] = act(bf16(X)[rows][in] @ W[out][in]^T + bias), fp32 accumulation; W holds bf16 bit
 * patterns. X is fp32 (rounded to bf16, nearest-even, on load — the reference contract) ... */
int opw_linear_bf16(const float *X, const uint16_t *W, const float *bias, float *Y, int rows, int in_features,
                    int out_features, int activation, void *stream);
/* ... or already bf16. */
int opw_linear_bf16_bf16(const uint16_t *X, const uint16_t *W, const float *bias, float *Y, int rows,
                         int in_features, int out_features, int activation, void *stream);
/* dst[i] = bf16 bits of src[i], round to nearest even (tests/model/ops_test.cu:77-82 recipe) */
int opw_convert_f32_to_bf16(const float *src, uint16_t *dst, int64_t n, void *stream);

/* ---- attention over a KV cache (fp32). q_heads/out [num_q_heads][T][head_dim];
 * caches [num_q_heads/kv_rep][cap][head_dim] with S valid entries; kv head = q head / kv_rep;
 * query t sits at position q_offset + t and sees keys 0..min(position, S-1); scale 1/sqrt(head_dim). ---- */
/* Flash causal prefill (reference: ops::attention_prefill_chunked, include/ops/attention_prefill.cuh:164-177;
 * requires S >= T, q_offset == S - T, head_dim in {16,32,48,64}, cap >= S) */
int opw_attention_prefill_f32(const float *q_heads, const float *kcache, const float *vcache, float *out, int T, int S,
                              int q_offset, int num_q_heads, int kv_rep, int head_dim, int cap, void *stream);
/* Workspace form of opw_attention_prefill_f32 (no counterpart in the reference; same results to
 * rounding). The query-tile groups with the most K/V tiles (more than split_threshold; negative
 * picks it from the shape and the CU count) run as two workgroups over the halves of their K/V
 * range, and the one that finishes last merges them: a one-round causal grid otherwise ends with
 * one workgroup running the longest range alone on its CU. rec needs no initialisation; counters
 * must be zero before the first call, and every call leaves them at zero. Calls that share a
 * workspace must not overlap. Smaller memory than opw_attention_prefill_workspace_size reports
 * splits fewer groups (none: the plain kernel). */
int opw_attention_prefill_workspace_size(int T, int S, int q_offset, int num_q_heads, int kv_rep, int head_dim,
                                         int split_threshold, int64_t *rec_floats, int64_t *counter_ints);
int opw_attention_prefill_ws_f32(const float *q_heads, const float *kcache, const float *vcache, float *out, int T,
                                 int S, int q_offset, int num_q_heads, int kv_rep, int head_dim, int cap, float *rec,
                                 int64_t rec_floats, int *counters, int64_t counter_ints, int split_threshold,
                                 void *stream);
/* One query per head against `len` cache entries (reference: ops::attention_decode,
 * include/ops/attention_decode.cuh:98-109; q/out [num_q_heads][head_dim], len <= 8192). The
 * reference's contract: one launch, nothing allocated (graph-capturable), head_dim in [1, 64], q and
 * caches at any 4-byte alignment, any kv_rep; q head h reads kv head h / kv_rep, so the caches hold
 * ceil(num_q_heads / kv_rep) kv heads of max_seq rows. */
int opw_attention_decode_f32(const float *q, const float *kcache, const float *vcache, float *out, int num_q_heads,
                             int kv_rep, int head_dim, int len, int max_seq, void *stream);
/* ... or from a caller workspace of opw_attention_decode_workspace_size() floats (no allocation). */
int opw_attention_decode_workspace_size(int num_q_heads, int max_len, int head_dim);
int opw_attention_decode_ws_f32(const float *q, const float *kcache, const float *vcache, float *out,
                                int num_q_heads, int kv_rep, int head_dim, int len, int max_seq, float *workspace,
                                int workspace_size, void *stream);
/* ... in one launch, as the Llama decode step runs it: the last chunk workgroup of each kv head merges
 * the head group's records. `counters` holds counters_size >= opw_attention_decode_counters_size() ints
 * (one 256-byte line per kv head), zero before the call and zero again after it; calls sharing counters
 * must not overlap. Same results as opw_attention_decode_ws_f32. No reference counterpart: the
 * reference's decode attention is one workgroup per q head with no cross-workgroup merge. */
int opw_attention_decode_counters_size(int num_q_heads, int kv_rep);
int opw_attention_decode_fused_f32(const float *q, const float *kcache, const float *vcache, float *out,
                                   int num_q_heads, int kv_rep, int head_dim, int len, int max_seq, float *workspace,
                                   int workspace_size, int *counters, int counters_size, void *stream);

/* ---- decoder-block steps (reference: include/ops/add.cuh:18-25, swiglu.cuh:19-26,
 *      causal_scale.cuh:24-33, embedding.cuh:24-34, split_heads.cuh:39-66, rope.cuh:34-46,
 *      argmax.cuh:59-63) ---- */
int opw_add_f32(const float *a, const float *b, float *out, long long n, void *stream);
int opw_swiglu_f32(const float *gate, const float *up, float *out, long long n, void *stream);
int opw_causal_scale_f32(float *scores, int rows, int cols, float scale, void *stream);
/* table [vocab][hidden]; an id outside [0, vocab) yields a NaN row (no out-of-table read). */
int opw_embedding_f32(const float *table, long long vocab, const int *ids, float *out, int n, int hidden,
                      void *stream);
int opw_embedding_bf16(const uint16_t *table, long long vocab, const int *ids, float *out, int n, int hidden,
                       void *stream);
int opw_split_heads_f32(const float *in, float *out, int rows, int heads, int head_dim, int out_row_stride,
                        int out_row_offset, void *stream);
int opw_merge_heads_f32(const float *in, float *out, int rows, int heads, int head_dim, int in_row_stride,
                        int in_row_offset, void *stream);
int opw_rope_f32(float *x, const float *inv_freq, int rows, int heads, int head_dim, int pos_start, void *stream);
/* out[0] (device int) = index of the maximum; ties -> lowest index, NaN never wins, all-NaN -> 0x7fffffff. */
int opw_argmax_f32(const float *x, int n, int *out, void *stream);

/* ---- kernels behind the Scan / Transform / GatherScatter builders. The reference builders
 *      carry only the operation metadata (include/builders/scan.cuh:7-43, transform.cuh:7-38,
 *      gather_scatter.cuh:7-36) and leave the kernel to their apply() callback. ---- */
/* Floats of workspace opw_scan_f32 needs for n elements (0 up to 16384); 16-byte aligned.
 * Its contents on entry do not matter; word 1 holds the number of timed-out waits of the
 * last scan that used it (0 unless the scan is broken). */
int opw_scan_workspace_size(int n);
/* op: 0 = sum, 1 = maximum (fmaxf, identity -inf); inclusive: 1 = out[i] covers x[0..i],
 * 0 = x[0..i-1] with out[0] = identity. In place (out == in) is allowed. workspace == NULL
 * selects the stream-ordered-allocation convenience overload. Scans sharing a workspace
 * must not run concurrently. */
int opw_scan_f32(const float *in, float *out, int n, int op, int inclusive, float *workspace, int workspace_size,
                 void *stream);
/* out [cols][rows] = transpose of in [rows][cols]; not in place. */
int opw_transpose_f32(const float *in, float *out, int rows, int cols, void *stream);
/* out[i] = in[i], i < n (TransformOp::copy and ::reshape). */
int opw_copy_f32(const float *in, float *out, int n, void *stream);
/* out[i] = in[idx[i]], i < count; an index outside [0, in_size) writes NaN. */
int opw_gather_f32(const float *in, long long in_size, const int *idx, float *out, int count, void *stream);
/* out[idx[i]] = in[i], i < count; an index outside [0, out_size) is skipped; duplicate indices race. */
int opw_scatter_f32(const float *in, const int *idx, float *out, long long out_size, int count, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OPWORKS_OPS_H */

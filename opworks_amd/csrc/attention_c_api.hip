// extern "C" attention surface of libopworks_amd.so (include/opworks_ops.h).

#include <hip/hip_runtime.h>

#include "../include/ops/attention.hpp"
#include "c_api_common.hpp"

using opworks::capi::guard;

extern "C" {

int opw_attention_prefill_f32(const float *q_heads, const float *kcache, const float *vcache, float *out, int T, int S,
                              int q_offset, int num_q_heads, int kv_rep, int head_dim, int cap, void *stream) {
    return guard([&] {
        opworks::ops::attention_prefill(q_heads, kcache, vcache, out, T, S, q_offset, num_q_heads, kv_rep, head_dim,
                                        cap, static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_attention_prefill_workspace_size(int T, int S, int q_offset, int num_q_heads, int kv_rep, int head_dim,
                                         int split_threshold, int64_t *rec_floats, int64_t *counter_ints) {
    return guard([&] {
        opworks::detail::require(rec_floats && counter_ints, "attention_prefill_workspace_size: null output");
        opworks::ops::attention_prefill_workspace_size(T, S, q_offset, num_q_heads, kv_rep, head_dim, split_threshold,
                                                       rec_floats, counter_ints);
        return 0;
    });
}

int opw_attention_prefill_ws_f32(const float *q_heads, const float *kcache, const float *vcache, float *out, int T,
                                 int S, int q_offset, int num_q_heads, int kv_rep, int head_dim, int cap, float *rec,
                                 int64_t rec_floats, int *counters, int64_t counter_ints, int split_threshold,
                                 void *stream) {
    return guard([&] {
        opworks::ops::attention_prefill_ws(q_heads, kcache, vcache, out, T, S, q_offset, num_q_heads, kv_rep, head_dim,
                                           cap, rec, rec_floats, counters, counter_ints, split_threshold,
                                           static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_attention_decode_f32(const float *q, const float *kcache, const float *vcache, float *out, int num_q_heads,
                             int kv_rep, int head_dim, int len, int max_seq, void *stream) {
    return guard([&] {
        opworks::ops::attention_decode(q, kcache, vcache, out, num_q_heads, kv_rep, head_dim, len, max_seq,
                                       static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_attention_decode_workspace_size(int num_q_heads, int max_len, int head_dim) {
    return guard([&] {
        opworks::detail::require(num_q_heads > 0 && max_len > 0 && head_dim > 0, "positive shape required");
        return opworks::ops::attention_decode_workspace_size(num_q_heads, max_len, head_dim);
    });
}

int opw_attention_decode_ws_f32(const float *q, const float *kcache, const float *vcache, float *out,
                                int num_q_heads, int kv_rep, int head_dim, int len, int max_seq, float *workspace,
                                int workspace_size, void *stream) {
    return guard([&] {
        opworks::ops::attention_decode_ws(q, kcache, vcache, out, num_q_heads, kv_rep, head_dim, len, max_seq,
                                          workspace, workspace_size, nullptr, 0, 0,
                                          static_cast<hipStream_t>(stream));
        return 0;
    });
}

int opw_attention_decode_counters_size(int num_q_heads, int kv_rep) {
    return guard([&] { return opworks::ops::attention_decode_counters_size(num_q_heads, kv_rep); });
}

int opw_attention_decode_fused_f32(const float *q, const float *kcache, const float *vcache, float *out,
                                   int num_q_heads, int kv_rep, int head_dim, int len, int max_seq, float *workspace,
                                   int workspace_size, int *counters, int counters_size, void *stream) {
    return guard([&] {
        opworks::detail::require(counters_size >= opworks::ops::attention_decode_counters_size(num_q_heads, kv_rep),
                                 "attention_decode_fused: counters are too small");
        opworks::ops::attention_decode_fused(q, kcache, vcache, out, num_q_heads, kv_rep, head_dim, len, max_seq,
                                             workspace, workspace_size, counters, static_cast<hipStream_t>(stream));
        return 0;
    });
}

} // extern "C"

#pragma once

// Per-session scratch of the Llama runtime (reference: include/runtime/
// workspace.cuh:10-55), allocated once when the session is created and reused
// by every prefill and decode step. Buffers with a counterpart in the
// reference keep its name (tokens, hidden, normed, q_heads, attn_out,
// logits). The reference's attn_heads is not needed: the prefill attention
// writes its rows with the heads merged, straight into attn_out (or, for
// bf16 weights, into the bf16 input copy). The others serve this build's
// fused kernels: the fused [q;k;v] projection output, the SwiGLU product,
// split-K partial tiles, the bf16 copy of each projection's input (bf16-weight
// models), the prefill attention's split records and counters, the one-row
// buffers of the decode step, the decode attention's chunk records and
// arrival counters, the LM head's per-workgroup argmax records, the device
// step state and the tokens a chained greedy decode produces.

#include <algorithm>
#include <cstdint>

#include "../core/typed_device_buffer.hpp"
#include "model_config.hpp"

namespace opworks {

// Sizes that depend on the kernels' geometry, supplied by the model.
struct WorkspaceSizes {
    int attn_chunks = 0;       // decode attention chunks at max_seq_len
    int lm_records = 0;        // LM-head workgroups (one argmax record each)
    int64_t splitk_floats = 0; // split-K partial tiles of the prefill GEMMs
    int state_ints = 0;        // device step state
    int argmax_groups = 0;     // workgroups of the records' reduction
    int attn_counter_ints = 0; // decode attention arrival counters (one cache line per kv head)
    int64_t prefill_split_floats = 0; // prefill attention: records of the split query-tile groups
    int64_t prefill_split_ints = 0;   // and their arrival counters
    bool bf16_inputs = false;  // bf16-weight model: a bf16 copy of each prefill projection's input
};

struct Workspace {
    // prefill: up to max_seq_len rows
    TypedDeviceBuffer<int32_t> tokens;   // [T] prompt ids
    TypedDeviceBuffer<float> hidden;     // [T, H] residual stream
    TypedDeviceBuffer<float> normed;     // [T, H]
    TypedDeviceBuffer<float> qkv;        // [T, (qh + 2 kvh) D] fused projection output
    TypedDeviceBuffer<float> q_heads;    // [qh, T, D]
    TypedDeviceBuffer<float> attn_out;   // [T, qh D]
    TypedDeviceBuffer<float> act;        // [T, I] silu(gate) * up
    TypedDeviceBuffer<float> splitk;     // split-K partial tiles
    TypedDeviceBuffer<bf16> x_bf16;      // [T, max(H, I, qh D)] projection input rounded to bf16 (bf16-weight models)
    TypedDeviceBuffer<float> attn_split;          // prefill attention: records of split query-tile groups
    TypedDeviceBuffer<int32_t> attn_split_counters; // their arrivals, zero between launches
    // decode step: one row
    TypedDeviceBuffer<float> step_hidden;   // [H] residual stream
    TypedDeviceBuffer<float> step_q;        // [qh D] post-RoPE query
    TypedDeviceBuffer<float> step_attn;     // [qh D] attention output
    TypedDeviceBuffer<float> step_act;      // [I] silu(gate) * up
    TypedDeviceBuffer<float> attn_partial;  // [qh][chunks][D + 2] chunk records
    TypedDeviceBuffer<int32_t> attn_counters; // per-kv-head arrivals, zero between launches
    TypedDeviceBuffer<float> logits;        // [V] last row's logits
    TypedDeviceBuffer<float> lm_best_val;   // [records]
    TypedDeviceBuffer<int32_t> lm_best_idx; // [records]
    TypedDeviceBuffer<float> lm_part_val;   // [argmax groups] partials of the records' reduction
    TypedDeviceBuffer<int32_t> lm_part_idx; // [argmax groups]
    TypedDeviceBuffer<int32_t> lm_counter;  // arrivals of the argmax groups (own 256-byte line), zero between launches
    TypedDeviceBuffer<int32_t> gen;         // [T] tokens of a chained greedy decode, by position
    TypedDeviceBuffer<int32_t> state;       // device step state
    WorkspaceSizes sizes;

    Workspace() = default;
    Workspace(const ModelConfig &cfg, int max_seq_len, const WorkspaceSizes &s) : sizes(s) {
        const int64_t T = max_seq_len, H = cfg.hidden_size, I = cfg.intermediate_size;
        const int64_t qw = cfg.q_width(), D = cfg.head_dim;
        tokens = TypedDeviceBuffer<int32_t>(T);
        hidden = TypedDeviceBuffer<float>(T * H);
        normed = TypedDeviceBuffer<float>(T * H);
        qkv = TypedDeviceBuffer<float>(T * cfg.qkv_width());
        q_heads = TypedDeviceBuffer<float>(T * qw);
        attn_out = TypedDeviceBuffer<float>(T * qw);
        act = TypedDeviceBuffer<float>(T * I);
        if (T >= 2) { // only a multi-row prefill runs the GEMMs
            splitk = TypedDeviceBuffer<float>(s.splitk_floats);
            if (s.bf16_inputs)
                x_bf16 = TypedDeviceBuffer<bf16>(T * std::max(std::max(H, I), qw));
            if (s.prefill_split_floats > 0 && s.prefill_split_ints > 0) {
                attn_split = TypedDeviceBuffer<float>(s.prefill_split_floats);
                attn_split_counters = TypedDeviceBuffer<int32_t>(s.prefill_split_ints);
            }
        }
        step_hidden = TypedDeviceBuffer<float>(H);
        step_q = TypedDeviceBuffer<float>(qw);
        step_attn = TypedDeviceBuffer<float>(qw);
        step_act = TypedDeviceBuffer<float>(I);
        attn_partial = TypedDeviceBuffer<float>(int64_t(cfg.num_q_heads) * s.attn_chunks * (D + 2));
        attn_counters = TypedDeviceBuffer<int32_t>(s.attn_counter_ints);
        logits = TypedDeviceBuffer<float>(cfg.vocab_size);
        lm_best_val = TypedDeviceBuffer<float>(s.lm_records);
        lm_best_idx = TypedDeviceBuffer<int32_t>(s.lm_records);
        lm_part_val = TypedDeviceBuffer<float>(s.argmax_groups);
        lm_part_idx = TypedDeviceBuffer<int32_t>(s.argmax_groups);
        lm_counter = TypedDeviceBuffer<int32_t>(64);
        gen = TypedDeviceBuffer<int32_t>(T);
        state = TypedDeviceBuffer<int32_t>(s.state_ints);
    }
};

} // namespace opworks

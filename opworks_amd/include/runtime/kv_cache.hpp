#pragma once

// Per-session KV cache (reference: include/runtime/kv_cache.cuh:11-35). For
// every layer one [num_kv_heads][max_seq_len][head_dim] fp32 slab holds K
// (after RoPE) and one holds V (as projected). `length` counts the valid
// entries, the same for every layer; reset() only forgets them: every kernel
// bounds its reads by the length, so stale bytes are never read.

#include <cstdint>
#include <vector>

#include "../core/typed_device_buffer.hpp"
#include "model_config.hpp"

namespace opworks {

struct KvCache {
    std::vector<TypedDeviceBuffer<float>> k; // per layer
    std::vector<TypedDeviceBuffer<float>> v;
    int max_seq_len = 0;
    int length = 0;

    KvCache() = default;
    KvCache(const ModelConfig &cfg, int max_seq_len) : max_seq_len(max_seq_len) {
        const int64_t slab = int64_t(cfg.num_kv_heads) * max_seq_len * cfg.head_dim;
        k.reserve(static_cast<size_t>(cfg.num_layers));
        v.reserve(static_cast<size_t>(cfg.num_layers));
        for (int l = 0; l < cfg.num_layers; ++l) {
            k.emplace_back(slab);
            v.emplace_back(slab);
        }
    }

    void reset() { length = 0; }
};

} // namespace opworks

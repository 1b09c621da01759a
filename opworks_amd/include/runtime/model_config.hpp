#pragma once

// Llama hyper-parameters from an HF-style config (the pack manifest's
// "config" object) — reference: include/runtime/model_config.cuh:14-89.

#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "json.hpp"

namespace opworks {

struct ModelConfig {
    int num_layers = 0;
    int hidden_size = 0;
    int intermediate_size = 0;
    int num_q_heads = 0;
    int num_kv_heads = 0;
    int head_dim = 0;
    int vocab_size = 0;
    float rms_norm_eps = 0.f;
    float rope_theta = 0.f;
    bool rope_llama3 = false;
    float rope_factor = 0.f;
    float rope_low_freq = 0.f;
    float rope_high_freq = 0.f;
    int rope_original_max_pos = 0;
    std::vector<int32_t> eos_token_ids;

    int kv_width() const { return num_kv_heads * head_dim; }
    int q_width() const { return num_q_heads * head_dim; }
    int kv_rep() const { return num_q_heads / num_kv_heads; }
    int qkv_width() const { return q_width() + 2 * kv_width(); }

    // An integer field that fits an int (sizes, counts, token ids).
    static int int_field(const json::Value &v, const char *what) {
        const int64_t x = v.as_int();
        if (x < INT32_MIN || x > INT32_MAX)
            throw std::runtime_error(std::string("config field ") + what + " out of range");
        return static_cast<int>(x);
    }

    // A finite real field that fits a float.
    static float float_field(const json::Value &v, const char *what) {
        const double x = v.as_number();
        if (!(x >= -3.0e38 && x <= 3.0e38))
            throw std::runtime_error(std::string("config field ") + what + " out of range");
        return static_cast<float>(x);
    }

    // `config` is the HF config object; `eos` the manifest's eos_token_ids (may be null).
    static ModelConfig from_json(const json::Value &c, const json::Value *eos) {
        ModelConfig m;
        m.num_layers = int_field(c.at("num_hidden_layers"), "num_hidden_layers");
        m.hidden_size = int_field(c.at("hidden_size"), "hidden_size");
        m.intermediate_size = int_field(c.at("intermediate_size"), "intermediate_size");
        m.num_q_heads = int_field(c.at("num_attention_heads"), "num_attention_heads");
        m.num_kv_heads = int_field(c.at("num_key_value_heads"), "num_key_value_heads");
        m.head_dim = c.find("head_dim") ? int_field(c.at("head_dim"), "head_dim")
                                        : (m.num_q_heads > 0 ? m.hidden_size / m.num_q_heads : 0);
        m.vocab_size = int_field(c.at("vocab_size"), "vocab_size");
        m.rms_norm_eps = float_field(c.at("rms_norm_eps"), "rms_norm_eps");
        m.rope_theta = float_field(c.at("rope_theta"), "rope_theta");
        if (const json::Value *rs = c.find("rope_scaling"); rs && !rs->is_null()) {
            if (rs->at("rope_type").as_string() != "llama3")
                throw std::runtime_error("unsupported rope_scaling type");
            m.rope_llama3 = true;
            m.rope_factor = float_field(rs->at("factor"), "factor");
            m.rope_low_freq = float_field(rs->at("low_freq_factor"), "low_freq_factor");
            m.rope_high_freq = float_field(rs->at("high_freq_factor"), "high_freq_factor");
            m.rope_original_max_pos =
                int_field(rs->at("original_max_position_embeddings"), "original_max_position_embeddings");
        }
        if (eos && !eos->is_null()) {
            if (eos->is_array()) {
                for (const auto &v : eos->as_array())
                    m.eos_token_ids.push_back(int_field(v, "eos_token_ids"));
            } else {
                m.eos_token_ids.push_back(int_field(*eos, "eos_token_ids"));
            }
        }
        m.validate();
        return m;
    }

    static ModelConfig from_manifest(const json::Value &manifest) {
        return from_json(manifest.at("config"), manifest.find("eos_token_ids"));
    }

    void validate() const {
        if (num_layers <= 0 || hidden_size <= 0 || head_dim <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
            num_q_heads % num_kv_heads != 0 || intermediate_size <= 0 || vocab_size <= 0)
            throw std::runtime_error("invalid model config");
        // widths are multiplied together in int (qkv_width, row strides); 2^24
        // is far above any released Llama and keeps every product in range
        constexpr int kMaxDim = 1 << 24;
        if (num_layers > kMaxDim || hidden_size > kMaxDim || intermediate_size > kMaxDim || vocab_size > kMaxDim)
            throw std::runtime_error("model config dimension out of range");
        if (static_cast<int64_t>(num_q_heads) * head_dim != hidden_size)
            throw std::runtime_error("num_attention_heads * head_dim != hidden_size");
        if (head_dim % 2 != 0)
            throw std::runtime_error("head_dim must be even");
        if (!(rms_norm_eps > 0.f) || !(rope_theta > 0.f))
            throw std::runtime_error("rms_norm_eps and rope_theta must be positive");
    }

    // inv_freq[i] for head_dim/2 rotary pairs with llama3 wavelength scaling,
    // computed in double and rounded to float (model_config.cuh:66-89 contract).
    std::vector<float> rope_inv_freq() const {
        const int half = head_dim / 2;
        std::vector<float> out(static_cast<size_t>(half));
        const double pi = 3.14159265358979323846;
        for (int i = 0; i < half; ++i) {
            double f = 1.0 / std::pow(static_cast<double>(rope_theta), (2.0 * i) / head_dim);
            if (rope_llama3) {
                // int / float and float - float are evaluated in float, as in the reference
                const double wavelen = 2.0 * pi / f;
                const double low_wl = static_cast<float>(rope_original_max_pos) / rope_low_freq;
                const double high_wl = static_cast<float>(rope_original_max_pos) / rope_high_freq;
                if (wavelen > low_wl) {
                    f /= rope_factor;
                } else if (wavelen >= high_wl) {
                    const double smooth = (rope_original_max_pos / wavelen - rope_low_freq) /
                                          static_cast<double>(rope_high_freq - rope_low_freq);
                    f = (1.0 - smooth) * f / rope_factor + smooth * f;
                }
            }
            out[static_cast<size_t>(i)] = static_cast<float>(f);
        }
        return out;
    }
};

} // namespace opworks

// extern "C" Llama runtime surface of libopworks_amd.so (include/opworks_llama.h).

#include <hip/hip_runtime.h>

#include <chrono>
#include <memory>
#include <string>
#include <vector>

#include "../include/models/llama.hpp"
#include "c_api_common.hpp"

using opworks::capi::capture_error;
using opworks::capi::guard;

namespace {

struct ModelHolder {
    std::unique_ptr<opworks::LlamaRuntime> model;
};
struct SessionHolder {
    ModelHolder *owner;
    std::unique_ptr<opworks::LlamaSession> session;
};

template <typename F> void *guard_ptr(F &&f, char *err, int err_len) {
    try {
        return f();
    } catch (const std::exception &e) {
        capture_error(e.what(), err, err_len);
    } catch (...) {
        capture_error("unknown C++ exception", err, err_len);
    }
    return nullptr;
}

SessionHolder *as_session(void *p) {
    if (!p)
        throw std::invalid_argument("null session");
    return static_cast<SessionHolder *>(p);
}

} // namespace

extern "C" {

void *opw_llama_load(const char *pack_path, char *err, int err_len) {
    return guard_ptr(
        [&]() -> void * {
            if (!pack_path)
                throw std::invalid_argument("null pack path");
            return new ModelHolder{opworks::load_llama(pack_path)};
        },
        err, err_len);
}

void opw_llama_free(void *model) { delete static_cast<ModelHolder *>(model); }

void *opw_llama_create_session(void *model, int max_seq_len, char *err, int err_len) {
    if (!model) {
        capture_error("null model", err, err_len);
        return nullptr;
    }
    return guard_ptr(
        [&]() -> void * {
            auto *m = static_cast<ModelHolder *>(model);
            return new SessionHolder{m, m->model->new_session(max_seq_len)};
        },
        err, err_len);
}

void opw_llama_destroy_session(void *session) { delete static_cast<SessionHolder *>(session); }

int opw_llama_reset_session(void *session, char *err, int err_len) {
    return guard(
        [&] {
            as_session(session)->session->reset();
            return 0;
        },
        err, err_len);
}

int opw_llama_prefill(void *session, const int32_t *tokens, int n, char *err, int err_len) {
    return guard(
        [&] {
            auto *s = as_session(session);
            if (!tokens && n > 0)
                throw std::invalid_argument("null token buffer");
            if (n < 0)
                throw std::invalid_argument("negative token count");
            std::vector<int32_t> ids(tokens, tokens + static_cast<size_t>(n));
            return static_cast<int>(s->owner->model->prefill(*s->session, ids));
        },
        err, err_len);
}

int opw_llama_decode_step(void *session, int32_t prev_token, char *err, int err_len) {
    return guard(
        [&] {
            auto *s = as_session(session);
            return static_cast<int>(s->owner->model->decode_step(*s->session, prev_token));
        },
        err, err_len);
}

int opw_llama_is_eos(void *session, int32_t token, char *err, int err_len) {
    return guard([&] { return as_session(session)->owner->model->is_eos(token) ? 1 : 0; }, err, err_len);
}

int opw_llama_last_logits(void *session, float *out, int n, char *err, int err_len) {
    return guard(
        [&] {
            auto *s = as_session(session);
            if (!out)
                throw std::invalid_argument("null logits buffer");
            s->owner->model->copy_last_logits(*s->session, out, n);
            return 0;
        },
        err, err_len);
}

int opw_llama_vocab_size(void *session) {
    return guard([&] { return as_session(session)->owner->model->config().vocab_size; });
}

const char *opw_llama_last_error(void) { return opworks::capi::last_error().c_str(); }

void *opw_llama_load_random(const char *config_json, uint64_t seed, float init_std, int norm_init, char *err,
                            int err_len) {
    return guard_ptr(
        [&]() -> void * {
            if (!config_json)
                throw std::invalid_argument("null config");
            if (!(init_std > 0.f))
                throw std::invalid_argument("init_std must be positive");
            if (norm_init != 0 && norm_init != 1)
                throw std::invalid_argument("norm_init must be 0 (ones) or 1 (uniform)");
            const opworks::json::Value cfg = opworks::json::parse(config_json);
            const opworks::ModelConfig mc = opworks::ModelConfig::from_json(cfg, cfg.find("eos_token_id"));
            // HF configs name the checkpoint dtype in "torch_dtype"; bfloat16 selects bf16 weights
            const opworks::json::Value *dt = cfg.find("torch_dtype");
            if (!dt)
                dt = cfg.find("dtype");
            const std::string dtype = dt ? dt->as_string() : "float32";
            if (dtype != "float32" && dtype != "bfloat16")
                throw std::invalid_argument("torch_dtype must be float32 or bfloat16");
            return new ModelHolder{opworks::load_llama_random(mc, seed, init_std,
                                                              static_cast<opworks::NormInit>(norm_init),
                                                              dtype == "bfloat16")};
        },
        err, err_len);
}

int opw_llama_config_inv_freq(const char *config_json, float *out, int n, char *err, int err_len) {
    return guard(
        [&] {
            if (!config_json || !out)
                throw std::invalid_argument("null config or output");
            const opworks::json::Value cfg = opworks::json::parse(config_json);
            const std::vector<float> f =
                opworks::ModelConfig::from_json(cfg, cfg.find("eos_token_id")).rope_inv_freq();
            if (n != static_cast<int>(f.size()))
                throw std::invalid_argument("output must hold head_dim / 2 floats");
            std::memcpy(out, f.data(), f.size() * sizeof(float));
            return 0;
        },
        err, err_len);
}

int opw_llama_model_config(void *model, int *out7, char *err, int err_len) {
    return guard(
        [&] {
            if (!model || !out7)
                throw std::invalid_argument("null model or output");
            const opworks::ModelConfig &c = static_cast<ModelHolder *>(model)->model->config();
            const int v[7] = {c.num_layers,   c.hidden_size, c.intermediate_size, c.num_q_heads,
                              c.num_kv_heads, c.head_dim,    c.vocab_size};
            for (int i = 0; i < 7; ++i)
                out7[i] = v[i];
            return 0;
        },
        err, err_len);
}

int opw_llama_debug_prefill(void *session, const int32_t *tokens, int n, float *captures, int64_t capacity,
                            char *err, int err_len) {
    return guard(
        [&] {
            auto *s = as_session(session);
            if (!tokens || n <= 0 || !captures)
                throw std::invalid_argument("debug_prefill needs tokens and a capture buffer");
            const opworks::ModelConfig &c = s->owner->model->config();
            const int64_t need = int64_t(c.num_layers + 1) * n * c.hidden_size;
            if (capacity < need)
                throw std::invalid_argument("capture buffer too small");
            std::vector<int32_t> ids(tokens, tokens + n);
            auto caps = s->owner->model->debug_prefill(*s->session, ids);
            float *dst = captures;
            for (const auto &h : caps) {
                std::memcpy(dst, h.data(), h.size() * sizeof(float));
                dst += h.size();
            }
            opworks::synchronize(s->session->stream);
            return static_cast<int>(s->session->h_state->next);
        },
        err, err_len);
}

int opw_llama_generate_greedy(void *session, const int32_t *prompt, int n, int max_new, int32_t *out_tokens,
                              double *prefill_ms, double *decode_ms, char *err, int err_len) {
    return guard(
        [&] {
            auto *s = as_session(session);
            if (!prompt || n <= 0 || max_new <= 0 || !out_tokens)
                throw std::invalid_argument("generate needs a prompt, max_new > 0 and an output buffer");
            opworks::LlamaRuntime &m = *s->owner->model;
            // checked before any work, so a rejected call leaves the session untouched
            if (int64_t(n) + max_new - 1 > s->session->cache.max_seq_len)
                throw std::invalid_argument("prompt plus max_new - 1 generated tokens exceed the session capacity");
            std::vector<int32_t> ids(prompt, prompt + n);
            using clock = std::chrono::steady_clock;
            const auto t0 = clock::now();
            int32_t tok = m.prefill(*s->session, ids);
            const auto t1 = clock::now();
            out_tokens[0] = tok;
            m.decode_greedy(*s->session, tok, max_new - 1, out_tokens + 1);
            const auto t2 = clock::now();
            if (prefill_ms)
                *prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
            if (decode_ms)
                *decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
            return max_new;
        },
        err, err_len);
}

int opw_llama_profile_decode_step(void *session, int32_t prev_token, float *kernel_ms, int capacity, char *err,
                                  int err_len) {
    return guard(
        [&] {
            auto *s = as_session(session);
            // one duration per decode stage of every layer plus the LM head, checked before any work
            const int stages = 5 * s->owner->model->config().num_layers + 1;
            if (!kernel_ms || capacity < stages)
                throw std::invalid_argument("kernel_ms needs 5 * layers + 1 entries");
            int32_t next = -1;
            std::vector<float> ms = s->owner->model->profile_decode_step(*s->session, prev_token, &next);
            if (static_cast<int>(ms.size()) != stages)
                throw std::logic_error("profile_decode_step timed an unexpected number of stages");
            std::memcpy(kernel_ms, ms.data(), ms.size() * sizeof(float));
            return static_cast<int>(ms.size());
        },
        err, err_len);
}

float opw_llama_time_decode_stage(void *session, int stage, int reps, char *err, int err_len) {
    float us = -1.f;
    const int rc = guard(
        [&] {
            auto *s = as_session(session);
            us = s->owner->model->time_decode_stage(*s->session, stage, reps);
            return 0;
        },
        err, err_len);
    return rc < 0 ? -1.f : us;
}

} // extern "C"

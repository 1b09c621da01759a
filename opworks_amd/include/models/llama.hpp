#pragma once

// Llama-3.x decoder on MI355X, fp32 weights (reference: include/models/llama.cuh:43-293).
//
// Same model-level contract as the reference's LlamaModelT / LlamaSession:
// load (pack or seeded random init) returning the model by value,
// create_session(max_seq <= 8192) returning the session by value (its cache
// member is a KvCache, reset by session.cache.reset()), prefill (fresh
// session, returns the first generated token), decode_step (appends one
// token, returns the next), is_eos, last_logits, copy_last_logits,
// hidden_state, debug_prefill. K is cached post-RoPE, V as projected; the LM
// head is the tied embedding applied to the last row. The weights'
// MI355X layout (fused q/k/v rows, interleaved gate/up rows) is described in
// runtime/weights.hpp.
// Decode is one captured HIP graph per session (5 kernels per layer + LM head);
// prefill runs the MFMA GEMMs with fused residual / SwiGLU epilogues and the
// flash attention kernel.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../core/hip_utils.hpp"
#include "../core/random.hpp"
#include "../core/typed_device_buffer.hpp"
#include "../ops/attention.hpp"
#include "../ops/gemm_f32.hpp"
#include "../ops/rms_norm.hpp"
#include "../ops/gemm_bf16.hpp"
#include "../ops/linear_bf16.hpp"
#include "../runtime/kv_cache.hpp"
#include "../runtime/model_config.hpp"
#include "../runtime/pack_reader.hpp"
#include "../runtime/weights.hpp"
#include "../runtime/workspace.hpp"
#include "llama_kernels.hpp"

namespace opworks {

namespace detail {

// Runtime handles a session owns: moving transfers them, destruction releases them.
struct SessionHandles {
    hipStream_t stream = nullptr;
    hipGraph_t graph = nullptr;          // the decode step, captured on first use
    hipGraphExec_t graph_exec = nullptr;
    hipGraph_t group_graph = nullptr;    // kDecodeGroup chained decode steps in one graph
    hipGraphExec_t group_exec = nullptr;
    llama::StepState *h_state = nullptr; // pinned host copy of the device step state
    std::vector<hipEvent_t> step_events; // chained decode: completion of the steps in flight

    SessionHandles() = default;
    SessionHandles(SessionHandles &&o) noexcept
        : stream(std::exchange(o.stream, nullptr)), graph(std::exchange(o.graph, nullptr)),
          graph_exec(std::exchange(o.graph_exec, nullptr)), group_graph(std::exchange(o.group_graph, nullptr)),
          group_exec(std::exchange(o.group_exec, nullptr)), h_state(std::exchange(o.h_state, nullptr)),
          step_events(std::move(o.step_events)) {
        o.step_events.clear();
    }
    SessionHandles &operator=(SessionHandles &&o) noexcept {
        if (this != &o) {
            release();
            stream = std::exchange(o.stream, nullptr);
            graph = std::exchange(o.graph, nullptr);
            graph_exec = std::exchange(o.graph_exec, nullptr);
            group_graph = std::exchange(o.group_graph, nullptr);
            group_exec = std::exchange(o.group_exec, nullptr);
            h_state = std::exchange(o.h_state, nullptr);
            step_events = std::move(o.step_events);
            o.step_events.clear();
        }
        return *this;
    }
    SessionHandles(const SessionHandles &) = delete;
    SessionHandles &operator=(const SessionHandles &) = delete;
    ~SessionHandles() { release(); }

    void release() noexcept {
        for (hipEvent_t e : step_events)
            (void)hipEventDestroy(e);
        step_events.clear();
        if (group_exec)
            (void)hipGraphExecDestroy(group_exec);
        if (group_graph)
            (void)hipGraphDestroy(group_graph);
        if (graph_exec)
            (void)hipGraphExecDestroy(graph_exec);
        if (graph)
            (void)hipGraphDestroy(graph);
        if (h_state)
            (void)hipHostFree(h_state);
        if (stream)
            (void)hipStreamDestroy(stream);
        group_exec = nullptr;
        group_graph = nullptr;
        graph_exec = nullptr;
        graph = nullptr;
        h_state = nullptr;
        stream = nullptr;
    }
};

} // namespace detail

// Per-session state (reference: LlamaSession, include/models/llama.cuh:47-76):
// the KV cache, the scratch workspace and a stream of its own, plus the decode
// graph and the pinned step state. Sessions are independent of the weight
// type; one model serves many sessions, each used by one host thread at a time.
struct LlamaSession : detail::SessionHandles {
    KvCache cache;
    Workspace workspace;
    int last_prefill_rows = 0;

    // Records of the prefill attention's split groups held per session (64 MiB).
    static constexpr int64_t kPrefillSplitCap = int64_t(1) << 24;

    // Sizes of the kernels' per-session scratch at max_seq_len.
    static WorkspaceSizes workspace_sizes(const ModelConfig &cfg, int max_seq_len, bool bf16_weights) {
        WorkspaceSizes ws;
        ws.bf16_inputs = bf16_weights;
        ws.attn_chunks = static_cast<int>(detail::blocks_for64(max_seq_len, detail::kAttnChunk));
        ws.lm_records = static_cast<int>(detail::blocks_for64(cfg.vocab_size, llama::kLmRows * llama::kWavesPerBlock));
        ws.splitk_floats = std::max(detail::kSplitKWorkspaceF32, detail::kSplitKWorkspaceBf16);
        ws.state_ints = sizeof(llama::StepState) / sizeof(int32_t);
        ws.argmax_groups = llama::kArgmaxGroups;
        ws.attn_counter_ints = cfg.num_kv_heads * detail::kAttnCounterStride;
        // the prefill attention's split records for the largest need over the prompt lengths this
        // session can take, at most kPrefillSplitCap floats (past it fewer groups split)
        if (max_seq_len >= 2 && cfg.head_dim % 16 == 0 && cfg.head_dim <= detail::kAttnMaxD) {
            for (int n = 16; n < max_seq_len + 16; n += 16) {
                const int t = n < max_seq_len ? n : max_seq_len;
                int64_t rec = 0, ctr = 0;
                ops::attention_prefill_workspace_size(t, t, 0, cfg.num_q_heads, cfg.kv_rep(), cfg.head_dim, -1, &rec,
                                                      &ctr);
                ws.prefill_split_floats = std::max(ws.prefill_split_floats, std::min(rec, kPrefillSplitCap));
                ws.prefill_split_ints = std::max(ws.prefill_split_ints, ctr);
            }
        }
        return ws;
    }

    LlamaSession(const ModelConfig &cfg, int max_seq_len, bool bf16_weights = false)
        : cache(cfg, max_seq_len), workspace(cfg, max_seq_len, workspace_sizes(cfg, max_seq_len, bf16_weights)) {
        OPWORKS_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        OPWORKS_HIP_CHECK(hipMemsetAsync(workspace.state.data(), 0, workspace.state.bytes(), stream));
        OPWORKS_HIP_CHECK(hipMemsetAsync(workspace.attn_counters.data(), 0, workspace.attn_counters.bytes(), stream));
        if (workspace.attn_split_counters.size() > 0)
            OPWORKS_HIP_CHECK(hipMemsetAsync(workspace.attn_split_counters.data(), 0,
                                             workspace.attn_split_counters.bytes(), stream));
        OPWORKS_HIP_CHECK(hipMemsetAsync(workspace.lm_counter.data(), 0, workspace.lm_counter.bytes(), stream));
        OPWORKS_HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&h_state), sizeof(llama::StepState)));
        *h_state = llama::StepState{0, 0, -1, 0};
        synchronize(stream);
    }
    LlamaSession(LlamaSession &&) noexcept = default;
    LlamaSession &operator=(LlamaSession &&) noexcept = default;

    // Forgets the cached tokens (the reference's session.cache.reset()).
    void reset() { cache.reset(); }

    llama::StepState *state() { return reinterpret_cast<llama::StepState *>(workspace.state.data()); }
};

// What the C ABI drives; implemented by LlamaModelT<float> and LlamaModelT<bf16>.
class LlamaRuntime {
  public:
    using Session = LlamaSession;
    virtual ~LlamaRuntime() = default;
    virtual const ModelConfig &config() const = 0;
    virtual const char *weight_dtype() const = 0; // "float32" | "bfloat16"
    virtual std::unique_ptr<Session> new_session(int max_seq_len) const = 0;
    virtual int32_t prefill(Session &s, const std::vector<int32_t> &ids) = 0;
    virtual int32_t decode_step(Session &s, int32_t token) = 0;
    virtual void decode_greedy(Session &s, int32_t token, int n, int32_t *out) = 0;
    virtual std::vector<float> profile_decode_step(Session &s, int32_t token, int32_t *next) = 0;
    virtual float time_decode_stage(Session &s, int stage, int reps) = 0;
    virtual bool is_eos(int32_t token) const = 0;
    virtual std::vector<float> last_logits(Session &s) const = 0;
    virtual void copy_last_logits(Session &s, float *out, int n) const = 0;
    virtual std::vector<float> hidden_state(Session &s, int rows) const = 0;
    virtual std::vector<std::vector<float>> debug_prefill(Session &s, const std::vector<int32_t> &ids) = 0;
};

// The Llama runtime over WT-typed weights (reference: LlamaModelT<WT>,
// include/models/llama.cuh:78-291; LlamaModel = fp32, LlamaModelBF16 = bf16).
template <typename WT> class LlamaModelT final : public LlamaRuntime {
    static constexpr bool kBf16 = std::is_same_v<WT, bf16>;
    static constexpr int kRowScale = llama::kRowScale<WT>;

  public:
    using Session = LlamaSession;
    static constexpr int kMaxSeqLen = detail::kAttnDecodeMaxLen; // 8192

    // Loads an OPWPACK1 pack of this model's dtype (scripts/llama/pack_format.py layout).
    static LlamaModelT load(const PackReader &pack) {
        const ModelConfig cfg = ModelConfig::from_manifest(pack.manifest());
        check_supported(cfg);
        return LlamaModelT(cfg, ModelWeights<WT>::load(pack, cfg));
    }
    static LlamaModelT load(const std::string &pack_path) { return load(PackReader(pack_path)); }

    // Seeded random weights: projections and embedding ~ N(0, std) (bf16:
    // rounded to nearest-even), norms per NormInit (bf16: rounded values).
    static LlamaModelT load_random(const ModelConfig &cfg, uint64_t seed, float std, NormInit norms) {
        check_supported(cfg);
        return LlamaModelT(cfg, ModelWeights<WT>::random(cfg, seed, std, norms));
    }

    const ModelConfig &config() const override { return cfg_; }
    const char *weight_dtype() const override { return kBf16 ? "bfloat16" : "float32"; }
    const ModelWeights<WT> &weights() const { return w_; }

    // A session of up to max_seq_len tokens (reference: create_session, llama.cuh:92-96).
    Session create_session(int max_seq_len) const {
        if (max_seq_len <= 0 || max_seq_len > kMaxSeqLen)
            throw std::invalid_argument("max_seq_len must be in (0, 8192]");
        return Session(cfg_, max_seq_len, kBf16);
    }
    std::unique_ptr<Session> new_session(int max_seq_len) const override {
        return std::make_unique<Session>(create_session(max_seq_len));
    }

    // Runs the prompt, fills the cache, returns the first generated token.
    int32_t prefill(Session &s, const std::vector<int32_t> &ids) override {
        check_prefill(s, ids);
        run_prefill(s, ids, nullptr);
        return s.h_state->next;
    }

    // Appends `token` at position length and returns the argmax of the next token.
    int32_t decode_step(Session &s, int32_t token) override {
        if (token < 0 || token >= cfg_.vocab_size)
            throw std::invalid_argument("token id outside the vocabulary");
        if (s.cache.length >= s.cache.max_seq_len)
            throw std::invalid_argument("session capacity exhausted");
        s.h_state->token = token;
        s.h_state->pos = s.cache.length;
        s.h_state->next = -1;
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.state(), s.h_state, sizeof(llama::StepState), hipMemcpyHostToDevice,
                                         s.stream));
        launch_decode(s);
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.h_state, s.state(), sizeof(llama::StepState), hipMemcpyDeviceToHost,
                                         s.stream));
        synchronize(s.stream);
        s.cache.length += 1;
        s.last_prefill_rows = 0;
        return s.h_state->next;
    }

    // n greedy decode steps from `token` (appended at position length): out[i]
    // is the token step i produces, the input of step i + 1. The argmax kernel
    // of each step records its token in gen[pos] and advances the device step
    // state (chain = 1), so the steps are launched back to back and the host
    // waits once, instead of once per token as decode_step does. The kernels
    // and results are those of n decode_step calls.
    void decode_greedy(Session &s, int32_t token, int n, int32_t *out) override {
        if (n <= 0)
            return;
        if (!out)
            throw std::invalid_argument("decode_greedy needs an output buffer");
        if (token < 0 || token >= cfg_.vocab_size)
            throw std::invalid_argument("token id outside the vocabulary");
        if (n > s.cache.max_seq_len - s.cache.length)
            throw std::invalid_argument("session capacity exhausted");
        struct ChainOff { // every other path runs with chain = 0
            llama::StepState *h;
            ~ChainOff() { h->chain = 0; }
        } chain_off{s.h_state};
        const int pos0 = s.cache.length;
        *s.h_state = llama::StepState{token, pos0, -1, 1};
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.state(), s.h_state, sizeof(llama::StepState), hipMemcpyHostToDevice,
                                         s.stream));
        // At most 16 steps are queued ahead of the GPU: enough that it never waits for the host,
        // few enough that eager mode (82 kernels per step) keeps a short queue. An event closes
        // every group of kDecodeGroup steps; a group starts once the group 4 before it has
        // completed. A whole group is one launch of a graph holding its steps.
        constexpr int kGroup = kDecodeGroup, kGroups = 2;
        while (static_cast<int>(s.step_events.size()) < kGroups) {
            hipEvent_t e;
            OPWORKS_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
            s.step_events.push_back(e);
        }
        for (int i = 0; i < n;) {
            const int g = i / kGroup;
            if (g >= kGroups)
                OPWORKS_HIP_CHECK(hipEventSynchronize(s.step_events[g % kGroups]));
            const int steps = n - i < kGroup ? n - i : kGroup;
            if (steps == kGroup)
                launch_decode_group(s);
            else
                for (int k = 0; k < steps; ++k)
                    launch_decode(s);
            i += steps;
            OPWORKS_HIP_CHECK(hipEventRecord(s.step_events[g % kGroups], s.stream));
        }
        OPWORKS_HIP_CHECK(hipMemcpyAsync(out, s.workspace.gen.data() + pos0, sizeof(int32_t) * static_cast<size_t>(n),
                                         hipMemcpyDeviceToHost, s.stream));
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.h_state, s.state(), sizeof(llama::StepState), hipMemcpyDeviceToHost,
                                         s.stream));
        synchronize(s.stream);
        s.last_prefill_rows = 0;
        if (s.h_state->chain == 0) {
            // a step produced no valid token and stopped the chain: the steps up to and including it
            // appended their tokens (the later queued steps recomputed it in place)
            const int failed = s.h_state->pos - pos0;
            s.cache.length = s.h_state->pos + 1;
            throw std::runtime_error("decode_greedy: step " + std::to_string(failed) + " produced no token id (argmax " +
                                     std::to_string(s.h_state->next) + ": no finite winner among the logits)");
        }
        s.cache.length += n;
    }

    // One decode step launched eagerly with an event before every kernel and
    // one after the last, all on the session stream; returns the kernel
    // durations in launch order (per layer: qkv_rope, attention, o_proj,
    // gate_up, down; then lm_head) and the next token in *next.
    std::vector<float> profile_decode_step(Session &s, int32_t token, int32_t *next) override {
        if (token < 0 || token >= cfg_.vocab_size)
            throw std::invalid_argument("token id outside the vocabulary");
        if (s.cache.length >= s.cache.max_seq_len)
            throw std::invalid_argument("session capacity exhausted");
        s.h_state->token = token;
        s.h_state->pos = s.cache.length;
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.state(), s.h_state, sizeof(llama::StepState), hipMemcpyHostToDevice,
                                         s.stream));
        std::vector<hipEvent_t> ev;
        const std::function<void()> rec = [&] {
            hipEvent_t e;
            OPWORKS_HIP_CHECK(hipEventCreate(&e));
            OPWORKS_HIP_CHECK(hipEventRecord(e, s.stream));
            ev.push_back(e);
        };
        tick_ = &rec;
        try {
            enqueue_decode(s);
        } catch (...) {
            tick_ = nullptr;
            throw;
        }
        tick_ = nullptr;
        rec();
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.h_state, s.state(), sizeof(llama::StepState), hipMemcpyDeviceToHost,
                                         s.stream));
        synchronize(s.stream);
        std::vector<float> ms(ev.size() - 1);
        for (size_t i = 0; i + 1 < ev.size(); ++i)
            OPWORKS_HIP_CHECK(hipEventElapsedTime(&ms[i], ev[i], ev[i + 1]));
        for (hipEvent_t e : ev)
            (void)hipEventDestroy(e);
        s.cache.length += 1;
        if (next)
            *next = s.h_state->next;
        return ms;
    }

    // Average duration in microseconds of one launch of a decode stage
    // (0 qkv_rope, 1 attention partial + combine, 2 o_proj, 3 gate_up,
    // 4 down, 5 lm_head + argmax): the stage alone is enqueued for every layer
    // in order, `reps` times, between two events on the session stream, so
    // consecutive launches stream different layers' weights. Uses the state
    // of the last decode step; the KV entry it writes lies past the session's
    // length and is overwritten by the next real step. Requires a prefill.
    float time_decode_stage(Session &s, int stage, int reps) override {
        if (stage < 0 || stage > 5)
            throw std::invalid_argument("decode stage must be in [0, 5]");
        if (reps <= 0)
            throw std::invalid_argument("reps must be positive");
        if (s.cache.length == 0 || s.cache.length >= s.cache.max_seq_len)
            throw std::invalid_argument("time_decode_stage needs a prefilled session with free capacity");
        s.h_state->token = 0;
        s.h_state->pos = s.cache.length;
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.state(), s.h_state, sizeof(llama::StepState), hipMemcpyHostToDevice,
                                         s.stream));
        hipEvent_t e0, e1;
        OPWORKS_HIP_CHECK(hipEventCreate(&e0));
        OPWORKS_HIP_CHECK(hipEventCreate(&e1));
        stage_mask_ = 1u << stage;
        try {
            enqueue_decode(s); // warm-up pass
            OPWORKS_HIP_CHECK(hipEventRecord(e0, s.stream));
            for (int r = 0; r < reps; ++r)
                enqueue_decode(s);
            OPWORKS_HIP_CHECK(hipEventRecord(e1, s.stream));
        } catch (...) {
            stage_mask_ = kAllStages;
            throw;
        }
        stage_mask_ = kAllStages;
        synchronize(s.stream);
        float ms = 0.f;
        OPWORKS_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        const int per_pass = stage == 5 ? 1 : cfg_.num_layers;
        return 1e3f * ms / float(reps * per_pass);
    }

    bool is_eos(int32_t token) const override {
        return std::find(cfg_.eos_token_ids.begin(), cfg_.eos_token_ids.end(), token) != cfg_.eos_token_ids.end();
    }

    std::vector<float> last_logits(Session &s) const override {
        std::vector<float> out(static_cast<size_t>(cfg_.vocab_size));
        copy_last_logits(s, out.data(), cfg_.vocab_size);
        return out;
    }

    void copy_last_logits(Session &s, float *out, int n) const override {
        if (n != cfg_.vocab_size)
            throw std::invalid_argument("logits buffer must hold vocab_size floats");
        OPWORKS_HIP_CHECK(hipMemcpyAsync(out, s.workspace.logits.data(), sizeof(float) * static_cast<size_t>(n),
                                         hipMemcpyDeviceToHost, s.stream));
        synchronize(s.stream);
    }

    // Residual stream of the last prefill: rows x H.
    std::vector<float> hidden_state(Session &s, int rows) const override {
        if (rows <= 0 || rows > s.cache.max_seq_len)
            throw std::invalid_argument("rows outside the session capacity");
        std::vector<float> out(static_cast<size_t>(rows) * cfg_.hidden_size);
        OPWORKS_HIP_CHECK(hipMemcpyAsync(out.data(), s.workspace.hidden.data(), out.size() * sizeof(float),
                                         hipMemcpyDeviceToHost, s.stream));
        synchronize(s.stream);
        return out;
    }

    // Like prefill, also returning the residual stream after the embedding and after each layer.
    std::vector<std::vector<float>> debug_prefill(Session &s, const std::vector<int32_t> &ids) override {
        check_prefill(s, ids);
        std::vector<std::vector<float>> captures;
        const int n = static_cast<int>(ids.size());
        run_prefill(s, ids, [&](int) {
            std::vector<float> h(static_cast<size_t>(n) * cfg_.hidden_size);
            const float *src = n == 1 ? s.workspace.step_hidden.data() : s.workspace.hidden.data();
            OPWORKS_HIP_CHECK(hipMemcpyAsync(h.data(), src, h.size() * sizeof(float), hipMemcpyDeviceToHost,
                                             s.stream));
            synchronize(s.stream);
            captures.push_back(std::move(h));
        });
        return captures;
    }

  private:
    LlamaModelT(const ModelConfig &cfg, ModelWeights<WT> &&w) : cfg_(cfg), w_(std::move(w)) {}

    ModelConfig cfg_;
    ModelWeights<WT> w_;
    // When set (profiling only), called before every kernel of the decode step.
    const std::function<void()> *tick_ = nullptr;
    // Stages enqueued by the decode step (timing only narrows it): bit 0
    // qkv_rope, 1 attention, 2 o_proj, 3 gate_up, 4 down, 5 lm_head + argmax.
    unsigned stage_mask_ = kAllStages;
    static constexpr unsigned kAllStages = 0x3f;
    bool stage_on(int stage) const { return (stage_mask_ >> stage) & 1u; }
    void tick() const {
        if (tick_)
            (*tick_)();
    }

    static void check_supported(const ModelConfig &cfg_) {
        const int H = cfg_.hidden_size, I = cfg_.intermediate_size;
        if (H % 256 != 0 || H / 256 > 16 || (H / 256 & (H / 256 - 1)) != 0)
            throw std::runtime_error("hidden_size must be 256 * {1,2,4,8,16}");
        if (I % 1024 != 0 || I / 1024 > 16 || (I / 1024 & (I / 1024 - 1)) != 0)
            throw std::runtime_error("intermediate_size must be 1024 * {1,2,4,8,16}");
        if (cfg_.head_dim != 64 && cfg_.head_dim != 32)
            throw std::runtime_error("head_dim must be 32 or 64");
        if (cfg_.kv_rep() > 16)
            throw std::runtime_error("at most 16 query heads per kv head");
        if (kBf16 && (H % 512 != 0 || I % 2048 != 0))
            throw std::runtime_error("bf16 weights need hidden_size % 512 == 0 and intermediate_size % 2048 == 0");
    }

    void check_prefill(Session &s, const std::vector<int32_t> &ids) const {
        for (int32_t id : ids)
            if (id < 0 || id >= cfg_.vocab_size)
                throw std::invalid_argument("token id outside the vocabulary");
        if (ids.empty())
            throw std::invalid_argument("prefill requires at least one token");
        if (static_cast<int>(ids.size()) > s.cache.max_seq_len)
            throw std::invalid_argument("prompt exceeds the session capacity");
        if (s.cache.length != 0)
            throw std::invalid_argument("prefill requires a fresh session (reset first)");
    }

    static float *layer_k(Session &s, int l) { return s.cache.k[static_cast<size_t>(l)].data(); }
    static float *layer_v(Session &s, int l) { return s.cache.v[static_cast<size_t>(l)].data(); }

    // ---- decode step (one token at state.pos) -----------------------------
    template <int kV, int kV2> void enqueue_decode_layer(Session &s, int l) const {
        const int H = cfg_.hidden_size, I = cfg_.intermediate_size, D = cfg_.head_dim;
        const int qh = cfg_.num_q_heads, kvh = cfg_.num_kv_heads;
        const int qkv_groups = (qh + 2 * kvh) * (D / 4); // 4 rows each
        hipStream_t st = s.stream;
        const LayerWeights<WT> &lw = w_.layers[static_cast<size_t>(l)];
        llama::QkvArgs<WT> qa{};
        // layer 0 reads the step token's embedding row in the qkv kernel (bf16 rows widened as
        // they are loaded), whose workgroup 0 also writes it into the residual stream
        qa.hidden_in = l == 0 ? nullptr : s.workspace.step_hidden.data();
        qa.embed = w_.embed_tokens.data();
        qa.hidden_out = s.workspace.step_hidden.data();
        qa.gamma = lw.input_norm.data();
        qa.wqkv = lw.qkv_proj.data();
        qa.inv_freq = w_.rope_inv_freq.data();
        qa.q_out = s.workspace.step_q.data();
        qa.kcache = layer_k(s, l);
        qa.vcache = layer_v(s, l);
        qa.state = s.state();
        qa.eps = cfg_.rms_norm_eps;
        qa.qh = qh;
        qa.kvh = kvh;
        qa.D = D;
        qa.cap = s.cache.max_seq_len;
        if (stage_on(0)) {
            tick();
            launch_async(st, llama::qkv_rope_kernel<kV, WT>, qkv_groups, llama::kBlock, qa);
        }
        llama::DecodeAttnArgs aa{};
        aa.q = s.workspace.step_q.data();
        aa.kcache = layer_k(s, l);
        aa.vcache = layer_v(s, l);
        aa.out = s.workspace.step_attn.data();
        aa.partial = s.workspace.attn_partial.data();
        aa.counters = s.workspace.attn_counters.data(); // fused merge: one launch per layer
        aa.len_ptr = s.workspace.state.data() + offsetof(llama::StepState, pos) / sizeof(int32_t); // length pos + 1
        aa.len_bias = 1;
        aa.kv_rep = cfg_.kv_rep();
        aa.D = D;
        aa.cap = s.cache.max_seq_len;
        aa.max_chunks = s.workspace.sizes.attn_chunks;
        aa.chunks_per_record = detail::decode_chunks_per_record(aa.kv_rep, aa.max_chunks);
        aa.scale = 1.f / std::sqrt(static_cast<float>(D));
        if (stage_on(1)) {
            tick();
            detail::attention_decode_launch(aa, kvh, st);
        }
        if (stage_on(2)) {
            tick();
            launch_async(st, llama::gemv_residual_kernel<kV, WT>, detail::blocks_for64(H, llama::kRows),
                         llama::kBlock, lw.o_proj.data(), s.workspace.step_attn.data(), s.workspace.step_hidden.data(), H);
        }
        if (stage_on(3)) {
            tick();
            launch_async(st, llama::swiglu_gemv_kernel<kV, WT>,
                         detail::blocks_for64(2 * I, llama::kWavesPerBlock * kRowScale),
                         llama::kBlock, s.workspace.step_hidden.data(), lw.post_norm.data(), cfg_.rms_norm_eps, lw.gate_up_proj.data(),
                         s.workspace.step_act.data(), I);
        }
        if (stage_on(4)) {
            tick();
            launch_async(st, llama::down_residual_kernel<kV2, WT>, detail::blocks_for64(H, llama::kRows), llama::kBlock,
                         lw.down_proj.data(), s.workspace.step_act.data(), s.workspace.step_hidden.data(), H);
        }
    }

    // All layers then the LM head; `hook(l)` (debug only) runs after layer l.
    void enqueue_decode(Session &s, const std::function<void(int)> &hook = nullptr) const {
        dispatch_widths([&](auto v, auto v2) {
            constexpr int kV = decltype(v)::value, kV2 = decltype(v2)::value;
            for (int l = 0; l < cfg_.num_layers; ++l) {
                enqueue_decode_layer<kV, kV2>(s, l);
                if (hook)
                    hook(l);
            }
            if (stage_on(5))
                enqueue_lm_head<kV>(s, s.workspace.step_hidden.data());
        });
    }

    template <int kV> void enqueue_lm_head(Session &s, const float *hidden_row) const {
        llama::LmHeadArgs<WT> la{};
        la.hidden_row = hidden_row;
        la.gamma = w_.final_norm.data();
        la.embed = w_.embed_tokens.data();
        la.logits = s.workspace.logits.data();
        la.best_val = s.workspace.lm_best_val.data();
        la.best_idx = s.workspace.lm_best_idx.data();
        la.eps = cfg_.rms_norm_eps;
        la.vocab = cfg_.vocab_size;
        tick();
        const int records = static_cast<int>(
            detail::blocks_for64(cfg_.vocab_size, llama::kLmRows * kRowScale * llama::kWavesPerBlock));
        launch_async(s.stream, llama::lm_head_kernel<kV, WT>, records, llama::kBlock, la);
        launch_async(s.stream, llama::argmax_records_kernel, llama::kArgmaxGroups, 256, s.workspace.lm_best_val.data(),
                     s.workspace.lm_best_idx.data(), records, s.workspace.lm_part_val.data(), s.workspace.lm_part_idx.data(),
                     s.workspace.lm_counter.data(), s.state(), s.workspace.gen.data(), cfg_.vocab_size);
    }

    // Calls f(IntTag<H / 256>, IntTag<I / 1024>); bf16 rows need whole 8-weight
    // packs per lane, so the narrowest widths exist for fp32 only (check_supported
    // rejects them for bf16 before any launch).
    template <typename F> void dispatch_widths(F &&f) const {
        const int v = cfg_.hidden_size / 256, v2 = cfg_.intermediate_size / 1024;
        auto call = [&](auto vt, auto v2t) {
            if constexpr (!kBf16 || (decltype(vt)::value % 2 == 0 && decltype(v2t)::value % 2 == 0))
                f(vt, v2t);
            else
                throw std::runtime_error("unsupported widths for bf16 weights");
        };
        auto with_v2 = [&](auto vt) {
            switch (v2) {
            case 1: call(vt, detail::IntTag<1>{}); break;
            case 2: call(vt, detail::IntTag<2>{}); break;
            case 4: call(vt, detail::IntTag<4>{}); break;
            case 8: call(vt, detail::IntTag<8>{}); break;
            case 16: call(vt, detail::IntTag<16>{}); break;
            default: throw std::runtime_error("unsupported intermediate_size");
            }
        };
        switch (v) {
        case 1: with_v2(detail::IntTag<1>{}); break;
        case 2: with_v2(detail::IntTag<2>{}); break;
        case 4: with_v2(detail::IntTag<4>{}); break;
        case 8: with_v2(detail::IntTag<8>{}); break;
        case 16: with_v2(detail::IntTag<16>{}); break;
        default: throw std::runtime_error("unsupported hidden_size");
        }
    }

    // Replays the session's decode graph (captured on first use). With
    // OPWORKS_DECODE_GRAPH=0 in the environment the same kernels are enqueued
    // one by one instead, for tools that do not follow graph launches.
    static bool use_graph() {
        static const bool on = [] {
            const char *v = std::getenv("OPWORKS_DECODE_GRAPH");
            return !(v && v[0] == '0');
        }();
        return on;
    }

    void launch_decode(Session &s) const {
        if (!use_graph()) {
            enqueue_decode(s);
            return;
        }
        if (!s.graph_exec)
            capture_decode_graph(s);
        OPWORKS_HIP_CHECK(hipGraphLaunch(s.graph_exec, s.stream));
    }

    // kDecodeGroup chained greedy steps (device state with chain = 1): one graph launch, with
    // no gap between the steps' graphs (about 8 us per step in separate launches).
    static constexpr int kDecodeGroup = 16;
    void launch_decode_group(Session &s) const {
        if (!use_graph()) {
            for (int k = 0; k < kDecodeGroup; ++k)
                enqueue_decode(s);
            return;
        }
        if (!s.group_exec)
            capture_graph(s, kDecodeGroup, s.group_graph, s.group_exec);
        OPWORKS_HIP_CHECK(hipGraphLaunch(s.group_exec, s.stream));
    }

    void capture_decode_graph(Session &s) const { capture_graph(s, 1, s.graph, s.graph_exec); }

    void capture_graph(Session &s, int steps, hipGraph_t &graph, hipGraphExec_t &exec) const {
        OPWORKS_HIP_CHECK(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal));
        try {
            for (int k = 0; k < steps; ++k)
                enqueue_decode(s);
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(s.stream, &g);
            if (g)
                (void)hipGraphDestroy(g);
            throw;
        }
        OPWORKS_HIP_CHECK(hipStreamEndCapture(s.stream, &graph));
        OPWORKS_HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    }

    // ---- prefill -------------------------------------------------------------
    void run_prefill(Session &s, const std::vector<int32_t> &ids, const std::function<void(int)> &hook) {
        const int n = static_cast<int>(ids.size());
        if (n == 1) { // one row: the decode kernels (the reference's rows == 1 path)
            s.h_state->token = ids[0];
            s.h_state->pos = 0;
            s.h_state->next = -1;
            OPWORKS_HIP_CHECK(hipMemcpyAsync(s.state(), s.h_state, sizeof(llama::StepState),
                                             hipMemcpyHostToDevice, s.stream));
            if (hook)
                run_decode_layers_with_hook(s, hook);
            else
                launch_decode(s);
        } else {
            OPWORKS_HIP_CHECK(hipMemcpyAsync(s.workspace.tokens.data(), ids.data(), sizeof(int32_t) * n, hipMemcpyHostToDevice,
                                             s.stream));
            s.h_state->pos = n; // the next decode position
            OPWORKS_HIP_CHECK(hipMemcpyAsync(s.state(), s.h_state, sizeof(llama::StepState),
                                             hipMemcpyHostToDevice, s.stream));
            enqueue_prefill(s, n, hook);
        }
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.h_state, s.state(), sizeof(llama::StepState), hipMemcpyDeviceToHost,
                                         s.stream));
        synchronize(s.stream);
        s.cache.length = n;
        s.last_prefill_rows = n;
    }

    // Single-row prefill with per-layer captures: the decode kernels launched eagerly.
    void run_decode_layers_with_hook(Session &s, const std::function<void(int)> &hook) {
        // Layer 0's first kernel writes the embedding row into the residual stream;
        // copy it beforehand so the "after embedding" capture sees it.
        const int H = cfg_.hidden_size;
        if constexpr (kBf16)
            launch_async(s.stream, llama::embed_token_kernel<WT>, detail::blocks_for64(H, 256), 256, w_.embed_tokens.data(),
                         s.state(), s.workspace.step_hidden.data(), H);
        else
            OPWORKS_HIP_CHECK(hipMemcpyAsync(s.workspace.step_hidden.data(), w_.embed_tokens.data() + int64_t(s.h_state->token) * H,
                                             sizeof(float) * H, hipMemcpyDeviceToDevice, s.stream));
        hook(-1);
        enqueue_decode(s, hook);
    }

    // Prefill projection C (per kStore) = A[M][K] W[N][K]^T: the fp32 MFMA GEMM
    // for fp32 weights; for bf16 weights the bf16 MFMA GEMM with A rounded to
    // bf16 on load from 16 rows (the reference's linear_mma_bf16 path,
    // models/llama.cuh:190-199), and below 16 rows the fp32 MFMA GEMM with fp32
    // inputs against the widened bf16 weights, as the reference's linear_dispatch does.
    // Outputs with too few tiles to fill the GPU (o_proj, down, qkv at a few
    // hundred rows) split K across workgroups into the session's workspace.
    // `reduce` (optional, split-K outputs): run in place of the split-K reduction kernel, see
    // gemm_f32_launch_splitk. Returns true when K was split (and `reduce`, if given, ran).
    template <detail::GemmStore kStore = detail::GemmStore::store, typename Reduce = std::nullptr_t>
    bool project(Session &s, const float *A, const WT *W, float *C, int M, int N, int K, hipStream_t st,
                 Reduce reduce = nullptr) const {
        using detail::IdentityEpilogue;
        constexpr bool kSplittable = kStore != detail::GemmStore::swiglu;
        const auto *Wb = reinterpret_cast<const uint16_t *>(W);
        if constexpr (kBf16) {
            // 2..15 rows: fp32 inputs against the widened bf16 weights, as the reference's
            // linear_dispatch does below 16 rows (include/models/llama.cuh:190-199)
            if (M < 16) {
                if constexpr (kSplittable)
                    return detail::gemm_f32_launch_splitk<detail::BLayout::nk, IdentityEpilogue, kStore, uint16_t>(
                        A, Wb, nullptr, C, M, N, K, IdentityEpilogue{}, s.workspace.splitk.data(), s.workspace.splitk.size(), st,
                        reduce);
                detail::gemm_f32_launch<detail::BLayout::nk, IdentityEpilogue, kStore, uint16_t>(
                    A, Wb, nullptr, C, M, N, K, IdentityEpilogue{}, st);
                return false;
            }
        }
        if constexpr (kBf16) {
            // From 16 rows the input is rounded to bf16 (nearest-even, the rounding the reference's
            // tensor-core GEMM applies as it stages X, include/ops/linear_mma.cuh:49) by a pass of its
            // own, then the GEMM loads both operands straight into LDS: the same products and sums
            // as rounding while staging (gate/up at T = 512: 77 -> 63.5 us per layer), on tiles
            // sized to the row count (gemm_bf16_launch_direct).
            auto &xb = s.workspace.x_bf16;
            if (int64_t(M) * K <= xb.size()) {
                auto *bits = reinterpret_cast<uint16_t *>(xb.data());
                launch_async(st, detail::convert_f32_bf16_kernel, detail::stream_grid(int64_t(M) * K), 256, A, bits,
                             int64_t(M) * K);
                return detail::gemm_bf16_launch_direct<IdentityEpilogue, kStore>(
                    bits, Wb, nullptr, C, M, N, K, IdentityEpilogue{}, s.workspace.splitk.data(), s.workspace.splitk.size(),
                    st, reduce);
            }
        }
        if constexpr (kBf16 && kSplittable) { // (no hook: the reduction kernel stores, the caller norms)
            detail::gemm_bf16_launch_splitk<float, IdentityEpilogue, kStore>(
                A, Wb, nullptr, C, M, N, K, IdentityEpilogue{}, s.workspace.splitk.data(), s.workspace.splitk.size(), st);
        } else if constexpr (kBf16) {
            detail::gemm_bf16_launch<float, IdentityEpilogue, kStore>(A, Wb, nullptr, C, M, N, K, IdentityEpilogue{},
                                                                      st);
        } else if constexpr (kSplittable) { // fp32 MFMA kernels: the oracle parity of the logits
            return detail::gemm_f32_launch_splitk<detail::BLayout::nk, IdentityEpilogue, kStore>(
                A, W, nullptr, C, M, N, K, IdentityEpilogue{}, s.workspace.splitk.data(), s.workspace.splitk.size(), st,
                reduce);
        } else { // the gate/up projection (SwiGLU store) on bf16x6 products, the others fp32 MFMA
            detail::gemm_f32_launch<detail::BLayout::nk, IdentityEpilogue, kStore>(
                A, W, nullptr, C, M, N, K, IdentityEpilogue{}, st, 1, kStore == detail::GemmStore::swiglu);
        }
        return false;
    }

    void enqueue_prefill(Session &s, int n, const std::function<void(int)> &hook) {
        const int H = cfg_.hidden_size, I = cfg_.intermediate_size, D = cfg_.head_dim;
        const int qh = cfg_.num_q_heads, kvh = cfg_.num_kv_heads, qkvw = cfg_.qkv_width();
        hipStream_t st = s.stream;
        launch_async(st, llama::embedding_kernel<WT>, detail::stream_grid(int64_t(n) * H / 4), 256, w_.embed_tokens.data(),
                     s.workspace.tokens.data(), s.workspace.hidden.data(), n, H);
        if (hook)
            hook(-1);
        // bf16 weights from 16 rows: every projection input is written as bf16 bits by the kernel
        // that produces it (RMSNorm, the head merge, the gate/up SwiGLU store), the rounding the
        // reference's tensor-core GEMM applies to X as it loads it (include/ops/linear_mma.cuh:49),
        // and the GEMMs load both operands straight into LDS. At T = 512 this removed 64 rounding
        // passes (6 us each) and halved those inputs' bytes.
        const bool xb = kBf16 && n >= 16 && s.workspace.x_bf16.size() >= int64_t(n) * std::max(H, qh * D);
        auto *xbits = reinterpret_cast<uint16_t *>(s.workspace.x_bf16.data());
        auto *act_bits = reinterpret_cast<uint16_t *>(s.workspace.act.data()); // [T][I] bf16 in the fp32 buffer
        using detail::GemmStore;
        using detail::IdentityEpilogue;
        auto direct = [&](auto store_tag, const uint16_t *A, const WT *W, float *C, int N, int K) {
            detail::gemm_bf16_launch_direct<IdentityEpilogue, decltype(store_tag)::value>(
                A, reinterpret_cast<const uint16_t *>(W), nullptr, C, n, N, K, IdentityEpilogue{},
                s.workspace.splitk.data(), s.workspace.splitk.size(), st);
        };
        using StoreTag = std::integral_constant<GemmStore, GemmStore::store>;
        using ResidualTag = std::integral_constant<GemmStore, GemmStore::residual>;
        using SwigluBf16Tag = std::integral_constant<GemmStore, GemmStore::swiglu_bf16>;
        float *hidden = s.workspace.hidden.data(), *normed = s.workspace.normed.data();
        const float eps = cfg_.rms_norm_eps;
        auto norm = [&](const float *gamma) {
            if (xb)
                detail::rms_norm_to_bf16(hidden, gamma, xbits, n, H, eps, st);
            else
                ops::rms_norm(hidden, gamma, normed, n, H, eps, st);
        };
        // A residual projection (o_proj, down) whose output RMSNorm(hidden) * gamma feeds the next
        // projection: when K is split, the norm runs inside the split-K reduction (one row pass and
        // one launch fewer); returns whether it did. A_f32 / A_bits: the fp32 or bf16 input.
        auto residual_then_norm = [&](const float *A_f32, const uint16_t *A_bits, const WT *W, int K,
                                      const float *gamma) -> bool {
            const bool fusable = gamma && detail::splitk_residual_rms_norm_ok(
                                              n, H, hidden, gamma, xb ? static_cast<const void *>(xbits) : normed);
            auto reduce = [&](float *ws, int splits) {
                if (xb)
                    detail::splitk_residual_rms_norm<uint16_t>(ws, splits, hidden, gamma, xbits, n, H, eps, st);
                else
                    detail::splitk_residual_rms_norm<float>(ws, splits, hidden, gamma, normed, n, H, eps, st);
            };
            if (!fusable) {
                if (xb)
                    direct(ResidualTag{}, A_bits, W, hidden, H, K);
                else
                    project<GemmStore::residual>(s, A_f32, W, hidden, n, H, K, st);
                return false;
            }
            if (xb)
                return detail::gemm_bf16_launch_direct<IdentityEpilogue, GemmStore::residual>(
                    A_bits, reinterpret_cast<const uint16_t *>(W), nullptr, hidden, n, H, K, IdentityEpilogue{},
                    s.workspace.splitk.data(), s.workspace.splitk.size(), st, reduce);
            return project<GemmStore::residual>(s, A_f32, W, hidden, n, H, K, st, reduce);
        };
        bool input_normed = false; // layer l's input norm ran in layer l - 1's down reduction
        for (int l = 0; l < cfg_.num_layers; ++l) {
            const LayerWeights<WT> &lw = w_.layers[static_cast<size_t>(l)];
            if (!input_normed)
                norm(lw.input_norm.data());
            // RoPE + head split + KV append; when the qkv projection splits K, this pass sums the
            // partial tiles itself in place of the split-K reduction
            auto rope_split = [&](const float *src, int splits) {
                launch_async(st, llama::rope_split_kernel, detail::stream_grid(int64_t(n) * (qh + 2 * kvh) * (D / 2)),
                             256, src, splits, w_.rope_inv_freq.data(), s.workspace.q_heads.data(), layer_k(s, l),
                             layer_v(s, l), n, qh, kvh, D, s.cache.max_seq_len, 0);
            };
            auto rope_from_partials = [&](float *ws, int splits) { rope_split(ws, splits); };
            const bool qkv_split =
                xb ? detail::gemm_bf16_launch_direct<IdentityEpilogue, GemmStore::store>(
                         xbits, reinterpret_cast<const uint16_t *>(lw.qkv_proj.data()), nullptr, s.workspace.qkv.data(),
                         n, qkvw, H, IdentityEpilogue{}, s.workspace.splitk.data(), s.workspace.splitk.size(), st,
                         rope_from_partials)
                   : project(s, normed, lw.qkv_proj.data(), s.workspace.qkv.data(), n, qkvw, H, st, rope_from_partials);
            if (!qkv_split)
                rope_split(s.workspace.qkv.data(), 0);
            // the attention writes its rows with the heads merged, [T][qh * D], as o_proj reads them
            // (bf16 bits for the bf16 GEMM), so no separate merge pass runs
            ops::attention_prefill_ws(s.workspace.q_heads.data(), layer_k(s, l), layer_v(s, l),
                                      xb ? reinterpret_cast<float *>(xbits) : s.workspace.attn_out.data(), n, n, 0, qh,
                                      cfg_.kv_rep(), D, s.cache.max_seq_len, s.workspace.attn_split.data(),
                                      s.workspace.attn_split.size(), s.workspace.attn_split_counters.data(),
                                      s.workspace.attn_split_counters.size(), -1, st, true, xb);
            if (!residual_then_norm(s.workspace.attn_out.data(), xbits, lw.o_proj.data(), qh * D, lw.post_norm.data()))
                norm(lw.post_norm.data());
            if (xb)
                direct(SwigluBf16Tag{}, xbits, lw.gate_up_proj.data(), reinterpret_cast<float *>(act_bits), 2 * I, H);
            else
                project<GemmStore::swiglu>(s, normed, lw.gate_up_proj.data(), s.workspace.act.data(), n, 2 * I, H, st);
            const float *next_gamma =
                l + 1 < cfg_.num_layers ? w_.layers[static_cast<size_t>(l) + 1].input_norm.data() : nullptr;
            input_normed = residual_then_norm(s.workspace.act.data(), act_bits, lw.down_proj.data(), I, next_gamma);
            if (hook)
                hook(l);
        }
        dispatch_widths(
            [&](auto v, auto) { enqueue_lm_head<decltype(v)::value>(s, s.workspace.hidden.data() + int64_t(n - 1) * H); });
    }
};

using LlamaModel = LlamaModelT<float>;
using LlamaModelBF16 = LlamaModelT<bf16>;

// Loads a pack and picks the model from its dtype (reference: src/llama_c_api.cu:56-73).
inline std::unique_ptr<LlamaRuntime> load_llama(const std::string &pack_path) {
    PackReader pack(pack_path);
    if (pack.dtype() == "float32")
        return std::make_unique<LlamaModel>(LlamaModel::load(pack));
    if (pack.dtype() == "bfloat16")
        return std::make_unique<LlamaModelBF16>(LlamaModelBF16::load(pack));
    throw std::runtime_error("unsupported pack dtype " + pack.dtype());
}

// Seeded random weights of either storage type.
inline std::unique_ptr<LlamaRuntime> load_llama_random(const ModelConfig &cfg, uint64_t seed, float std,
                                                       NormInit norms, bool bf16_weights) {
    if (bf16_weights)
        return std::make_unique<LlamaModelBF16>(LlamaModelBF16::load_random(cfg, seed, std, norms));
    return std::make_unique<LlamaModel>(LlamaModel::load_random(cfg, seed, std, norms));
}

} // namespace opworks

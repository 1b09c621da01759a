#pragma once

// Llama-3.x decoder on MI355X, fp32 weights (reference: include/models/llama.cuh:43-293).
//
// Same model-level contract as the reference's LlamaModelT / LlamaSession:
// load (pack or seeded random init), create_session(max_seq <= 8192),
// prefill (fresh session, returns the first generated token), decode_step
// (appends one token, returns the next), is_eos, last_logits,
// copy_last_logits, hidden_state, debug_prefill. K is cached post-RoPE, V as
// projected; the LM head is the tied embedding applied to the last row.
//
// MI355X layout of the weights in HBM (differs from the HF layout on purpose):
//  * wqkv  [(qh + 2 kvh) D][H]  q, k and v rows concatenated: one GEMV/GEMM;
//  * wgu   [2 I][H]             gate_i and up_i rows interleaved, so one wave's
//                               rows give silu(gate) * up directly;
//  * wo [H][qh D], wdown [H][I], embed [V][H] as in HF.
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
#include <vector>

#include "../core/hip_utils.hpp"
#include "../core/random.hpp"
#include "../core/typed_device_buffer.hpp"
#include "../ops/attention.hpp"
#include "../ops/gemm_f32.hpp"
#include "../ops/rms_norm.hpp"
#include "../ops/gemm_bf16.hpp"
#include "../runtime/model_config.hpp"
#include "../runtime/pack_reader.hpp"
#include "llama_kernels.hpp"

namespace opworks {

namespace llama_detail {

// Stream ids of the seeded random initialisation (see random.hpp). Logical
// tensors are generated in the HF layout: element (o, i) of a [out][in]
// projection is draw o * in + i of its stream.
constexpr uint64_t kStreamEmbed = 1;
constexpr uint64_t kStreamFinalNorm = 2;
inline uint64_t layer_stream(int layer, int which) { return 64 + 16 * static_cast<uint64_t>(layer) + which; }
enum LayerTensor { kQ = 0, kK = 1, kV = 2, kO = 3, kGate = 4, kUp = 5, kDown = 6, kInNorm = 7, kPostNorm = 8 };

template <typename T> __device__ __forceinline__ T store_as(float v) {
    if constexpr (std::is_same_v<T, bf16>)
        return bf16{float_to_bf16_rne(v)};
    else
        return v;
}

// dst[(r * row_stride + row_offset) * cols + c] = N(mean, sd) draw r * cols + c
// (rounded to nearest-even for a bf16 destination)
template <typename T>
__global__ __launch_bounds__(256) static void fill_rows_normal_kernel(T *dst, int64_t rows, int cols, int row_stride,
                                                                      int row_offset, uint64_t key, float mean,
                                                                      float sd) {
    OPWORKS_GRID_LOOP(i, rows * cols) {
        const int64_t r = i / cols, c = i % cols;
        dst[(r * row_stride + row_offset) * cols + c] = store_as<T>(rng::normal(key, static_cast<uint64_t>(i), mean, sd));
    }
}
// round_bf16: the values a bf16 pack would hold, kept in fp32
__global__ __launch_bounds__(256) static void fill_uniform_kernel(float *dst, int64_t n, uint64_t key, float lo,
                                                                  float hi, bool round_bf16) {
    OPWORKS_GRID_LOOP(i, n) {
        const float v = rng::uniform(key, static_cast<uint64_t>(i), lo, hi);
        dst[i] = round_bf16 ? bf16_to_float(float_to_bf16_rne(v)) : v;
    }
}
__global__ __launch_bounds__(256) static void fill_const_kernel(float *dst, int64_t n, float v) {
    OPWORKS_GRID_LOOP(i, n) { dst[i] = v; }
}

inline int fill_grid(int64_t n) {
    const int64_t need = detail::blocks_for64(n, 256), cap = 65536;
    return static_cast<int>(need < cap ? (need > 0 ? need : 1) : cap);
}

} // namespace llama_detail

// Norm weights of the seeded init: ones (HF init) or U[0.5, 1.5] (exercises gamma in tests).
enum class NormInit { ones = 0, uniform = 1 };

// WT: storage of the projections and the embedding (float or bf16); norm
// weights and every activation stay fp32 (reference: runtime/weights.cuh:16-27).
template <typename WT> struct LlamaLayerWeights {
    TypedDeviceBuffer<float> input_norm, post_norm; // [H]
    TypedDeviceBuffer<WT> wqkv;                     // [(qh + 2 kvh) D][H]
    TypedDeviceBuffer<WT> wo;                       // [H][qh D]
    TypedDeviceBuffer<WT> wgu;                      // [2 I][H], rows gate_0, up_0, gate_1, ...
    TypedDeviceBuffer<WT> wdown;                    // [H][I]
};

template <typename WT> struct LlamaWeights {
    TypedDeviceBuffer<WT> embed;         // [V][H], also the LM head
    TypedDeviceBuffer<float> final_norm; // [H]
    TypedDeviceBuffer<float> inv_freq;   // [D/2]
    std::vector<LlamaLayerWeights<WT>> layers;
};

struct LlamaSession {
    int max_seq_len = 0;
    int length = 0; // valid cache entries
    hipStream_t stream = nullptr;
    // KV cache: [layer][kvh][cap][D] for K and for V
    TypedDeviceBuffer<float> kcache, vcache;
    // decode step
    TypedDeviceBuffer<float> d_hidden, d_q, d_attn, d_act, logits, attn_partial, lm_best_val;
    TypedDeviceBuffer<int32_t> lm_best_idx, gen, state_buf, ids; // gen[pos]: token chained decode produced at pos
    TypedDeviceBuffer<int32_t> attn_counters; // [kvh] arrival counters of the fused decode attention, zero at rest
    // prefill
    TypedDeviceBuffer<float> hidden, normed, qkv, q_heads, attn_heads, attn, act;
    TypedDeviceBuffer<float> splitk_ws; // partial tiles of split-K projections
    int attn_max_chunks = 0;
    int lm_grid = 0;
    llama::StepState *h_state = nullptr; // pinned
    int32_t *h_token = nullptr;          // pinned
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    std::vector<hipEvent_t> step_events; // chained decode: completion of the steps in flight
    int last_prefill_rows = 0;

    LlamaSession() = default;
    LlamaSession(const LlamaSession &) = delete;
    LlamaSession &operator=(const LlamaSession &) = delete;
    ~LlamaSession() {
        for (hipEvent_t e : step_events)
            (void)hipEventDestroy(e);
        if (graph_exec)
            (void)hipGraphExecDestroy(graph_exec);
        if (graph)
            (void)hipGraphDestroy(graph);
        if (h_state)
            (void)hipHostFree(h_state);
        if (h_token)
            (void)hipHostFree(h_token);
        if (stream)
            (void)hipStreamDestroy(stream);
    }

    // Reset only invalidates the length; stale cache bytes are never read.
    void reset() { length = 0; }

    llama::StepState *state() { return reinterpret_cast<llama::StepState *>(state_buf.data()); }
};

// What the C ABI drives; implemented by LlamaModelT<float> and LlamaModelT<bf16>.
class LlamaRuntime {
  public:
    using Session = LlamaSession;
    virtual ~LlamaRuntime() = default;
    virtual const ModelConfig &config() const = 0;
    virtual const char *weight_dtype() const = 0; // "float32" | "bfloat16"
    virtual std::unique_ptr<Session> create_session(int max_seq_len) const = 0;
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

  public:
    using Session = LlamaSession;
    static constexpr int kMaxSeqLen = detail::kAttnDecodeMaxLen; // 8192

    // Loads an OPWPACK1 pack of this model's dtype (scripts/llama/pack_format.py layout).
    static std::unique_ptr<LlamaModelT> load(const PackReader &pack) {
        if (pack.dtype() != (kBf16 ? "bfloat16" : "float32"))
            throw std::runtime_error(std::string(kBf16 ? "bf16" : "fp32") + " model requires a " +
                                     (kBf16 ? "bfloat16" : "float32") + " pack (got " + pack.dtype() + ")");
        auto m = std::unique_ptr<LlamaModelT>(new LlamaModelT(ModelConfig::from_manifest(pack.manifest())));
        m->check_supported();
        m->allocate();
        m->upload_pack(pack);
        return m;
    }
    static std::unique_ptr<LlamaModelT> load(const std::string &pack_path) { return load(PackReader(pack_path)); }

    // Seeded random weights: projections and embedding ~ N(0, std) (bf16:
    // rounded to nearest-even), norms per NormInit (bf16: rounded values).
    static std::unique_ptr<LlamaModelT> load_random(const ModelConfig &cfg, uint64_t seed, float std,
                                                    NormInit norms) {
        auto m = std::unique_ptr<LlamaModelT>(new LlamaModelT(cfg));
        m->check_supported();
        m->allocate();
        m->init_random(seed, std, norms);
        return m;
    }

    const ModelConfig &config() const override { return cfg_; }
    const char *weight_dtype() const override { return kBf16 ? "bfloat16" : "float32"; }
    const LlamaWeights<WT> &weights() const { return w_; }

    std::unique_ptr<Session> create_session(int max_seq_len) const override {
        if (max_seq_len <= 0 || max_seq_len > kMaxSeqLen)
            throw std::invalid_argument("max_seq_len must be in (0, 8192]");
        auto s = std::make_unique<Session>();
        const int64_t T = max_seq_len, H = cfg_.hidden_size, I = cfg_.intermediate_size;
        const int64_t kvh = cfg_.num_kv_heads, D = cfg_.head_dim, qh = cfg_.num_q_heads, L = cfg_.num_layers;
        s->max_seq_len = max_seq_len;
        OPWORKS_HIP_CHECK(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
        s->kcache = TypedDeviceBuffer<float>(L * kvh * T * D);
        s->vcache = TypedDeviceBuffer<float>(L * kvh * T * D);
        s->d_hidden = TypedDeviceBuffer<float>(H);
        s->d_q = TypedDeviceBuffer<float>(qh * D);
        s->d_attn = TypedDeviceBuffer<float>(qh * D);
        s->d_act = TypedDeviceBuffer<float>(I);
        s->logits = TypedDeviceBuffer<float>(cfg_.vocab_size);
        s->attn_max_chunks = static_cast<int>(detail::blocks_for64(T, detail::kAttnChunk));
        s->attn_partial = TypedDeviceBuffer<float>(qh * s->attn_max_chunks * (D + 2));
        s->lm_grid = static_cast<int>(detail::blocks_for64(cfg_.vocab_size, llama::kRows * llama::kWavesPerBlock));
        s->lm_best_val = TypedDeviceBuffer<float>(s->lm_grid);
        s->lm_best_idx = TypedDeviceBuffer<int32_t>(s->lm_grid);
        s->gen = TypedDeviceBuffer<int32_t>(T);
        s->attn_counters = TypedDeviceBuffer<int32_t>(kvh);
        s->state_buf = TypedDeviceBuffer<int32_t>(4);
        s->ids = TypedDeviceBuffer<int32_t>(T);
        s->hidden = TypedDeviceBuffer<float>(T * H);
        s->normed = TypedDeviceBuffer<float>(T * H);
        s->qkv = TypedDeviceBuffer<float>(T * cfg_.qkv_width());
        s->q_heads = TypedDeviceBuffer<float>(T * qh * D);
        s->attn_heads = TypedDeviceBuffer<float>(T * qh * D);
        s->attn = TypedDeviceBuffer<float>(T * qh * D);
        s->act = TypedDeviceBuffer<float>(T * I);
        if (T >= 2) // only a multi-row prefill runs the GEMMs
            s->splitk_ws = TypedDeviceBuffer<float>(kBf16 ? detail::kSplitKWorkspaceBf16 : detail::kSplitKWorkspaceF32);
        OPWORKS_HIP_CHECK(hipMemsetAsync(s->state_buf.data(), 0, sizeof(int32_t) * 4, s->stream));
        OPWORKS_HIP_CHECK(hipMemsetAsync(s->attn_counters.data(), 0, sizeof(int32_t) * kvh, s->stream));
        OPWORKS_HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&s->h_state), sizeof(llama::StepState)));
        *s->h_state = llama::StepState{0, 0, -1, 0};
        OPWORKS_HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&s->h_token), sizeof(int32_t)));
        synchronize(s->stream);
        return s;
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
        if (s.length >= s.max_seq_len)
            throw std::invalid_argument("session capacity exhausted");
        s.h_state->token = token;
        s.h_state->pos = s.length;
        s.h_state->next = -1;
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.state(), s.h_state, sizeof(llama::StepState), hipMemcpyHostToDevice,
                                         s.stream));
        launch_decode(s);
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.h_state, s.state(), sizeof(llama::StepState), hipMemcpyDeviceToHost,
                                         s.stream));
        synchronize(s.stream);
        s.length += 1;
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
        if (n > s.max_seq_len - s.length)
            throw std::invalid_argument("session capacity exhausted");
        struct ChainOff { // every other path runs with chain = 0
            llama::StepState *h;
            ~ChainOff() { h->chain = 0; }
        } chain_off{s.h_state};
        const int pos0 = s.length;
        *s.h_state = llama::StepState{token, pos0, -1, 1};
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.state(), s.h_state, sizeof(llama::StepState), hipMemcpyHostToDevice,
                                         s.stream));
        // At most 16 steps are queued ahead of the GPU: enough that it never waits for the host,
        // few enough that eager mode (82 kernels per step) keeps a short queue. An event closes
        // every group of 4 steps; a group starts once the group 4 before it has completed.
        constexpr int kGroup = 4, kGroups = 4;
        while (static_cast<int>(s.step_events.size()) < kGroups) {
            hipEvent_t e;
            OPWORKS_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
            s.step_events.push_back(e);
        }
        for (int i = 0; i < n; ++i) {
            const int g = i / kGroup;
            if (i % kGroup == 0 && g >= kGroups)
                OPWORKS_HIP_CHECK(hipEventSynchronize(s.step_events[g % kGroups]));
            launch_decode(s);
            if (i % kGroup == kGroup - 1)
                OPWORKS_HIP_CHECK(hipEventRecord(s.step_events[g % kGroups], s.stream));
        }
        OPWORKS_HIP_CHECK(hipMemcpyAsync(out, s.gen.data() + pos0, sizeof(int32_t) * static_cast<size_t>(n),
                                         hipMemcpyDeviceToHost, s.stream));
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.h_state, s.state(), sizeof(llama::StepState), hipMemcpyDeviceToHost,
                                         s.stream));
        synchronize(s.stream);
        s.length += n;
        s.last_prefill_rows = 0;
    }

    // One decode step launched eagerly with an event before every kernel and
    // one after the last, all on the session stream; returns the kernel
    // durations in launch order (per layer: qkv_rope, attention, o_proj,
    // gate_up, down; then lm_head) and the next token in *next.
    std::vector<float> profile_decode_step(Session &s, int32_t token, int32_t *next) override {
        if (token < 0 || token >= cfg_.vocab_size)
            throw std::invalid_argument("token id outside the vocabulary");
        if (s.length >= s.max_seq_len)
            throw std::invalid_argument("session capacity exhausted");
        s.h_state->token = token;
        s.h_state->pos = s.length;
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
        s.length += 1;
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
        if (s.length == 0 || s.length >= s.max_seq_len)
            throw std::invalid_argument("time_decode_stage needs a prefilled session with free capacity");
        s.h_state->token = 0;
        s.h_state->pos = s.length;
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
        OPWORKS_HIP_CHECK(hipMemcpyAsync(out, s.logits.data(), sizeof(float) * static_cast<size_t>(n),
                                         hipMemcpyDeviceToHost, s.stream));
        synchronize(s.stream);
    }

    // Residual stream of the last prefill: rows x H.
    std::vector<float> hidden_state(Session &s, int rows) const override {
        if (rows <= 0 || rows > s.max_seq_len)
            throw std::invalid_argument("rows outside the session capacity");
        std::vector<float> out(static_cast<size_t>(rows) * cfg_.hidden_size);
        OPWORKS_HIP_CHECK(hipMemcpyAsync(out.data(), s.hidden.data(), out.size() * sizeof(float),
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
            const float *src = n == 1 ? s.d_hidden.data() : s.hidden.data();
            OPWORKS_HIP_CHECK(hipMemcpyAsync(h.data(), src, h.size() * sizeof(float), hipMemcpyDeviceToHost,
                                             s.stream));
            synchronize(s.stream);
            captures.push_back(std::move(h));
        });
        return captures;
    }

  private:
    explicit LlamaModelT(const ModelConfig &cfg) : cfg_(cfg) {}

    ModelConfig cfg_;
    LlamaWeights<WT> w_;
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

    void check_supported() const {
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
        if (static_cast<int>(ids.size()) > s.max_seq_len)
            throw std::invalid_argument("prompt exceeds the session capacity");
        if (s.length != 0)
            throw std::invalid_argument("prefill requires a fresh session (reset first)");
    }

    void allocate() {
        const int64_t H = cfg_.hidden_size, I = cfg_.intermediate_size, V = cfg_.vocab_size;
        w_.embed = TypedDeviceBuffer<WT>(V * H);
        w_.final_norm = TypedDeviceBuffer<float>(H);
        w_.inv_freq = TypedDeviceBuffer<float>::from_host(cfg_.rope_inv_freq());
        w_.layers.resize(static_cast<size_t>(cfg_.num_layers));
        for (auto &l : w_.layers) {
            l.input_norm = TypedDeviceBuffer<float>(H);
            l.post_norm = TypedDeviceBuffer<float>(H);
            l.wqkv = TypedDeviceBuffer<WT>(int64_t(cfg_.qkv_width()) * H);
            l.wo = TypedDeviceBuffer<WT>(H * cfg_.q_width());
            l.wgu = TypedDeviceBuffer<WT>(2 * I * H);
            l.wdown = TypedDeviceBuffer<WT>(H * I);
        }
    }

    void init_random(uint64_t seed, float sd, NormInit norms) {
        using namespace llama_detail;
        const int64_t H = cfg_.hidden_size, I = cfg_.intermediate_size, V = cfg_.vocab_size;
        const int64_t qw = cfg_.q_width(), kw = cfg_.kv_width();
        auto rows_fill = [&](WT *dst, int64_t rows, int64_t cols, int stride, int offset, uint64_t stream) {
            launch_async(nullptr, fill_rows_normal_kernel<WT>, fill_grid(rows * cols), 256, dst, rows,
                         static_cast<int>(cols), stride, offset, rng::stream_key(seed, stream), 0.f, sd);
        };
        auto norm_fill = [&](float *dst, uint64_t stream) {
            if (norms == NormInit::ones)
                launch_async(nullptr, fill_const_kernel, fill_grid(H), 256, dst, H, 1.f);
            else
                launch_async(nullptr, fill_uniform_kernel, fill_grid(H), 256, dst, H, rng::stream_key(seed, stream),
                             0.5f, 1.5f, kBf16);
        };
        rows_fill(w_.embed.data(), V, H, 1, 0, kStreamEmbed);
        norm_fill(w_.final_norm.data(), kStreamFinalNorm);
        for (int l = 0; l < cfg_.num_layers; ++l) {
            LlamaLayerWeights<WT> &lw = w_.layers[static_cast<size_t>(l)];
            rows_fill(lw.wqkv.data(), qw, H, 1, 0, layer_stream(l, kQ));
            rows_fill(lw.wqkv.data() + qw * H, kw, H, 1, 0, layer_stream(l, kK));
            rows_fill(lw.wqkv.data() + (qw + kw) * H, kw, H, 1, 0, layer_stream(l, kV));
            rows_fill(lw.wo.data(), H, qw, 1, 0, layer_stream(l, kO));
            rows_fill(lw.wgu.data(), I, H, 2, 0, layer_stream(l, kGate));
            rows_fill(lw.wgu.data(), I, H, 2, 1, layer_stream(l, kUp));
            rows_fill(lw.wdown.data(), H, I, 1, 0, layer_stream(l, kDown));
            norm_fill(lw.input_norm.data(), layer_stream(l, kInNorm));
            norm_fill(lw.post_norm.data(), layer_stream(l, kPostNorm));
        }
        synchronize(nullptr);
    }

    void upload_pack(const PackReader &pack) {
        const int64_t H = cfg_.hidden_size, I = cfg_.intermediate_size, V = cfg_.vocab_size;
        const int64_t qw = cfg_.q_width(), kw = cfg_.kv_width();
        // one pinned staging buffer of WT elements, sized for the largest tensor
        const int64_t largest = std::max<int64_t>(V * H, I * H);
        WT *stage = nullptr;
        OPWORKS_HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&stage), sizeof(WT) * largest));
        struct Free {
            void *p;
            ~Free() { (void)hipHostFree(p); }
        } guard{stage};
        auto read = [&](const std::string &name, int64_t numel) {
            if (pack.meta(name).numel != numel)
                throw std::runtime_error(name + ": element count mismatch");
            pack.read_into(name, stage, sizeof(WT) * static_cast<size_t>(numel));
        };
        auto put = [&](WT *dst, int64_t numel) {
            OPWORKS_HIP_CHECK(hipMemcpy(dst, stage, sizeof(WT) * numel, hipMemcpyHostToDevice));
        };
        auto put_rows_strided = [&](WT *dst, int64_t rows, int64_t cols, int offset) {
            OPWORKS_HIP_CHECK(hipMemcpy2D(dst + offset * cols, sizeof(WT) * 2 * cols, stage, sizeof(WT) * cols,
                                          sizeof(WT) * cols, rows, hipMemcpyHostToDevice));
        };
        // norm weights are fp32 on the device; a bf16 pack stores them as bf16
        // (reference: runtime/weights.cuh:57-66, read_bf16_as_float)
        auto put_norm = [&](const std::string &name, float *dst) {
            read(name, H);
            std::vector<float> f(static_cast<size_t>(H));
            for (int64_t i = 0; i < H; ++i) {
                if constexpr (kBf16)
                    f[static_cast<size_t>(i)] = bf16_to_float(stage[i].bits);
                else
                    f[static_cast<size_t>(i)] = stage[i];
            }
            OPWORKS_HIP_CHECK(hipMemcpy(dst, f.data(), sizeof(float) * H, hipMemcpyHostToDevice));
        };
        read("model.embed_tokens.weight", V * H);
        put(w_.embed.data(), V * H);
        put_norm("model.norm.weight", w_.final_norm.data());
        for (int l = 0; l < cfg_.num_layers; ++l) {
            const std::string p = "model.layers." + std::to_string(l) + ".";
            LlamaLayerWeights<WT> &lw = w_.layers[static_cast<size_t>(l)];
            put_norm(p + "input_layernorm.weight", lw.input_norm.data());
            read(p + "self_attn.q_proj.weight", qw * H);
            put(lw.wqkv.data(), qw * H);
            read(p + "self_attn.k_proj.weight", kw * H);
            put(lw.wqkv.data() + qw * H, kw * H);
            read(p + "self_attn.v_proj.weight", kw * H);
            put(lw.wqkv.data() + (qw + kw) * H, kw * H);
            read(p + "self_attn.o_proj.weight", H * qw);
            put(lw.wo.data(), H * qw);
            put_norm(p + "post_attention_layernorm.weight", lw.post_norm.data());
            read(p + "mlp.gate_proj.weight", I * H);
            put_rows_strided(lw.wgu.data(), I, H, 0);
            read(p + "mlp.up_proj.weight", I * H);
            put_rows_strided(lw.wgu.data(), I, H, 1);
            read(p + "mlp.down_proj.weight", H * I);
            put(lw.wdown.data(), H * I);
        }
        if (!pack.has("lm_head.weight"))
            throw std::runtime_error("pack has neither lm_head.weight nor a tying alias");
        if (pack.meta("lm_head.weight").offset != pack.meta("model.embed_tokens.weight").offset)
            throw std::runtime_error("untied lm_head.weight is not supported (Llama-3.2 ties it to the embedding)");
    }

    float *layer_k(Session &s, int l) const {
        return s.kcache.data() + int64_t(l) * cfg_.num_kv_heads * s.max_seq_len * cfg_.head_dim;
    }
    float *layer_v(Session &s, int l) const {
        return s.vcache.data() + int64_t(l) * cfg_.num_kv_heads * s.max_seq_len * cfg_.head_dim;
    }

    // ---- decode step (one token at state.pos) -----------------------------
    template <int kV, int kV2> void enqueue_decode_layer(Session &s, int l) const {
        const int H = cfg_.hidden_size, I = cfg_.intermediate_size, D = cfg_.head_dim;
        const int qh = cfg_.num_q_heads, kvh = cfg_.num_kv_heads;
        const int qkv_groups = (qh + 2 * kvh) * (D / 4); // 4 rows each
        hipStream_t st = s.stream;
        const LlamaLayerWeights<WT> &lw = w_.layers[static_cast<size_t>(l)];
        llama::QkvArgs<WT> qa{};
        // layer 0 reads the step token's embedding row: fp32 tables directly in
        // the qkv kernel, bf16 tables widened into the residual stream first
        qa.hidden_in = (l == 0 && !kBf16) ? nullptr : s.d_hidden.data();
        qa.embed = w_.embed.data();
        qa.hidden_out = s.d_hidden.data();
        qa.gamma = lw.input_norm.data();
        qa.wqkv = lw.wqkv.data();
        qa.inv_freq = w_.inv_freq.data();
        qa.q_out = s.d_q.data();
        qa.kcache = layer_k(s, l);
        qa.vcache = layer_v(s, l);
        qa.state = s.state();
        qa.eps = cfg_.rms_norm_eps;
        qa.qh = qh;
        qa.kvh = kvh;
        qa.D = D;
        qa.cap = s.max_seq_len;
        if (stage_on(0)) {
            tick();
            if (kBf16 && l == 0)
                launch_async(st, llama::embed_token_kernel<WT>, detail::blocks_for64(H, 256), 256, w_.embed.data(),
                             s.state(), s.d_hidden.data(), H);
            launch_async(st, llama::qkv_rope_kernel<kV, WT>, qkv_groups, llama::kBlock, qa);
        }
        llama::DecodeAttnArgs aa{};
        aa.q = s.d_q.data();
        aa.kcache = layer_k(s, l);
        aa.vcache = layer_v(s, l);
        aa.out = s.d_attn.data();
        aa.partial = s.attn_partial.data();
        aa.counters = s.attn_counters.data(); // fused merge: one launch per layer
        aa.len_ptr = s.state_buf.data() + offsetof(llama::StepState, pos) / sizeof(int32_t); // length pos + 1
        aa.len_bias = 1;
        aa.kv_rep = cfg_.kv_rep();
        aa.D = D;
        aa.cap = s.max_seq_len;
        aa.max_chunks = s.attn_max_chunks;
        aa.scale = 1.f / std::sqrt(static_cast<float>(D));
        if (stage_on(1)) {
            tick();
            detail::attention_decode_launch(aa, kvh, st);
        }
        if (stage_on(2)) {
            tick();
            launch_async(st, llama::gemv_residual_kernel<kV, WT>, detail::blocks_for64(H, llama::kRows),
                         llama::kBlock, lw.wo.data(), s.d_attn.data(), s.d_hidden.data(), H);
        }
        if (stage_on(3)) {
            tick();
            launch_async(st, llama::swiglu_gemv_kernel<kV, WT>, detail::blocks_for64(2 * I, llama::kWavesPerBlock),
                         llama::kBlock, s.d_hidden.data(), lw.post_norm.data(), cfg_.rms_norm_eps, lw.wgu.data(),
                         s.d_act.data(), I);
        }
        if (stage_on(4)) {
            tick();
            launch_async(st, llama::down_residual_kernel<kV2, WT>, detail::blocks_for64(H, llama::kRows), llama::kBlock,
                         lw.wdown.data(), s.d_act.data(), s.d_hidden.data(), H);
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
                enqueue_lm_head<kV>(s, s.d_hidden.data());
        });
    }

    template <int kV> void enqueue_lm_head(Session &s, const float *hidden_row) const {
        llama::LmHeadArgs<WT> la{};
        la.hidden_row = hidden_row;
        la.gamma = w_.final_norm.data();
        la.embed = w_.embed.data();
        la.logits = s.logits.data();
        la.best_val = s.lm_best_val.data();
        la.best_idx = s.lm_best_idx.data();
        la.eps = cfg_.rms_norm_eps;
        la.vocab = cfg_.vocab_size;
        tick();
        launch_async(s.stream, llama::lm_head_kernel<kV, WT>, s.lm_grid, llama::kBlock, la);
        launch_async(s.stream, llama::argmax_records_kernel, 1, 1024, s.lm_best_val.data(), s.lm_best_idx.data(),
                     s.lm_grid, s.state(), s.gen.data());
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

    void capture_decode_graph(Session &s) const {
        OPWORKS_HIP_CHECK(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal));
        try {
            enqueue_decode(s);
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(s.stream, &g);
            if (g)
                (void)hipGraphDestroy(g);
            throw;
        }
        OPWORKS_HIP_CHECK(hipStreamEndCapture(s.stream, &s.graph));
        OPWORKS_HIP_CHECK(hipGraphInstantiate(&s.graph_exec, s.graph, nullptr, nullptr, 0));
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
            OPWORKS_HIP_CHECK(hipMemcpyAsync(s.ids.data(), ids.data(), sizeof(int32_t) * n, hipMemcpyHostToDevice,
                                             s.stream));
            s.h_state->pos = n; // the next decode position
            OPWORKS_HIP_CHECK(hipMemcpyAsync(s.state(), s.h_state, sizeof(llama::StepState),
                                             hipMemcpyHostToDevice, s.stream));
            enqueue_prefill(s, n, hook);
        }
        OPWORKS_HIP_CHECK(hipMemcpyAsync(s.h_state, s.state(), sizeof(llama::StepState), hipMemcpyDeviceToHost,
                                         s.stream));
        synchronize(s.stream);
        s.length = n;
        s.last_prefill_rows = n;
    }

    // Single-row prefill with per-layer captures: the decode kernels launched eagerly.
    void run_decode_layers_with_hook(Session &s, const std::function<void(int)> &hook) {
        // Layer 0's first kernel writes the embedding row into the residual stream;
        // copy it beforehand so the "after embedding" capture sees it.
        const int H = cfg_.hidden_size;
        if constexpr (kBf16)
            launch_async(s.stream, llama::embed_token_kernel<WT>, detail::blocks_for64(H, 256), 256, w_.embed.data(),
                         s.state(), s.d_hidden.data(), H);
        else
            OPWORKS_HIP_CHECK(hipMemcpyAsync(s.d_hidden.data(), w_.embed.data() + int64_t(s.h_state->token) * H,
                                             sizeof(float) * H, hipMemcpyDeviceToDevice, s.stream));
        hook(-1);
        enqueue_decode(s, hook);
    }

    // Prefill projection C (per kStore) = A[M][K] W[N][K]^T: the fp32 MFMA GEMM
    // for fp32 weights; for bf16 weights the bf16 MFMA GEMM with A rounded to
    // bf16 on load (the reference's linear_mma_bf16 path, models/llama.cuh:190-199;
    // it takes that path from 16 rows, this build from 2, see the design notes).
    // Outputs with too few tiles to fill the GPU (o_proj, down, qkv at a few
    // hundred rows) split K across workgroups into the session's workspace.
    template <detail::GemmStore kStore = detail::GemmStore::store>
    void project(Session &s, const float *A, const WT *W, float *C, int M, int N, int K, hipStream_t st) const {
        using detail::IdentityEpilogue;
        constexpr bool kSplittable = kStore != detail::GemmStore::swiglu;
        const auto *Wb = reinterpret_cast<const uint16_t *>(W);
        if constexpr (kBf16) {
            // 2..15 rows: fp32 inputs against the widened bf16 weights, as the reference's
            // linear_dispatch does below 16 rows (include/models/llama.cuh:190-199)
            if (M < 16) {
                if constexpr (kSplittable)
                    detail::gemm_f32_launch_splitk<detail::BLayout::nk, IdentityEpilogue, kStore, uint16_t>(
                        A, Wb, nullptr, C, M, N, K, IdentityEpilogue{}, s.splitk_ws.data(), s.splitk_ws.size(), st);
                else
                    detail::gemm_f32_launch<detail::BLayout::nk, IdentityEpilogue, kStore, uint16_t>(
                        A, Wb, nullptr, C, M, N, K, IdentityEpilogue{}, st);
                return;
            }
        }
        if constexpr (kBf16 && kSplittable)
            detail::gemm_bf16_launch_splitk<float, IdentityEpilogue, kStore>(
                A, Wb, nullptr, C, M, N, K, IdentityEpilogue{}, s.splitk_ws.data(), s.splitk_ws.size(), st);
        else if constexpr (kBf16)
            detail::gemm_bf16_launch<float, IdentityEpilogue, kStore>(A, Wb, nullptr, C, M, N, K, IdentityEpilogue{},
                                                                      st);
        else if constexpr (kSplittable)
            detail::gemm_f32_launch_splitk<detail::BLayout::nk, IdentityEpilogue, kStore>(
                A, W, nullptr, C, M, N, K, IdentityEpilogue{}, s.splitk_ws.data(), s.splitk_ws.size(), st);
        else
            detail::gemm_f32_launch<detail::BLayout::nk, IdentityEpilogue, kStore>(A, W, nullptr, C, M, N, K,
                                                                                  IdentityEpilogue{}, st);
    }

    void enqueue_prefill(Session &s, int n, const std::function<void(int)> &hook) {
        const int H = cfg_.hidden_size, I = cfg_.intermediate_size, D = cfg_.head_dim;
        const int qh = cfg_.num_q_heads, kvh = cfg_.num_kv_heads, qkvw = cfg_.qkv_width();
        hipStream_t st = s.stream;
        launch_async(st, llama::embedding_kernel<WT>, detail::stream_grid(int64_t(n) * H / 4), 256, w_.embed.data(),
                     s.ids.data(), s.hidden.data(), n, H);
        if (hook)
            hook(-1);
        for (int l = 0; l < cfg_.num_layers; ++l) {
            const LlamaLayerWeights<WT> &lw = w_.layers[static_cast<size_t>(l)];
            ops::rms_norm(s.hidden.data(), lw.input_norm.data(), s.normed.data(), n, H, cfg_.rms_norm_eps, st);
            project(s, s.normed.data(), lw.wqkv.data(), s.qkv.data(), n, qkvw, H, st);
            launch_async(st, llama::rope_split_kernel, detail::stream_grid(int64_t(n) * (qh + 2 * kvh) * (D / 2)),
                         256, s.qkv.data(), w_.inv_freq.data(), s.q_heads.data(), layer_k(s, l), layer_v(s, l), n, qh,
                         kvh, D, s.max_seq_len, 0);
            ops::attention_prefill(s.q_heads.data(), layer_k(s, l), layer_v(s, l), s.attn_heads.data(), n, n, 0, qh,
                                   cfg_.kv_rep(), D, s.max_seq_len, st);
            launch_async(st, llama::merge_heads_kernel, detail::stream_grid(int64_t(n) * qh * D), 256,
                         s.attn_heads.data(), s.attn.data(), n, qh, D);
            project<detail::GemmStore::residual>(s, s.attn.data(), lw.wo.data(), s.hidden.data(), n, H, qh * D,
                                                 st);
            ops::rms_norm(s.hidden.data(), lw.post_norm.data(), s.normed.data(), n, H, cfg_.rms_norm_eps, st);
            project<detail::GemmStore::swiglu>(s, s.normed.data(), lw.wgu.data(), s.act.data(), n, 2 * I, H, st);
            project<detail::GemmStore::residual>(s, s.act.data(), lw.wdown.data(), s.hidden.data(), n, H, I, st);
            if (hook)
                hook(l);
        }
        dispatch_widths(
            [&](auto v, auto) { enqueue_lm_head<decltype(v)::value>(s, s.hidden.data() + int64_t(n - 1) * H); });
    }
};

using LlamaModel = LlamaModelT<float>;
using LlamaModelBF16 = LlamaModelT<bf16>;

// Loads a pack and picks the model from its dtype (reference: src/llama_c_api.cu:56-73).
inline std::unique_ptr<LlamaRuntime> load_llama(const std::string &pack_path) {
    PackReader pack(pack_path);
    if (pack.dtype() == "float32")
        return LlamaModel::load(pack);
    if (pack.dtype() == "bfloat16")
        return LlamaModelBF16::load(pack);
    throw std::runtime_error("unsupported pack dtype " + pack.dtype());
}

// Seeded random weights of either storage type.
inline std::unique_ptr<LlamaRuntime> load_llama_random(const ModelConfig &cfg, uint64_t seed, float std,
                                                       NormInit norms, bool bf16_weights) {
    if (bf16_weights)
        return LlamaModelBF16::load_random(cfg, seed, std, norms);
    return LlamaModel::load_random(cfg, seed, std, norms);
}

} // namespace opworks

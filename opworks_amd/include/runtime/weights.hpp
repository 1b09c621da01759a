#pragma once

// Device-resident Llama weights (reference: include/runtime/weights.cuh:17-94).
// WT is the storage type of the projections and the embedding (float or
// bf16); norm weights are always fp32, as in the reference.
//
// The MI355X layout differs from the HF one where a fused kernel wants it,
// so those members carry their own names:
//  * qkv_proj     [(qh + 2 kvh) D][H]  q, k and v rows concatenated: one GEMV / GEMM;
//  * gate_up_proj [2 I][H]             gate_i and up_i rows interleaved (2i, 2i + 1),
//                                      so one wave's rows give silu(gate) * up;
//  * o_proj [H][qh D], down_proj [H][I], embed_tokens [V][H] (also the tied
//    LM head), input_norm / post_norm / final_norm [H] as in HF.
// ModelWeights::load reads an OPWPACK1 pack written by the reference's exporter
// (HF tensor names) into this layout; ModelWeights::random draws seeded
// weights with the counter-based generator of core/random.hpp, so a CPU
// restatement can draw the same values.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "../core/bf16.hpp"
#include "../core/hip_utils.hpp"
#include "../core/random.hpp"
#include "../core/typed_device_buffer.hpp"
#include "model_config.hpp"
#include "pack_reader.hpp"

namespace opworks {

// Norm weights of the seeded init: ones (HF init) or U[0.5, 1.5] (exercises gamma in tests).
enum class NormInit { ones = 0, uniform = 1 };

namespace weights_detail {

// Stream ids of the seeded initialisation. Logical tensors are drawn in the HF
// layout: element (o, i) of a [out][in] projection is draw o * in + i of its stream.
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

} // namespace weights_detail

template <typename WT> struct LayerWeights {
    TypedDeviceBuffer<float> input_norm;  // [H]
    TypedDeviceBuffer<WT> qkv_proj;       // [(qh + 2 kvh) D][H]
    TypedDeviceBuffer<WT> o_proj;         // [H][qh D]
    TypedDeviceBuffer<float> post_norm;   // [H]
    TypedDeviceBuffer<WT> gate_up_proj;   // [2 I][H], rows gate_0, up_0, gate_1, ...
    TypedDeviceBuffer<WT> down_proj;      // [H][I]
};

template <typename WT> struct ModelWeights {
    static_assert(std::is_same_v<WT, float> || std::is_same_v<WT, bf16>, "weights are float or bf16");
    static constexpr bool kBf16 = std::is_same_v<WT, bf16>;

    TypedDeviceBuffer<WT> embed_tokens;     // [V][H], also the LM head (tied)
    TypedDeviceBuffer<float> final_norm;    // [H]
    std::vector<LayerWeights<WT>> layers;
    TypedDeviceBuffer<float> rope_inv_freq; // [head_dim / 2]

    // Device memory for cfg, contents unset (rope_inv_freq excepted).
    static ModelWeights allocate(const ModelConfig &cfg) {
        const int64_t H = cfg.hidden_size, I = cfg.intermediate_size, V = cfg.vocab_size;
        ModelWeights w;
        w.embed_tokens = TypedDeviceBuffer<WT>(V * H);
        w.final_norm = TypedDeviceBuffer<float>(H);
        w.rope_inv_freq = TypedDeviceBuffer<float>::from_host(cfg.rope_inv_freq());
        w.layers.resize(static_cast<size_t>(cfg.num_layers));
        for (LayerWeights<WT> &l : w.layers) {
            l.input_norm = TypedDeviceBuffer<float>(H);
            l.post_norm = TypedDeviceBuffer<float>(H);
            l.qkv_proj = TypedDeviceBuffer<WT>(int64_t(cfg.qkv_width()) * H);
            l.o_proj = TypedDeviceBuffer<WT>(H * cfg.q_width());
            l.gate_up_proj = TypedDeviceBuffer<WT>(2 * I * H);
            l.down_proj = TypedDeviceBuffer<WT>(H * I);
        }
        return w;
    }

    // Reads a pack of this storage type (float32 or bfloat16); bf16 packs store
    // the norms as bf16 too, which are widened to fp32 (the reference's
    // read_bf16_as_float, runtime/weights.cuh:57-66). Tensors go through one
    // pinned staging buffer sized for the largest of them.
    static ModelWeights load(const PackReader &pack, const ModelConfig &cfg, hipStream_t stream = nullptr) {
        if (pack.dtype() != (kBf16 ? "bfloat16" : "float32"))
            throw std::runtime_error(std::string(kBf16 ? "bf16" : "fp32") + " model requires a " +
                                     (kBf16 ? "bfloat16" : "float32") + " pack (got " + pack.dtype() + ")");
        ModelWeights w = allocate(cfg);
        const int64_t H = cfg.hidden_size, I = cfg.intermediate_size, V = cfg.vocab_size;
        const int64_t qw = cfg.q_width(), kw = cfg.kv_width();
        const int64_t largest = std::max<int64_t>(V * H, I * H);
        WT *stage = nullptr;
        OPWORKS_HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&stage), sizeof(WT) * largest));
        struct PinnedFree {
            void *p;
            ~PinnedFree() { (void)hipHostFree(p); }
        } release{stage};
        auto read = [&](const std::string &name, int64_t numel) {
            if (pack.meta(name).numel != numel)
                throw std::runtime_error(name + ": element count mismatch");
            pack.read_into(name, stage, sizeof(WT) * static_cast<size_t>(numel));
        };
        auto put = [&](WT *dst, int64_t numel) {
            OPWORKS_HIP_CHECK(hipMemcpyAsync(dst, stage, sizeof(WT) * numel, hipMemcpyHostToDevice, stream));
            synchronize(stream); // the staging buffer is reused by the next tensor
        };
        auto put_interleaved = [&](WT *dst, int64_t rows, int64_t cols, int offset) {
            OPWORKS_HIP_CHECK(hipMemcpy2DAsync(dst + offset * cols, sizeof(WT) * 2 * cols, stage, sizeof(WT) * cols,
                                               sizeof(WT) * cols, rows, hipMemcpyHostToDevice, stream));
            synchronize(stream);
        };
        auto put_norm = [&](const std::string &name, TypedDeviceBuffer<float> &dst) {
            read(name, H);
            std::vector<float> f(static_cast<size_t>(H));
            for (int64_t i = 0; i < H; ++i) {
                if constexpr (kBf16)
                    f[static_cast<size_t>(i)] = bf16_to_float(stage[i].bits);
                else
                    f[static_cast<size_t>(i)] = stage[i];
            }
            detail::copy_and_wait(dst.data(), f.data(), dst.bytes(), hipMemcpyHostToDevice, stream);
        };
        read("model.embed_tokens.weight", V * H);
        put(w.embed_tokens.data(), V * H);
        put_norm("model.norm.weight", w.final_norm);
        for (int l = 0; l < cfg.num_layers; ++l) {
            const std::string p = "model.layers." + std::to_string(l) + ".";
            LayerWeights<WT> &lw = w.layers[static_cast<size_t>(l)];
            put_norm(p + "input_layernorm.weight", lw.input_norm);
            read(p + "self_attn.q_proj.weight", qw * H);
            put(lw.qkv_proj.data(), qw * H);
            read(p + "self_attn.k_proj.weight", kw * H);
            put(lw.qkv_proj.data() + qw * H, kw * H);
            read(p + "self_attn.v_proj.weight", kw * H);
            put(lw.qkv_proj.data() + (qw + kw) * H, kw * H);
            read(p + "self_attn.o_proj.weight", H * qw);
            put(lw.o_proj.data(), H * qw);
            put_norm(p + "post_attention_layernorm.weight", lw.post_norm);
            read(p + "mlp.gate_proj.weight", I * H);
            put_interleaved(lw.gate_up_proj.data(), I, H, 0);
            read(p + "mlp.up_proj.weight", I * H);
            put_interleaved(lw.gate_up_proj.data(), I, H, 1);
            read(p + "mlp.down_proj.weight", H * I);
            put(lw.down_proj.data(), H * I);
        }
        if (!pack.has("lm_head.weight"))
            throw std::runtime_error("pack has neither lm_head.weight nor a tying alias");
        if (pack.meta("lm_head.weight").offset != pack.meta("model.embed_tokens.weight").offset)
            throw std::runtime_error("untied lm_head.weight is not supported (Llama-3.2 ties it to the embedding)");
        return w;
    }

    // Seeded weights: projections and the embedding ~ N(0, sd) (bf16: rounded
    // to nearest-even), norms per NormInit (bf16: the rounded values).
    static ModelWeights random(const ModelConfig &cfg, uint64_t seed, float sd, NormInit norms) {
        using namespace weights_detail;
        ModelWeights w = allocate(cfg);
        const int64_t H = cfg.hidden_size, I = cfg.intermediate_size, V = cfg.vocab_size;
        const int64_t qw = cfg.q_width(), kw = cfg.kv_width();
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
        rows_fill(w.embed_tokens.data(), V, H, 1, 0, kStreamEmbed);
        norm_fill(w.final_norm.data(), kStreamFinalNorm);
        for (int l = 0; l < cfg.num_layers; ++l) {
            LayerWeights<WT> &lw = w.layers[static_cast<size_t>(l)];
            rows_fill(lw.qkv_proj.data(), qw, H, 1, 0, layer_stream(l, kQ));
            rows_fill(lw.qkv_proj.data() + qw * H, kw, H, 1, 0, layer_stream(l, kK));
            rows_fill(lw.qkv_proj.data() + (qw + kw) * H, kw, H, 1, 0, layer_stream(l, kV));
            rows_fill(lw.o_proj.data(), H, qw, 1, 0, layer_stream(l, kO));
            rows_fill(lw.gate_up_proj.data(), I, H, 2, 0, layer_stream(l, kGate));
            rows_fill(lw.gate_up_proj.data(), I, H, 2, 1, layer_stream(l, kUp));
            rows_fill(lw.down_proj.data(), H, I, 1, 0, layer_stream(l, kDown));
            norm_fill(lw.input_norm.data(), layer_stream(l, kInNorm));
            norm_fill(lw.post_norm.data(), layer_stream(l, kPostNorm));
        }
        synchronize(nullptr);
        return w;
    }
};

} // namespace opworks

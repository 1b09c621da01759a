// The Llama runtime driven through its C++ API the way the reference's own
// model tests drive theirs (tests/model/model_test_body.cuh:52-306 and
// test_common.cuh:75-83): the model loaded by value from a weight pack, sessions
// created by value, debug_prefill captures, prefill / decode_step, last_logits,
// session.cache.reset(), and fixtures read with PackReader::read / read_int32 /
// meta().shape. The fixtures pack is written by the test suite from the CPU
// oracle (tests/test_model_api_gpu.py); a bf16 weight pack selects
// LlamaModelBF16 and the bf16 tolerances.
//
//   model_api <weights.pack> <fixtures.pack>
//
// Exit status: 0 pass, 1 a check failed, 2 bad usage or unreadable files,
// 77 no HIP device.
#include <models/llama.hpp>

#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

namespace {

using opworks::PackReader;

struct Agreement {
    double nrmse = 0, cosine = 0, max_abs = 0;
};

Agreement agreement(const std::vector<float> &got, const std::vector<float> &want) {
    Agreement a;
    if (got.size() != want.size() || want.empty()) {
        a.nrmse = a.max_abs = INFINITY;
        return a;
    }
    double err2 = 0, ref2 = 0, dot = 0, got2 = 0;
    for (size_t i = 0; i < want.size(); ++i) {
        const double g = got[i], w = want[i], e = g - w;
        a.max_abs = std::fmax(a.max_abs, std::fabs(e));
        err2 += e * e;
        ref2 += w * w;
        dot += g * w;
        got2 += g * g;
    }
    const double n = static_cast<double>(want.size());
    a.nrmse = std::sqrt(err2 / n) / std::fmax(std::sqrt(ref2 / n), 1e-6);
    a.cosine = dot / std::fmax(std::sqrt(got2 * ref2), 1e-30);
    return a;
}

struct Tolerances {
    double nrmse, cosine;
};

class Checks {
  public:
    void close(const std::string &name, const std::vector<float> &got, const std::vector<float> &want,
               Tolerances tol) {
        const Agreement a = agreement(got, want);
        const bool ok = a.nrmse <= tol.nrmse && a.cosine >= tol.cosine;
        std::printf("%-26s %s  nrmse=%.3g cos=%.9f max_abs=%.3g\n", name.c_str(), ok ? "PASS" : "FAIL", a.nrmse,
                    a.cosine, a.max_abs);
        failed_ += !ok;
    }
    void same(const std::string &name, bool ok, const std::string &detail = "") {
        std::printf("%-26s %s%s%s\n", name.c_str(), ok ? "PASS" : "FAIL", detail.empty() ? "" : "  ",
                    detail.c_str());
        failed_ += !ok;
    }
    int failed() const { return failed_; }

  private:
    int failed_ = 0;
};

template <typename WT> int run(const char *weights_path, const PackReader &fx) {
    using ModelT = opworks::LlamaModelT<WT>;
    constexpr bool bf16 = std::is_same_v<WT, opworks::bf16>;
    Checks checks;
    const Tolerances hidden_tol = bf16 ? Tolerances{1e-2, 0.999} : Tolerances{1e-5, 0.99999};
    const Tolerances logit_tol = hidden_tol;

    ModelT model = ModelT::load(weights_path);
    const std::vector<int32_t> ids = fx.read_int32("input_ids");
    const std::vector<int32_t> generated = fx.read_int32("generated_ids");
    const int T = static_cast<int>(ids.size());
    checks.same("fixture.shape", fx.meta("input_ids").shape == std::vector<int64_t>{T});

    { // per-layer residual stream and last-row logits
        auto session = model.create_session(2048);
        const auto captures = model.debug_prefill(session, ids);
        checks.same("debug_prefill.count", static_cast<int>(captures.size()) == model.config().num_layers + 1);
        for (int i = 0; i <= model.config().num_layers && i < static_cast<int>(captures.size()); ++i) {
            const std::string name = i == 0 ? "hidden.embed" : "hidden.layer" + std::to_string(i - 1);
            checks.close(name, captures[static_cast<size_t>(i)], fx.read(name), hidden_tol);
        }
        checks.close("logits.last", model.last_logits(session), fx.read("logits.last"), logit_tol);
    }

    auto greedy = [&](typename ModelT::Session &session, const std::vector<int32_t> &prompt, size_t count) {
        std::vector<int32_t> out;
        int32_t tok = model.prefill(session, prompt);
        for (size_t i = 0; i < count; ++i) {
            out.push_back(tok);
            if (i + 1 < count)
                tok = model.decode_step(session, tok);
        }
        return out;
    };

    { // greedy ids, then the same after session.cache.reset()
        auto session = model.create_session(2048);
        const std::vector<int32_t> first = greedy(session, ids, generated.size());
        checks.same("generation.greedy", first == generated, std::to_string(first.size()) + " tokens");
        session.cache.reset();
        checks.same("session.reset_repeat", greedy(session, ids, generated.size()) == first);
    }

    { // KV cache: prefill(L) + decode(ids[L]) against prefill(L + 1), over a length sweep
        int bad = 0;
        for (int L : {1, 2, 7, 31, 32, 33}) {
            if (L + 1 > T)
                continue;
            auto a = model.create_session(2048);
            model.prefill(a, std::vector<int32_t>(ids.begin(), ids.begin() + L));
            model.decode_step(a, ids[static_cast<size_t>(L)]);
            auto b = model.create_session(2048);
            model.prefill(b, std::vector<int32_t>(ids.begin(), ids.begin() + L + 1));
            const Agreement d = agreement(model.last_logits(a), model.last_logits(b));
            if (!(d.nrmse <= logit_tol.nrmse && d.cosine >= logit_tol.cosine)) {
                ++bad;
                std::fprintf(stderr, "kv sweep L=%d: nrmse=%.3g cos=%.9f\n", L, d.nrmse, d.cosine);
            }
        }
        checks.same("kv_cache.length_sweep", bad == 0);
    }

    { // interleaved sessions do not interfere; a session moved mid-generation keeps its state
        const std::vector<int32_t> p1(ids.begin(), ids.begin() + T / 2), p2(ids.begin() + T / 2, ids.end());
        auto s1 = model.create_session(2048);
        auto s2 = model.create_session(2048);
        int32_t t1 = model.prefill(s1, p1), t2 = model.prefill(s2, p2);
        for (int i = 0; i < 4; ++i) {
            t1 = model.decode_step(s1, t1);
            t2 = model.decode_step(s2, t2);
        }
        auto moved = std::move(s1);
        for (int i = 0; i < 4; ++i) {
            t1 = model.decode_step(moved, t1);
            t2 = model.decode_step(s2, t2);
        }
        auto r1 = model.create_session(2048);
        auto r2 = model.create_session(2048);
        int32_t u1 = model.prefill(r1, p1), u2 = model.prefill(r2, p2);
        for (int i = 0; i < 8; ++i) {
            u1 = model.decode_step(r1, u1);
            u2 = model.decode_step(r2, u2);
        }
        checks.same("session.concurrent", t1 == u1 && t2 == u2);
    }

    { // the runtime types: a model moved into another object, weights and a cache of their own
        ModelT again = std::move(model);
        auto session = again.create_session(64);
        checks.same("model.moved", again.prefill(session, std::vector<int32_t>(ids.begin(), ids.begin() + 5)) ==
                                        [&] {
                                            auto fresh = ModelT::load(weights_path);
                                            auto s = fresh.create_session(64);
                                            return fresh.prefill(s, std::vector<int32_t>(ids.begin(),
                                                                                         ids.begin() + 5));
                                        }());
        const opworks::ModelConfig &cfg = again.config();
        opworks::KvCache cache(cfg, 16);
        checks.same("kv_cache.shape", static_cast<int>(cache.k.size()) == cfg.num_layers && cache.length == 0 &&
                                          cache.k[0].size() == int64_t(cfg.num_kv_heads) * 16 * cfg.head_dim);
        checks.same("session.cache.length", session.cache.length == 5 && session.cache.max_seq_len == 64);
        const PackReader wp(weights_path);
        const auto weights = opworks::ModelWeights<WT>::load(wp, cfg);
        const std::vector<float> norm = weights.final_norm.to_host();
        const std::vector<float> want = bf16 ? wp.read_bf16_as_float("model.norm.weight") : wp.read("model.norm.weight");
        checks.same("model_weights.load", norm == want && static_cast<int>(weights.layers.size()) == cfg.num_layers);
        checks.same("pack.read_raw", wp.read_raw("model.norm.weight").size() ==
                                         static_cast<size_t>(cfg.hidden_size) * (bf16 ? 2 : 4));
    }
    std::printf(checks.failed() == 0 ? "PASS: model API\n" : "FAIL: %d model API check(s)\n", checks.failed());
    return checks.failed() == 0 ? 0 : 1;
}

} // namespace

int main(int argc, char **argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s <weights.pack> <fixtures.pack>\n", argv[0]);
        return 2;
    }
    int devices = 0;
    const hipError_t st = hipGetDeviceCount(&devices);
    if (st == hipErrorNoDevice || st == hipErrorInsufficientDriver || (st == hipSuccess && devices == 0)) {
        std::puts("SKIP: no HIP device");
        return 77;
    }
    OPWORKS_HIP_CHECK(st);
    try {
        const PackReader fixtures(argv[2]);
        const std::string dtype = PackReader(argv[1]).dtype();
        if (dtype == "bfloat16")
            return run<opworks::bf16>(argv[1], fixtures);
        return run<float>(argv[1], fixtures);
    } catch (const std::exception &e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 2;
    }
}
